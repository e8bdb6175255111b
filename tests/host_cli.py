"""Helpers for the C++ drivers under spock_amd/bin (tests only)."""
import json
import subprocess
from pathlib import Path

import numpy as np

from conftest import ROOT

BIN = ROOT / "spock_amd" / "bin"
CHUNK_CLI = BIN / "spock-deltanet-chunk"
SESSION_CLI = BIN / "spock-deltanet-session"


def chunk_fixture(q, k, v, g, beta, init=None, chunk_size=64, l2=True) -> dict:
    """The JSON input of spock-deltanet-chunk, as tests/run_deltanet_chunk_unit.py:130-145
    writes it: [head][token][dim] arrays flattened, g/beta [head][token]."""
    H, T, dk = q.shape
    return {"num_heads": int(H), "sequence_length": int(T), "key_dim": int(dk),
            "value_dim": int(v.shape[2]), "chunk_size": int(chunk_size), "use_qk_l2norm": bool(l2),
            "query": q.ravel().tolist(), "key": k.ravel().tolist(), "value": v.ravel().tolist(),
            "g": g.ravel().tolist(), "beta": beta.ravel().tolist(),
            "initial_state": None if init is None else init.ravel().tolist()}


def run_chunk_cli(tmp: Path, fixture, timeout=120):
    p = tmp / "fixture.json"
    p.write_text(fixture if isinstance(fixture, str) else json.dumps(fixture))
    return subprocess.run([str(CHUNK_CLI), "--input", str(p)], capture_output=True, text=True,
                          timeout=timeout)


def parse_chunk_output(stdout: str, H, T, dk, dv):
    out = json.loads(stdout)
    core = np.asarray(out["core_attn_out"], dtype=np.float32).reshape(H, T, dv)
    state = np.asarray(out["final_state"], dtype=np.float32).reshape(H, dk, dv)
    return core, state
