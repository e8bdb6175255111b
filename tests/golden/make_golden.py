"""Writes the chunk-rule golden vectors from the REFERENCE's own compiled code.

Runs in the build container only (needs oracle/_ref/libref_chunk.so, built by
oracle/Makefile from /root/reference/src/runtime/deltanet_chunk.cpp).  Output:

  chunk_unit_case.npz  inputs of the reference's unit test
                       (tests/run_deltanet_chunk_unit.py:104-128: torch.manual_seed(0),
                       H=2, T=5, dk=3, dv=2, C=4, L2 on, non-zero initial state) and
                       the reference rule's outputs for them;
  chunk_cases.json     the probe cases of apps/spock-deltanet-chunk-prefill-probe.cpp:
                       62-84 and the north-star config 0, with the SHA-256 of the
                       reference rule's float32 outputs (inputs are regenerated
                       deterministically by tests/chunk_cases.py).

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent))
sys.path.insert(0, str(HERE.parents[1]))

import oracle_lib  # noqa: E402
import chunk_cases  # noqa: E402


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def unit_case():
    import torch  # only to reproduce the reference test's seeded inputs
    torch.manual_seed(0)
    H, T, dk, dv, C = 2, 5, 3, 2, 4
    q = torch.randn(1, T, H, dk, dtype=torch.float32)
    k = torch.randn(1, T, H, dk, dtype=torch.float32)
    v = torch.randn(1, T, H, dv, dtype=torch.float32)
    g = torch.randn(1, T, H, dtype=torch.float32) * 0.2 - 0.3
    beta = torch.sigmoid(torch.randn(1, T, H, dtype=torch.float32))
    init = torch.randn(1, H, dk, dv, dtype=torch.float32) * 0.1
    hm = lambda x: x.squeeze(0).transpose(0, 1).contiguous().numpy()  # [H][T][...]
    inputs = {"q": hm(q), "k": hm(k), "v": hm(v), "g": hm(g), "beta": hm(beta),
              "init": init.squeeze(0).numpy()}
    core, state = oracle_lib.chunk_rule(inputs["q"], inputs["k"], inputs["v"], inputs["g"],
                                        inputs["beta"], init=inputs["init"], chunk=C, l2=True,
                                        use_ref=True)
    np.savez(HERE / "chunk_unit_case.npz", **inputs, core=core, state=state,
             meta=np.array([H, T, dk, dv, C, 1], dtype=np.int32))


def cases():
    out = {}
    for name, spec in chunk_cases.CASES.items():
        inp = chunk_cases.make_inputs(name)
        core, state = oracle_lib.chunk_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                            chunk=spec["C"], l2=False, use_ref=True)
        out[name] = {
            "spec": spec,
            "inputs_sha256": chunk_cases.inputs_digest(inp),
            "core_sha256": sha(core),
            "state_sha256": sha(state),
            "core_max_abs": float(np.abs(core).max()),
            "state_max_abs": float(np.abs(state).max()),
        }
    (HERE / "chunk_cases.json").write_text(json.dumps(out, indent=1, sort_keys=True) + "\n")


if __name__ == "__main__":
    if not oracle_lib.ref_available():
        raise SystemExit("oracle/_ref/libref_chunk.so is not built (make -C oracle)")
    unit_case()
    cases()
    print("wrote", HERE / "chunk_unit_case.npz", HERE / "chunk_cases.json")
