"""Config 4 on the GPU: the full Qwen3.5-0.8B-shaped random-init model (24
layers: 18 gated DeltaNet + 6 gated full attention, hidden 1024, vocab
248320, seeded fp16 weights), 512-token prompt, 128 greedy tokens.

Bar: the greedy tokens equal the CPU oracle's (tests/golden/config4_tokens.json,
written by tests/golden/make_config4_golden.py from the same seeded weights,
whose SHA-256 is checked first), bit for bit, with the default (ordered)
prefill; the matrix-core prefill must give the same first token.
"""
import hashlib
import json

import numpy as np
import pytest

from conftest import GOLDEN

pytestmark = pytest.mark.gpu


def _sha256(path, chunk=1 << 24):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        for b in iter(lambda: f.read(chunk), b""):
            h.update(b)
    return h.hexdigest()


@pytest.fixture(scope="module")
def golden():
    return json.loads((GOLDEN / "config4_tokens.json").read_text())


@pytest.fixture(scope="module")
def artifact(tmp_path_factory, golden):
    from spock_amd import model
    a = golden["artifact"]
    p = tmp_path_factory.mktemp("config4") / "artifact"
    print("[config4] writing the synthetic artifact", flush=True)
    model.write_synthetic_artifact(p, layers=a["layers"], vocab=a["vocab"], seed=a["seed"])
    assert _sha256(p / "text_weights.bin") == a["text_weights_sha256"], "synthetic weights differ from the golden's"
    return p


def _prompt(golden):
    from spock_amd import synth
    n = golden["prompt"]["length"]
    return (synth.splitmix64(4, n) % np.uint64(golden["artifact"]["vocab"])).astype(np.int32)


@pytest.mark.parametrize("fused", [False, True])
def test_config4_greedy_tokens_bitexact(dev, artifact, golden, fused):
    """fused: each DeltaNet layer's input projections and decode step in one
    launch (spk_deltanet_inproj_step)."""
    from spock_amd import model
    print(f"[config4] ordered prefill + 128 greedy tokens, fused step {fused}", flush=True)
    with model.Session(artifact, fused_dn_step=fused) as s:
        r = s.generate(_prompt(golden), golden["new_tokens"])
    got = r.tokens.tolist()
    want = golden["tokens"]
    first_bad = next((i for i, (a, b) in enumerate(zip(got, want)) if a != b), None)
    print(f"[config4] prefill {r.prefill_ms:.1f} ms, decode {r.decode_ms:.1f} ms for {r.decode_steps} steps, "
          f"first mismatch {first_bad}", flush=True)
    assert got == want


def test_config4_matrix_prefill_first_token(dev, artifact, golden):
    from spock_amd import model
    print("[config4] matrix-core prefill", flush=True)
    with model.Session(artifact, matrix_prefill=True) as s:
        r = s.generate(_prompt(golden), 8)
    assert int(r.tokens[0]) == golden["tokens"][0]
