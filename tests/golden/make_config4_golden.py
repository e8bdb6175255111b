"""Writes tests/golden/config4_tokens.json: the CPU oracle's greedy tokens for
config 4 (full Qwen3.5-0.8B-shaped model, 24 layers, vocab 248320, seeded
synthetic weights, 512-token prompt, 128 greedy tokens), with the SHA-256 of
the synthetic weights the tokens were computed on.

    python tests/golden/make_config4_golden.py [--workdir /tmp/spock-config4]

The weights come from the product's seeded artifact writer
(spock_amd.model.write_synthetic_artifact); the tokens from the oracle's
full-model restatement (oracle/model.c).  Takes a few minutes on 8 cores.
"""
import argparse
import hashlib
import json
import sys
import time
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

import numpy as np  # noqa: E402

LAYERS, VOCAB, SEED = 24, 248320, 2026
PROMPT_LEN, NEW_TOKENS, PROMPT_SEED = 512, 128, 4


def prompt():
    from spock_amd import synth
    return (synth.splitmix64(PROMPT_SEED, PROMPT_LEN) % np.uint64(VOCAB)).astype(np.int32)


def sha256_file(path, chunk=1 << 24):
    h = hashlib.sha256()
    with open(path, "rb") as f:
        while True:
            b = f.read(chunk)
            if not b:
                break
            h.update(b)
    return h.hexdigest()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--workdir", default="/tmp/spock-config4")
    args = ap.parse_args()
    from spock_amd import model
    import oracle_model
    art = Path(args.workdir) / "artifact"
    model.write_synthetic_artifact(art, layers=LAYERS, vocab=VOCAB, seed=SEED)
    digest = sha256_file(art / "text_weights.bin")
    om = oracle_model.OracleModel(art, max_seq=2048)
    t0 = time.time()
    toks = om.generate(prompt(), NEW_TOKENS)
    out = {
        "config": "config4: 24 layers (18 gated DeltaNet, 6 full attention), hidden 1024, vocab 248320",
        "artifact": {"layers": LAYERS, "vocab": VOCAB, "seed": SEED, "text_weights_sha256": digest},
        "prompt": {"length": PROMPT_LEN, "generator": "splitmix64(seed=4) % vocab"},
        "new_tokens": NEW_TOKENS,
        "tokens": [int(t) for t in toks],
        "oracle_seconds": round(time.time() - t0, 1),
    }
    (HERE / "config4_tokens.json").write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps({k: v for k, v in out.items() if k != "tokens"}))


if __name__ == "__main__":
    main()
