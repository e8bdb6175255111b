"""GPU parity of the Qwen3.5-shaped decode session (include/spock_model.h)
against the oracle's full model (oracle/model.h) on seeded synthetic artifacts.

* Decode: from an identical state (the oracle's, after its prefill), every
  decode step gives bit-identical greedy tokens, fp16 logits and hidden state
  (the per-token operation order is the oracle's), with and without the
  recorded HIP graph.
* Default (ordered) prefill: bit-identical logits, hidden state, DeltaNet
  state, conv state and KV cache; greedy generation token-for-token equal.
* Matrix-core prefill (MFMA projections and chunk rule): close to the oracle
  (fp32 accumulation order differs), same greedy token.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

LAYERS, VOCAB, SEED, MAX_SEQ = 4, 8192, 11, 256


@pytest.fixture(scope="module")
def small_artifact(tmp_path_factory):
    from spock_amd import model
    p = tmp_path_factory.mktemp("art") / "small"
    model.write_synthetic_artifact(p, layers=LAYERS, vocab=VOCAB, seed=SEED)
    return p


def _prompt(n, seed=5):
    from spock_amd import synth
    return (synth.splitmix64(seed, n) % np.uint64(VOCAB)).astype(np.int32)


@pytest.mark.parametrize("use_graph,one_launch,fused", [(True, True, True), (False, True, True),
                                                        (True, False, True), (True, True, False),
                                                        (False, False, False)])
def test_decode_from_oracle_state_bitexact(dev, small_artifact, use_graph, one_launch, fused):
    """one_launch=False: the final norm + lm_head with the atomic key, then
    the take, instead of the default single launch.  fused=False: each
    DeltaNet layer's input projections and decode step as two launches."""
    import oracle_model
    from spock_amd import model
    print(f"[session decode graph={use_graph} lm_head one_launch={one_launch} fused={fused}]", flush=True)
    om = oracle_model.OracleModel(small_artifact, max_seq=MAX_SEQ)
    prompt = _prompt(70)
    tok = om.prefill(prompt)
    snap = om.snapshot()
    want = []
    t = tok
    for i in range(12):
        t, logits, hidden = om.decode(t, want_logits=True)
        want.append(t)
    with model.Session(small_artifact, max_seq=MAX_SEQ, use_graph=use_graph, lm_head_one_launch=one_launch,
                       fused_dn_step=fused) as s:
        s.set_state(snap["dn_state"], snap["conv"], snap["kv"], snap["pos"], tok)
        got = s.decode(12)
        glogits, ghidden = s.last_output()
        st = s.get_state()
    assert got.tolist() == want
    assert np.array_equal(ghidden, hidden)
    assert np.array_equal(glogits, logits)
    assert st["pos"] == 70 + 12
    assert np.array_equal(st["dn_state"].view(np.uint32), om.snapshot()["dn_state"].view(np.uint32))
    assert np.array_equal(st["conv"], om.snapshot()["conv"])
    assert np.array_equal(st["kv"], om.snapshot()["kv"])


def test_ordered_prefill_and_generate_bitexact(dev, small_artifact):
    import oracle_model
    from spock_amd import model
    print("[session ordered prefill + generate]", flush=True)
    om = oracle_model.OracleModel(small_artifact, max_seq=MAX_SEQ)
    prompt = _prompt(133, seed=9)
    tok, logits, hidden = om.prefill(prompt, want_logits=True)
    snap = om.snapshot()
    with model.Session(small_artifact, max_seq=MAX_SEQ) as s:
        gtok = s.prefill(prompt)
        glogits, ghidden = s.last_output()
        st = s.get_state()
        assert gtok == tok
        assert np.array_equal(glogits, logits) and np.array_equal(ghidden, hidden)
        assert np.array_equal(st["dn_state"].view(np.uint32), snap["dn_state"].view(np.uint32))
        assert np.array_equal(st["conv"], snap["conv"]) and np.array_equal(st["kv"], snap["kv"])
        r = s.generate(prompt, 24)
    want = om.generate(prompt, 24)
    assert r.tokens.tolist() == want.tolist()


def test_matrix_prefill_close_to_oracle(dev, small_artifact):
    import oracle_model
    from spock_amd import model
    print("[session matrix prefill]", flush=True)
    om = oracle_model.OracleModel(small_artifact, max_seq=MAX_SEQ)
    prompt = _prompt(133, seed=9)
    tok, logits, hidden = om.prefill(prompt, want_logits=True)
    with model.Session(small_artifact, max_seq=MAX_SEQ, matrix_prefill=True) as s:
        gtok = s.prefill(prompt)
        glogits, ghidden = s.last_output()
        st = s.get_state()
    lf = logits.view(np.float16).astype(np.float32)
    gf = glogits.view(np.float16).astype(np.float32)
    diff = float(np.max(np.abs(lf - gf)))
    sd = float(np.max(np.abs(st["dn_state"] - om.snapshot()["dn_state"])))
    print(f"prefill: max |logit diff| {diff:.4g}, max |state diff| {sd:.3g}, tokens {gtok} vs {tok}")
    assert gtok == tok
    assert diff <= 0.05
    assert sd <= 1e-2
    assert st["pos"] == 133


def test_generate_api_and_errors(dev, small_artifact):
    from spock_amd import model
    with model.Session(small_artifact, max_seq=64) as s:
        r = s.generate(_prompt(20), 10)
        assert len(r.tokens) == 10 and r.decode_steps == 9 and r.used_graph
        assert all(0 <= t < VOCAB for t in r.tokens)
        r2 = s.generate(_prompt(20), 10)  # decode() resets: same prompt, same tokens
        assert r2.tokens.tolist() == r.tokens.tolist()
        with pytest.raises(model.ModelError, match="max_seq"):
            s.generate(_prompt(60), 10)
        with pytest.raises(model.ModelError, match="vocab"):
            s.prefill([VOCAB + 1])


def test_long_generation_past_8192_tokens(dev, small_artifact):
    """The token history holds one entry per position (capacity max_seq), so
    a session with max_seq > 8192 generates more than 8192 tokens; asking for
    more than max_seq allows is a clean error, not an out-of-range copy."""
    from spock_amd import model
    print("[session 8300-token generation, max_seq 9000]", flush=True)
    with model.Session(small_artifact, max_seq=9000) as s:
        short = s.generate(_prompt(8), 24)
        r = s.generate(_prompt(8), 8300)
        assert len(r.tokens) == 8300 and r.decode_steps == 8299
        assert r.tokens[:24].tolist() == short.tokens.tolist()
        assert all(0 <= t < VOCAB for t in r.tokens)
        with pytest.raises(model.ModelError, match="max_seq"):
            s.generate(_prompt(8), 8994)


@pytest.mark.parametrize("use_graph,n", [(True, 12), (False, 12), (True, 200)])
def test_gpu_timestamps(dev, small_artifact, use_graph, n):
    """Per-step and per-region GPU times (DecodeResult::per_token_gpu_us and
    gpu_region_us, vk_decode.hpp:19-20): same tokens as an untimed session;
    one time per decode step; the regions of a step tile it exactly, in step
    order, so their sums equal the per-step sum.  200 tokens run past two
    64-step event batches, so the event sets are reused."""
    from spock_amd import model
    print(f"[session gpu timestamps graph={use_graph} n={n}]", flush=True)
    prompt = _prompt(20)
    with model.Session(small_artifact, max_seq=256, use_graph=use_graph) as s:
        base = s.generate(prompt, n)
        assert base.per_token_gpu_us is None and base.gpu_region_us is None
    with model.Session(small_artifact, max_seq=256, use_graph=use_graph, gpu_timestamps=1) as s:
        r = s.generate(prompt, n)
    assert r.tokens.tolist() == base.tokens.tolist() and r.used_graph == use_graph
    assert r.gpu_region_us is None
    t = r.per_token_gpu_us
    assert t is not None and len(t) == n - 1 and (t > 0).all()
    assert 0.5 * r.gpu_decode_ms * 1e3 <= t.sum() <= r.gpu_decode_ms * 1e3 * (1 + 1e-6) + 1.0
    with model.Session(small_artifact, max_seq=256, use_graph=use_graph, gpu_timestamps=2) as s:
        r2 = s.generate(prompt, n)
        assert r2.tokens.tolist() == base.tokens.tolist() and not r2.used_graph
        t2, reg = r2.per_token_gpu_us, r2.gpu_region_us
        assert t2 is not None and len(t2) == n - 1 and (t2 > 0).all()
        assert list(reg) == [f"layer_{i}" for i in range(LAYERS)] + ["lm_head", "argmax"]
        assert all(v > 0 for v in reg.values())
        assert abs(sum(reg.values()) - t2.sum()) <= 1e-3 * t2.sum() + 0.05
        # a call without decode steps leaves no timings
        r3 = s.generate(prompt, 1)
        assert r3.per_token_gpu_us is None and r3.gpu_region_us is None
    with pytest.raises(model.ModelError, match="gpu_timestamps"):
        model.Session(small_artifact, max_seq=64, gpu_timestamps=3)
