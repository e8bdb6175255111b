"""Pins the oracle's chunk rule (oracle.c orc_chunk_rule, restating
deltanet_chunk.cpp:53-284) against:
  - the reference's own compiled rule: golden digests written by
    tests/golden/make_golden.py from oracle/_ref, and live when _ref is built;
  - the fp64 token-sequential recurrence (closed form of the chunk rule);
  - special cases that reduce to something known (C=1, beta=0, padding,
    orthonormal keys with beta=1 and g=0).
"""
import hashlib
import json

import numpy as np
import pytest

import chunk_cases
from conftest import GOLDEN, max_rel


def _sha(a):
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


GOLD = json.loads((GOLDEN / "chunk_cases.json").read_text())


@pytest.mark.parametrize("name", sorted(GOLD))
def test_oracle_matches_reference_golden(oracle, name):
    g = GOLD[name]
    inp = chunk_cases.make_inputs(name)
    assert chunk_cases.inputs_digest(inp) == g["inputs_sha256"], "input regeneration drifted"
    core, state = oracle.chunk_rule(inp["q"], inp["k"], inp["v"], inp["g"], inp["beta"],
                                    chunk=g["spec"]["C"])
    assert _sha(core) == g["core_sha256"]
    assert _sha(state) == g["state_sha256"]


def test_oracle_matches_reference_unit_case(oracle):
    """The reference unit test's case (tests/run_deltanet_chunk_unit.py:104-128)."""
    z = np.load(GOLDEN / "chunk_unit_case.npz")
    H, T, dk, dv, C, l2 = z["meta"]
    core, state = oracle.chunk_rule(z["q"], z["k"], z["v"], z["g"], z["beta"], init=z["init"],
                                    chunk=int(C), l2=bool(l2))
    assert np.array_equal(core.view(np.uint32), z["core"].view(np.uint32))
    assert np.array_equal(state.view(np.uint32), z["state"].view(np.uint32))
    # and the reference's own tolerance against its torch rule: |diff| <= 1e-5
    c64, s64 = oracle.delta_recurrence_f64(z["q"], z["k"], z["v"], z["g"], z["beta"],
                                           init=z["init"], l2=True)
    assert np.abs(core - c64).max() <= 1e-5 and np.abs(state - s64).max() <= 1e-5


@pytest.mark.skipif(not __import__("oracle_lib").ref_available(), reason="oracle/_ref not built")
@pytest.mark.parametrize("H,T,C,l2,init", [(3, 1, 64, False, False), (2, 63, 64, True, True),
                                           (2, 65, 64, False, True), (1, 130, 16, True, False),
                                           (4, 37, 8, False, True)])
def test_oracle_bitexact_vs_reference_live(oracle, H, T, C, l2, init):
    inp = __import__("spock_amd.synth", fromlist=["x"]).chunk_inputs(H, T, seed=7 + T, l2=not l2)
    st0 = np.random.default_rng(T).normal(0, 0.1, (H, 128, 128)).astype(np.float32) if init else None
    a = oracle.chunk_rule(**inp, init=st0, chunk=C, l2=l2)
    b = oracle.chunk_rule(**inp, init=st0, chunk=C, l2=l2, use_ref=True)
    for x, y in zip(a, b):
        assert np.array_equal(x.view(np.uint32), y.view(np.uint32))


@pytest.mark.parametrize("T,C", [(104, 64), (64, 64), (1, 64), (200, 32), (33, 1)])
def test_chunk_rule_equals_recurrence(oracle, T, C):
    from spock_amd import synth
    inp = synth.chunk_inputs(4, T, seed=T)
    init = np.random.default_rng(1).normal(0, 0.05, (4, 128, 128)).astype(np.float32)
    core, state = oracle.chunk_rule(**inp, init=init, chunk=C)
    c64, s64 = oracle.delta_recurrence_f64(**inp, init=init)
    assert max_rel(core, c64) < 2e-6
    assert max_rel(state, s64) < 2e-6


def test_beta_zero_is_pure_decay(oracle):
    from spock_amd import synth
    inp = synth.chunk_inputs(2, 70, seed=3)
    inp["beta"][:] = 0.0
    init = np.random.default_rng(2).normal(0, 1, (2, 128, 128)).astype(np.float32)
    core, state = oracle.chunk_rule(**inp, init=init)
    gsum = inp["g"].astype(np.float64).sum(axis=1)
    assert max_rel(state, init * np.exp(gsum)[:, None, None]) < 1e-5
    gc = np.cumsum(inp["g"].astype(np.float64), axis=1)
    scale = 1 / np.sqrt(128.0)
    expect = np.einsum("htk,hkv->htv", inp["q"].astype(np.float64) * scale, init) * np.exp(gc)[..., None]
    assert max_rel(core, expect) < 1e-5


def test_padding_tokens_do_not_change_state(oracle):
    """T=104 is zero-padded to 128 internally; an explicit zero tail (g=0,
    beta=0, k=v=0) must give the same result bit for bit."""
    from spock_amd import synth
    inp = synth.chunk_inputs(3, 104, seed=11)
    core, state = oracle.chunk_rule(**inp)
    pad = {k_: np.concatenate([v_, np.zeros((3, 24) + v_.shape[2:], np.float32)], axis=1)
           for k_, v_ in inp.items()}
    core2, state2 = oracle.chunk_rule(**pad)
    assert np.array_equal(state.view(np.uint32), state2.view(np.uint32))
    assert np.array_equal(core.view(np.uint32), core2[:, :104].view(np.uint32))


def test_orthonormal_keys_overwrite(oracle):
    """beta=1, g=0 and orthonormal keys: after token t, S^T k_t == v_t."""
    H, T = 1, 48
    rng = np.random.default_rng(5)
    Q, _ = np.linalg.qr(rng.normal(size=(128, 128)))
    k = Q[:T].astype(np.float32)[None]
    v = rng.normal(size=(1, T, 128)).astype(np.float32)
    q = k.copy()
    g = np.zeros((1, T), np.float32)
    beta = np.ones((1, T), np.float32)
    core, state = oracle.chunk_rule(q, k, v, g, beta, chunk=16)
    recovered = np.einsum("tk,kv->tv", k[0].astype(np.float64), state[0].astype(np.float64))
    assert np.abs(recovered - v[0]).max() < 2e-5
    # o_t = S_t^T q_t / sqrt(128) with q_t = k_t, and S_t^T k_t = v_t
    assert np.abs(core[0] * np.sqrt(128.0) - v[0]).max() < 2e-4


def test_varlen_equals_per_sequence(oracle):
    from spock_amd import synth
    lens = [5, 0, 64, 130]
    cu = synth.cu_seqlens_from(lens)
    inp = synth.chunk_inputs(2, int(cu[-1]), seed=9)
    core, state = oracle.chunk_rule_varlen(**inp, cu=cu)
    for s, L in enumerate(lens):
        t0 = cu[s]
        if L == 0:
            assert not state[s].any()
            continue
        sub = {k_: v_[:, t0:t0 + L] for k_, v_ in inp.items()}
        c1, s1 = oracle.chunk_rule(**sub)
        assert np.array_equal(core[:, t0:t0 + L], c1)
        assert np.array_equal(state[s], s1)


def test_config_errors(oracle):
    lib = oracle.lib()
    assert lib.orc_chunk_rule(0, 1, 1, 1, 1, 0, *([None] * 8)) == -1
