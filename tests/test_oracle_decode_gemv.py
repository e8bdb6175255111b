"""Pins the oracle's decode step, GEMV, lm_head and argmax:
  - unfused recurrence == reference GPU capture (layer 0, step 1) bit for bit;
  - beta == sigmoid(captured b) within 1 ulp of the captured fp32 bits;
  - fused step vs an fp64 restatement of the shader math;
  - GEMV vs fp64 dot products rounded once, in each of the three reference
    summation orders, and rows that only the named order sums exactly;
  - argmax vs an independent restatement of argmax.comp on crafted ties.
"""
import numpy as np
import pytest

from conftest import GOLDEN, fp16_ulp

D = GOLDEN / "ref_data"


def _fixture():
    q = np.fromfile(D / "layer0_step1_dn_q_2048.fp16", np.uint16)
    k = np.fromfile(D / "layer0_step1_dn_k_2048.fp16", np.uint16)
    v = np.fromfile(D / "layer0_step1_dn_v_2048.fp16", np.uint16)
    gb = np.fromfile(D / "layer0_step1_dn_g_beta_32.u32", np.uint32).view(np.float32)
    st = np.fromfile(D / "layer0_step1_dn_recurrent_state_pre_262176.f32", np.float32).copy()
    st[16 * 128 * 128:] = gb
    core = np.fromfile(D / "layer0_step1_dn_core_2048.fp16", np.uint16)
    return np.concatenate([q, k, v]), st, core, gb


def test_fixture_digests():
    import hashlib
    for line in (D / "SHA256SUMS").read_text().splitlines():
        digest, name = line.split()
        assert hashlib.sha256((D / name).read_bytes()).hexdigest() == digest, name


def test_recurrent_matches_reference_capture_exactly(oracle):
    qkv, st, core, _ = _fixture()
    out, _ = oracle.recurrent(qkv, st)
    assert np.array_equal(out[4096:], core)


def test_beta_matches_captured_bits(oracle):
    _, _, _, gb = _fixture()
    b = oracle.h2f(np.fromfile(D / "layer0_step1_dn_b_16.fp16", np.uint16))
    beta = (np.float32(1) / (np.float32(1) + oracle.expf(-b))).astype(np.float32)
    d = np.abs(beta.view(np.int32).astype(np.int64) - gb[16:].view(np.int32).astype(np.int64))
    assert d.max() <= 1


def _decode_f64(inp, layer, eps=1e-6):
    """fp64 restatement of conv_l2_qk + recurrent_gbeta_norm_gate for one
    sequence; fp16 roundings at the shader's points (via numpy casts)."""
    h = lambda a: np.asarray(a, np.uint16).view(np.float16).astype(np.float64)
    r16 = lambda x: np.asarray(x, np.float64).astype(np.float16).astype(np.float64)
    qkv = h(inp["qkv"][0]); cs = h(inp["conv_state"][0]); w = h(inp["conv_w"])
    win = np.concatenate([cs[:, 1:], qkv[:, None]], axis=1)
    s = (win * w).sum(1)
    y = r16(s / (1 + np.exp(-s)))
    for blk in range(32):
        seg = y[blk * 128:(blk + 1) * 128]
        y[blk * 128:(blk + 1) * 128] = r16(seg / np.sqrt((seg * seg).sum() + 1e-6))
    S = inp["state"][0].astype(np.float64).copy()
    out = np.zeros(2048)
    for hh in range(16):
        a = h(inp["a"][0][hh]); b = h(inp["b"][0][hh])
        alog, dtb = inp["a_log_bias"][layer, hh].astype(np.float64)
        g = -np.exp(alog) * np.log1p(np.exp(a + dtb)); beta = 1 / (1 + np.exp(-b))
        qv = y[hh * 128:(hh + 1) * 128] / np.sqrt(128.0)
        kv = y[2048 + hh * 128: 2048 + (hh + 1) * 128]
        vv = y[4096 + hh * 128: 4096 + (hh + 1) * 128]
        Sh = S[hh] * np.exp(g)
        delta = (vv - Sh.T @ kv) * beta
        Sh = Sh + np.outer(kv, delta)
        o = Sh.T @ qv
        nrm = o / np.sqrt((o * o).mean() + eps)
        z = h(inp["z"][0][hh * 128:(hh + 1) * 128])
        out[hh * 128:(hh + 1) * 128] = r16(r16(inp["norm_w"] * nrm) * z / (1 + np.exp(-z)))
        S[hh] = Sh
    return y, out, S


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_decode_step_vs_fp64(oracle, seed):
    from spock_amd import synth
    inp = synth.decode_inputs(1, seed=seed)
    inp["norm_w"] = synth.normal(seed, 128, std=0.3, mean=1.0)
    eq, ecs, est = oracle.decode_step(inp, layer_idx=4)
    y64, out64, S64 = _decode_f64(inp, 4)
    f16 = lambda x: np.asarray(x).astype(np.float16).view(np.uint16)
    assert fp16_ulp(eq[0, :4096], f16(y64[:4096])).max() <= 1
    assert fp16_ulp(eq[0, 4096:], f16(out64)).max() <= 2
    assert np.abs(est[0] - S64).max() <= 1e-5 * max(1.0, np.abs(S64).max())
    win = np.concatenate([inp["conv_state"][0][:, 1:], inp["qkv"][0][:, None]], axis=1)
    assert np.array_equal(ecs[0], win)
    qn = eq[0, :2048].view(np.float16).astype(np.float64).reshape(16, 128)
    assert np.allclose((qn ** 2).sum(1), 1.0, atol=3e-3)  # unit L2 norm per head


@pytest.mark.parametrize("out_dim,in_dim", [(64, 1024), (33, 3584), (17, 64), (8, 2048)])
def test_matvec_vs_fp64(oracle, out_dim, in_dim):
    from spock_amd import synth
    W = synth.gemv_weights(out_dim, in_dim, seed=in_dim)
    x = synth.gemv_input(in_dim, seed=out_dim)
    y = oracle.matvec_f16(W, x)
    exact = W.view(np.float16).astype(np.float64) @ x.view(np.float16).astype(np.float64)
    assert fp16_ulp(y, exact.astype(np.float16).view(np.uint16)).max() <= 1


@pytest.mark.parametrize("order", ["strided", "serial"])
@pytest.mark.parametrize("out_dim,in_dim", [(64, 1024), (33, 3584), (17, 64), (9, 200), (5, 1000), (3, 1)])
def test_matvec_orders_vs_fp64(oracle, order, out_dim, in_dim):
    from spock_amd import synth
    W = synth.gemv_weights(out_dim, in_dim, seed=in_dim + 3)
    x = synth.gemv_input(in_dim, seed=out_dim + 5)
    y = oracle.matvec_f16_order(W, x, order)
    exact = W.view(np.float16).astype(np.float64) @ x.view(np.float16).astype(np.float64)
    assert fp16_ulp(y, exact.astype(np.float16).view(np.uint16)).max() <= 1


def _cancel_rows(in_dim):
    """One row per summation order whose exact sum only that order keeps
    (x = 1): +L and -L (L = 2048) meet first inside one of that order's
    partial sums, so the small terms (s = 2^-14, sums exact in fp32) survive.
    In the other orders at least one small term is added to +L or -L on its
    own first, and s is a quarter of an fp32 ulp of 2048, so it is lost."""
    L, s = 2048.0, 2.0 ** -14
    sp = in_dim // 64 if in_dim % 64 == 0 else 4
    rows = {}
    w = np.full(in_dim, s)          # matvec_tiled: lanes 5 and 37 meet at tree stride 32
    w[5::64] = 0.0
    w[37::64] = 0.0
    w[5], w[37] = L, -L
    rows["strided"] = w
    w = np.full(in_dim, s)          # matvec: +L, zeros, then -L opens lane 1's span
    w[0], w[1:sp], w[sp] = L, 0.0, -L
    rows["serial"] = w
    if in_dim % 64 == 0 and sp >= 2:
        w = np.full(in_dim, s)      # lm_head_tiled: both open lane 2's span; one s before them
        w[1:2 * sp] = 0.0
        w[2 * sp], w[2 * sp + 1] = L, -L
        rows["spans"] = w
    return rows


@pytest.mark.parametrize("in_dim", [256, 200, 1024])
def test_matvec_orders_cancellation_rows(oracle, in_dim):
    rows = _cancel_rows(in_dim)
    x = np.full(in_dim, np.float16(1.0)).view(np.uint16)
    orders = [o for o in ("strided", "serial", "spans") if o != "spans" or in_dim % 64 == 0]
    for row_order, w in rows.items():
        exact = np.float16(w.sum())  # L - L cancels; the small terms are exact
        assert exact != 0
        W = w.astype(np.float16).view(np.uint16).reshape(1, in_dim)
        for order in orders:
            got = oracle.matvec_f16_order(W, x, order)[0]
            if order == row_order:
                assert got == exact.view(np.uint16), (row_order, order)
            else:
                assert got != exact.view(np.uint16), (row_order, order)


def _argmax_shader(vals):
    """Independent restatement of argmax.comp:27-63 (256 invocations)."""
    v = vals.view(np.float16).astype(np.float32)
    n = len(v)
    E = (n + 255) // 256
    best = []
    for l in range(256):
        m, mi = -3.402823466e38, 0
        for i in range(l * E, min(n, l * E + E)):
            if v[i] > m:
                m, mi = v[i], i
        best.append((m, mi))
    stride = 128
    while stride:
        for l in range(stride):
            if best[l + stride][0] > best[l][0]:
                best[l] = best[l + stride]
        stride //= 2
    return best[0][1]


def test_argmax_tie_rules(oracle):
    rng = np.random.default_rng(0)
    n = 2560  # E = 10
    cases = []
    v = np.zeros(n, np.float16); v[[640, 1280]] = 3; cases.append(v)      # bit-reversed lane order
    v = np.zeros(n, np.float16); v[[7, 5]] = 1; cases.append(v)           # same lane: first
    cases.append(np.full(n, np.nan, np.float16))
    v = np.full(n, -np.inf, np.float16); v[999] = -65504; cases.append(v)
    v = np.zeros(n, np.float16); v[::3] = -0.0; cases.append(v)
    for _ in range(20):
        cases.append(rng.integers(-2, 3, n).astype(np.float16))
    for v in cases:
        u = v.view(np.uint16)
        assert oracle.argmax_f16(u) == _argmax_shader(u)
    # the tie rule is not "lowest index": blocks 64 and 128 tie -> block 128 wins
    v = np.zeros(n, np.float16); v[[640, 1280]] = 3
    assert oracle.argmax_f16(v.view(np.uint16)) == 1280
