"""GPU parity of the Qwen3.5 model kernels (include/spock_hip.h, model section)
against the oracle (oracle/model.h).

Bar: bit-exact fp16 outputs for every decode-path kernel (fused projections,
attention, norms, gates, DeltaNet prompt conv / g / beta / gated norm), whose
operation order the oracle restates; the MFMA prompt GEMM is checked against
an fp64 product within the fp32-accumulation error bound K 2^-24 sum|a w| plus
one fp16 rounding (its accumulation order is the matrix cores', not the
matvec's), and must be correctly rounded for the typical element.
"""
import ctypes as C

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _h(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.uint16).view(np.float16)).to(dev)


def _f(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)


def _u16(t):
    return t.cpu().numpy().view(np.uint16)


def _p(a):
    return a.ctypes.data


def _rand16(seed, n, std=1.0):
    from spock_amd import synth
    return synth.f16(synth.normal(seed, n, std=std))


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _om():
    import oracle_model
    return oracle_model.lib()


def _orc_matvec(W, x):
    out = np.zeros(W.shape[0], np.uint16)
    _om().orc_matmul_rows(_p(W), _p(x), _p(out), W.shape[0], W.shape[1], 1)
    return out


def _gemv(inp, outs):
    from spock_amd import _lib
    arr = (_lib.SpkGemvOutput * len(outs))()
    for i, (W, y, res, n) in enumerate(outs):
        arr[i].W, arr[i].y, arr[i].residual, arr[i].out_dim = W, y, res, n
    _lib.check(_lib.lib().spk_gemv_fused(C.byref(inp), arr, len(outs), _stream()), "spk_gemv_fused")


# up to 4 outputs run in one launch; 5..8 are split over two launches (the
# first alone writes h_out)
@pytest.mark.parametrize("shapes", [[6144, 2048, 16, 16], [16, 512, 1024, 20, 2048, 48]])
def test_gemv_rmsnorm_with_embedding_row(dev, shapes):
    from spock_amd import _lib
    print(f"[gemv rmsnorm+token {shapes}]", flush=True)
    V = 512
    E = _rand16(1, V * 1024, 0.02).reshape(V, 1024)
    w = _rand16(2, 1024, 0.02)
    Ws = [_rand16(10 + i, n * 1024, 0.02).reshape(n, 1024) for i, n in enumerate(shapes)]
    tok = 317
    dE, dw = _h(E, dev), _h(w, dev)
    dWs = [_h(W, dev) for W in Ws]
    ys = [torch.empty(n, dtype=torch.float16, device=dev) for n in shapes]
    h_out = torch.empty(1024, dtype=torch.float16, device=dev)
    dtok = torch.tensor([tok], dtype=torch.int32, device=dev)
    inp = _lib.SpkGemvInput()
    inp.kind, inp.in_dim, inp.x, inp.x2 = _lib.SPK_GEMV_IN_RMSNORM, 1024, dE.data_ptr(), dw.data_ptr()
    inp.token, inp.token_rows, inp.h_out = dtok.data_ptr(), V, h_out.data_ptr()
    _gemv(inp, [(W.data_ptr(), y.data_ptr(), None, n) for W, y, n in zip(dWs, ys, shapes)])
    torch.cuda.synchronize()
    xn = np.zeros(1024, np.uint16)
    _om().orc_rmsnorm1024(_p(np.ascontiguousarray(E[tok])), _p(w), _p(xn))
    assert np.array_equal(_u16(h_out), E[tok])
    for W, y in zip(Ws, ys):
        assert np.array_equal(_u16(y), _orc_matvec(W, xn))


@pytest.mark.parametrize("in_dim,silu", [(2048, False), (3584, True), (1024, False), (512, True)])
def test_gemv_plain_or_silu_with_residual_in_place(dev, in_dim, silu):
    from spock_amd import _lib
    print(f"[gemv in={in_dim} silu={silu}]", flush=True)
    n = 1024
    W = _rand16(20, n * in_dim, 0.02).reshape(n, in_dim)
    x = _rand16(21, in_dim)
    u = _rand16(22, in_dim)
    r = _rand16(23, n)
    dW, dx, du, dr = _h(W, dev), _h(x, dev), _h(u, dev), _h(r, dev)
    inp = _lib.SpkGemvInput()
    inp.kind = _lib.SPK_GEMV_IN_SILU_GATE if silu else _lib.SPK_GEMV_IN_PLAIN
    inp.in_dim, inp.x, inp.x2 = in_dim, dx.data_ptr(), du.data_ptr() if silu else None
    _gemv(inp, [(dW.data_ptr(), dr.data_ptr(), dr.data_ptr(), n)])
    torch.cuda.synchronize()
    xin = x
    if silu:
        xin = np.zeros(in_dim, np.uint16)
        _om().orc_silu_gate(_p(x), _p(u), _p(xin), in_dim)
    d = _orc_matvec(W, xin)
    exp = np.zeros(n, np.uint16)
    _om().orc_residual_add(_p(r), _p(d), _p(exp), n)
    assert np.array_equal(_u16(dr), exp)


@pytest.mark.parametrize("with_token", [False, True])
def test_deltanet_inproj_step_equals_the_two_calls(dev, with_token):
    """spk_deltanet_inproj_step (projections and decode step in one launch,
    the last of a head's workgroups running its step) against
    spk_gemv_fused + spk_deltanet_decode_step on copies of the same buffers,
    two steps in a row: every output, the state and the conv history bit for
    bit, and the arrival counts back at zero after each call."""
    from spock_amd import _lib, synth
    print(f"[inproj+step token={with_token}]", flush=True)
    lib = _lib.lib()
    V = 512
    E = _rand16(30, V * 1024).reshape(V, 1024)
    nrm = _rand16(31, 1024, 0.1)
    shapes = [6144, 2048, 16, 16]
    Ws = [_h(_rand16(32 + i, n * 1024, 0.02).reshape(n, 1024), dev) for i, n in enumerate(shapes)]
    dE, dn = _h(E, dev), _h(nrm, dev)
    dtok = torch.tensor([211], dtype=torch.int32, device=dev)
    inp = synth.decode_inputs(1, seed=7)
    nw = np.random.default_rng(8).uniform(0.5, 1.5, 128).astype(np.float32)
    shared = {"conv_w": _h(inp["conv_w"], dev), "alb": _f(inp["a_log_bias"], dev), "nw": _f(nw, dev)}
    arrive = torch.zeros(16 * 64, dtype=torch.int32, device=dev)

    def buffers():
        b = {"state": _f(inp["state"], dev), "conv": _h(inp["conv_state"], dev), "h_out": torch.zeros(1024, dtype=torch.float16, device=dev)}
        b["x"] = dE if with_token else _h(E[5], dev)
        b["ys"] = [torch.zeros(n, dtype=torch.float16, device=dev) for n in shapes]
        return b

    def args(b):
        gi = _lib.SpkGemvInput()
        gi.kind, gi.in_dim, gi.x, gi.x2 = _lib.SPK_GEMV_IN_RMSNORM, 1024, b["x"].data_ptr(), dn.data_ptr()
        if with_token:
            gi.token, gi.token_rows, gi.h_out = dtok.data_ptr(), V, b["h_out"].data_ptr()
        outs = (_lib.SpkGemvOutput * 4)()
        for i, (W, y, n) in enumerate(zip(Ws, b["ys"], shapes)):
            outs[i].W, outs[i].y, outs[i].out_dim = W.data_ptr(), y.data_ptr(), n
        d = _lib.SpkDecodeArgs()
        d.batch, d.num_heads, d.layer_idx = 1, 16, 5
        d.qkv, d.qkv_stride = b["ys"][0].data_ptr(), 6144
        d.conv_state, d.conv_state_stride, d.conv_weight = b["conv"].data_ptr(), 6144 * 4, shared["conv_w"].data_ptr()
        d.a, d.b, d.ab_stride = b["ys"][2].data_ptr(), b["ys"][3].data_ptr(), 16
        d.a_log_bias, d.state, d.state_stride = shared["alb"].data_ptr(), b["state"].data_ptr(), 16 * 128 * 128
        d.z, d.z_stride, d.norm_weight = b["ys"][1].data_ptr(), 2048, shared["nw"].data_ptr()
        return gi, outs, d

    ref, fus = buffers(), buffers()
    gr, orr, dr = args(ref)
    gf, of, df = args(fus)
    for step in range(2):
        _lib.check(lib.spk_gemv_fused(C.byref(gr), orr, 4, _stream()), "projections")
        _lib.check(lib.spk_deltanet_decode_step(C.byref(dr), _stream()), "decode step")
        _lib.check(lib.spk_deltanet_inproj_step(C.byref(gf), of, C.byref(df), arrive.data_ptr(), _stream()),
                   "inproj step")
        torch.cuda.synchronize()
        for i in range(4):
            assert torch.equal(ref["ys"][i], fus["ys"][i]), (step, i)
        assert torch.equal(ref["state"], fus["state"]), step
        assert torch.equal(ref["conv"], fus["conv"]), step
        assert torch.equal(ref["h_out"], fus["h_out"]), step
        assert int(arrive.abs().sum()) == 0, step


def test_workgroups_are_dealt_to_xcds_round_robin(dev):
    """The fused DeltaNet launch and the attention combine hand rows between
    workgroups whose ids are congruent mod 8 through the L2 of their XCD:
    the dispatch must deal workgroup ids to the 8 XCDs round-robin.  The
    first workgroup's XCD continues the rotation of earlier dispatches (seen
    at 0 and at 6), so the check is (id + start) mod 8, over several
    launches of different sizes."""
    from spock_amd import _lib
    for n in (4096, 4093, 37, 4096):
        out = torch.full((n,), -1, dtype=torch.int32, device=dev)
        _lib.check(_lib.lib().spk_selftest_xcc_ids(n, out.data_ptr(), _stream()), "xcc ids")
        torch.cuda.synchronize()
        ids = out.cpu().numpy()
        assert 0 <= ids[0] < 8, ids[0]
        assert np.array_equal(ids, (np.arange(n) + ids[0]) % 8), (n, np.unique(ids))


def test_deltanet_inproj_step_rejects_bad_args(dev):
    from spock_amd import _lib
    lib = _lib.lib()
    gi = _lib.SpkGemvInput()
    gi.kind, gi.in_dim = _lib.SPK_GEMV_IN_PLAIN, 1024
    outs = (_lib.SpkGemvOutput * 4)()
    d = _lib.SpkDecodeArgs()
    arrive = torch.zeros(16 * 64, dtype=torch.int32, device=dev)
    assert lib.spk_deltanet_inproj_step(C.byref(gi), outs, C.byref(d), None, _stream()) == -1
    x = torch.zeros(1024, dtype=torch.float16, device=dev)
    gi.x, gi.x2 = x.data_ptr(), x.data_ptr()
    assert lib.spk_deltanet_inproj_step(C.byref(gi), outs, C.byref(d), arrive.data_ptr(), _stream()) == -5  # kind


def test_gemv_rejects_aliasing_and_shapes(dev):
    from spock_amd import _lib
    x = torch.zeros(1024, dtype=torch.float16, device=dev)
    W = torch.zeros(16, 1024, dtype=torch.float16, device=dev)
    inp = _lib.SpkGemvInput()
    inp.kind, inp.in_dim, inp.x = _lib.SPK_GEMV_IN_PLAIN, 1024, x.data_ptr()
    arr = (_lib.SpkGemvOutput * 1)()
    arr[0].W, arr[0].y, arr[0].out_dim = W.data_ptr(), x.data_ptr(), 16
    assert _lib.lib().spk_gemv_fused(C.byref(inp), arr, 1, _stream()) == -5
    inp.kind, inp.in_dim = _lib.SPK_GEMV_IN_RMSNORM, 2048
    assert _lib.lib().spk_gemv_fused(C.byref(inp), arr, 1, _stream()) == -2


def _attn_inputs(seed, max_seq, pos, T=1):
    import oracle_model
    rope = np.zeros(max_seq * 64, np.float32)
    oracle_model.lib().orc_rope_table(max_seq, _p(rope))
    kv = np.zeros(max_seq * 1024, np.uint16)
    kv[: pos * 1024] = _rand16(seed, pos * 1024)
    qg = _rand16(seed + 1, T * 4096)
    k = _rand16(seed + 2, T * 512)
    v = _rand16(seed + 3, T * 512)
    qn = _rand16(seed + 4, 256, 0.02)
    kn = _rand16(seed + 5, 256, 0.02)
    return rope, kv, qg, k, v, qn, kn


def _oracle_attention(rope, kv, qg, k, v, qn, kn, pos0, T):
    """Per token in order: norms, RoPE, cache store, attention, sigmoid gate."""
    L = _om()
    kv = kv.copy()
    out = np.zeros(T * 2048, np.uint16)
    for t in range(T):
        pos = pos0 + t
        q = np.zeros(2048, np.uint16)
        for h in range(8):
            L.orc_head_rmsnorm256(_p(np.ascontiguousarray(qg[t * 4096 + h * 512: t * 4096 + h * 512 + 256])),
                                  _p(qn), _p(q[h * 256:]))
        kk = np.zeros(512, np.uint16)
        for h in range(2):
            L.orc_head_rmsnorm256(_p(np.ascontiguousarray(k[t * 512 + h * 256: t * 512 + h * 256 + 256])),
                                  _p(kn), _p(kk[h * 256:]))
        cs = np.ascontiguousarray(rope[pos * 64: pos * 64 + 64])
        L.orc_rope_apply(_p(q), 8, _p(cs))
        L.orc_rope_apply(_p(kk), 2, _p(cs))
        kv[pos * 1024: pos * 1024 + 512] = kk
        kv[pos * 1024 + 512: pos * 1024 + 1024] = v[t * 512: t * 512 + 512]
        for h in range(8):
            att = np.zeros(256, np.uint16)
            L.orc_attend(_p(q[h * 256:]), _p(kv), h // 4, pos + 1, _p(att))
            gate = np.ascontiguousarray(qg[t * 4096 + h * 512 + 256: t * 4096 + h * 512 + 512])
            L.orc_sigmoid_gate(_p(att), _p(gate), _p(out[t * 2048 + h * 256:]), 256)
    return out, kv


def _attn_args(dev, rope, kv, qg, k, v, qn, kn, max_seq, T, positions):
    from spock_amd import _lib
    d = {n: _h(a, dev) for n, a in (("kv", kv), ("qg", qg), ("k", k), ("v", v), ("qn", qn), ("kn", kn))}
    d["rope"] = _f(rope, dev)
    d["out"] = torch.empty(T * 2048, dtype=torch.float16, device=dev)
    ws = int(_lib.lib().spk_attention_workspace_size(positions, T))
    d["ws"] = torch.zeros(ws, dtype=torch.uint8, device=dev)  # the o_proj form's arrival counts start at zero
    a = _lib.SpkAttnArgs()
    a.qg, a.k, a.v = d["qg"].data_ptr(), d["k"].data_ptr(), d["v"].data_ptr()
    a.q_norm_w, a.k_norm_w, a.rope = d["qn"].data_ptr(), d["kn"].data_ptr(), d["rope"].data_ptr()
    a.kv_cache, a.max_seq, a.out = d["kv"].data_ptr(), max_seq, d["out"].data_ptr()
    a.workspace, a.workspace_bytes = d["ws"].data_ptr(), ws
    return a, d


@pytest.mark.parametrize("pos", [0, 70, 511, 700])
def test_attention_inproj_equals_gemv_fused(dev, pos):
    """spk_attention_inproj: the same q|gate, k, v as spk_gemv_fused; the K/V
    rows it reads ahead (0..pos, clamped to max_seq) are left unchanged."""
    from spock_amd import _lib
    print(f"[attention inproj pos={pos}]", flush=True)
    max_seq = 512
    h = _rand16(40, 1024)
    w = _rand16(41, 1024, 0.02)
    Ws = [_rand16(42 + i, n * 1024, 0.02).reshape(n, 1024) for i, n in enumerate((4096, 512, 512))]
    kv = _rand16(45, max_seq * 1024)
    dh, dw, dkv = _h(h, dev), _h(w, dev), _h(kv, dev)
    dWs = [_h(W, dev) for W in Ws]
    ref = [torch.empty(n, dtype=torch.float16, device=dev) for n in (4096, 512, 512)]
    got = [torch.full((n,), float("nan"), dtype=torch.float16, device=dev) for n in (4096, 512, 512)]
    gi = _lib.SpkGemvInput()
    gi.kind, gi.in_dim, gi.x, gi.x2 = _lib.SPK_GEMV_IN_RMSNORM, 1024, dh.data_ptr(), dw.data_ptr()
    _gemv(gi, [(W.data_ptr(), y.data_ptr(), None, n) for W, y, n in zip(dWs, ref, (4096, 512, 512))])
    outs = (_lib.SpkGemvOutput * 3)()
    for o, W, y, n in zip(outs, dWs, got, (4096, 512, 512)):
        o.W, o.y, o.out_dim = W.data_ptr(), y.data_ptr(), n
    aa = _lib.SpkAttnArgs()
    aa.qg, aa.k, aa.v = got[0].data_ptr(), got[1].data_ptr(), got[2].data_ptr()
    dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
    aa.kv_cache, aa.max_seq, aa.pos_dev = dkv.data_ptr(), max_seq, dpos.data_ptr()
    for _ in range(2):
        _lib.check(_lib.lib().spk_attention_inproj(C.byref(gi), outs, C.byref(aa), _stream()), "spk_attention_inproj")
    torch.cuda.synchronize()
    for r, g in zip(ref, got):
        assert torch.equal(r, g)
    assert np.array_equal(_u16(dkv), kv)


@pytest.mark.parametrize("pos", [0, 1, 63, 64, 200, 511])
def test_attention_decode_bitexact(dev, pos):
    from spock_amd import _lib
    print(f"[attention decode pos={pos}]", flush=True)
    max_seq = 512
    rope, kv, qg, k, v, qn, kn = _attn_inputs(100 + pos, max_seq, pos)
    a, d = _attn_args(dev, rope, kv, qg, k, v, qn, kn, max_seq, 1, max_seq)
    dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
    a.pos_dev = dpos.data_ptr()
    _lib.check(_lib.lib().spk_attention_decode(C.byref(a), _stream()), "spk_attention_decode")
    torch.cuda.synchronize()
    exp, ekv = _oracle_attention(rope, kv, qg, k, v, qn, kn, pos, 1)
    assert np.array_equal(_u16(d["kv"]), ekv)
    assert np.array_equal(_u16(d["out"]), exp)


@pytest.mark.parametrize("pos0,T", [(0, 1), (0, 3), (61, 5), (0, 70), (30, 100), (190, 66)])
def test_attention_prefill_bitexact(dev, pos0, T):
    from spock_amd import _lib
    print(f"[attention prefill pos0={pos0} T={T}]", flush=True)
    max_seq = 256
    rope, kv, qg, k, v, qn, kn = _attn_inputs(200 + T, max_seq, pos0, T)
    a, d = _attn_args(dev, rope, kv, qg, k, v, qn, kn, max_seq, T, pos0 + T)
    _lib.check(_lib.lib().spk_attention_prefill(C.byref(a), pos0, T, _stream()), "spk_attention_prefill")
    torch.cuda.synchronize()
    exp, ekv = _oracle_attention(rope, kv, qg, k, v, qn, kn, pos0, T)
    assert np.array_equal(_u16(d["kv"]), ekv)
    assert np.array_equal(_u16(d["out"]), exp)


def test_attention_decode_position_out_of_range_writes_nothing(dev):
    from spock_amd import _lib
    max_seq = 128
    rope, kv, qg, k, v, qn, kn = _attn_inputs(7, max_seq, 5)
    a, d = _attn_args(dev, rope, kv, qg, k, v, qn, kn, max_seq, 1, max_seq)
    d["out"].fill_(0)
    dpos = torch.tensor([max_seq], dtype=torch.int32, device=dev)
    a.pos_dev = dpos.data_ptr()
    _lib.check(_lib.lib().spk_attention_decode(C.byref(a), _stream()), "spk_attention_decode")
    torch.cuda.synchronize()
    assert np.array_equal(_u16(d["kv"]), kv)
    assert not _u16(d["out"]).any()


@pytest.mark.parametrize("n,rows", [(1024, 7), (256, 13)])
def test_rmsnorm_rows_bitexact(dev, n, rows):
    from spock_amd import _lib
    x = _rand16(30 + n, rows * n)
    w = _rand16(31, n, 0.02)
    dx, dw = _h(x, dev), _h(w, dev)  # held until the kernel has run
    y = torch.empty(rows * n, dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().spk_rmsnorm_f16(dx.data_ptr(), dw.data_ptr(), y.data_ptr(), rows, n, _stream()),
               "spk_rmsnorm_f16")
    torch.cuda.synchronize()
    exp = np.zeros(rows * n, np.uint16)
    fn = _om().orc_rmsnorm1024 if n == 1024 else _om().orc_head_rmsnorm256
    for r in range(rows):
        fn(_p(np.ascontiguousarray(x[r * n:(r + 1) * n])), _p(w), _p(exp[r * n:]))
    assert np.array_equal(_u16(y), exp)


def test_elementwise_gates_bitexact(dev):
    from spock_amd import _lib
    n = 100_003
    g, u = _rand16(40, n, 3.0), _rand16(41, n)
    dg, du = _h(g, dev), _h(u, dev)
    y1 = torch.empty(n, dtype=torch.float16, device=dev)  # dg, du held above
    y2 = torch.empty(n, dtype=torch.float16, device=dev)
    L = _lib.lib()
    _lib.check(L.spk_silu_gate_f16(dg.data_ptr(), du.data_ptr(), y1.data_ptr(), n, _stream()), "silu")
    _lib.check(L.spk_residual_add_f16(dg.data_ptr(), du.data_ptr(), y2.data_ptr(), n, _stream()), "residual")
    torch.cuda.synchronize()
    e1, e2 = np.zeros(n, np.uint16), np.zeros(n, np.uint16)
    _om().orc_silu_gate(_p(g), _p(u), _p(e1), n)
    _om().orc_residual_add(_p(g), _p(u), _p(e2), n)
    assert np.array_equal(_u16(y1), e1)
    assert np.array_equal(_u16(y2), e2)


def test_embedding_rows(dev):
    from spock_amd import _lib
    V = 300
    E = _rand16(50, V * 1024, 0.02).reshape(V, 1024)
    ids = np.array([0, 299, 17, -1, 300, 17], np.int32)
    y = torch.empty(len(ids) * 1024, dtype=torch.float16, device=dev)
    dE, dids = _h(E, dev), torch.from_numpy(ids).to(dev)
    _lib.check(_lib.lib().spk_embedding_f16(dE.data_ptr(), dids.data_ptr(), len(ids), V, y.data_ptr(), _stream()),
               "spk_embedding_f16")
    torch.cuda.synchronize()
    got = _u16(y).reshape(len(ids), 1024)
    for i, t in enumerate(ids):
        assert np.array_equal(got[i], E[t] if 0 <= t < V else np.zeros(1024, np.uint16))


@pytest.mark.parametrize("T", [1, 5, 64, 133])
def test_deltanet_prefill_conv_bitexact(dev, oracle, T):
    from spock_amd import _lib
    print(f"[dn prefill conv T={T}]", flush=True)
    qkv = _rand16(60 + T, T * 6144).reshape(T, 6144)
    cs0 = _rand16(61, 6144 * 4)
    cw = _rand16(62, 6144 * 4, 0.3)
    dq, dcs, dcw = _h(qkv, dev), _h(cs0, dev), _h(cw, dev)
    hm = [torch.empty(16 * T * 128, dtype=torch.float16, device=dev) for _ in range(3)]
    _lib.check(_lib.lib().spk_deltanet_prefill_conv(dq.data_ptr(), 6144, dcs.data_ptr(), dcw.data_ptr(), T,
                                                    *[x.data_ptr() for x in hm], _stream()), "prefill conv")
    torch.cuda.synchronize()
    cs = cs0.copy()
    exp = np.zeros((T, 6144), np.uint16)
    for t in range(T):
        row = qkv[t].copy()
        oracle.lib().orc_conv_l2_qk(6144, 4, 2048, 16, _p(row), _p(cs), _p(cw))
        exp[t] = row
    assert np.array_equal(_u16(dcs), cs)
    for j, x in enumerate(hm):
        got = _u16(x).reshape(16, T, 128)
        want = exp[:, j * 2048:(j + 1) * 2048].reshape(T, 16, 128).transpose(1, 0, 2)
        assert np.array_equal(got, want), ["q", "k", "v"][j]


def test_deltanet_prefill_gbeta_and_norm_gate_bitexact(dev, oracle):
    from spock_amd import _lib
    T, layer = 37, 2
    a, b = _rand16(70, T * 16), _rand16(71, T * 16)
    alb = np.stack([np.linspace(-1, 1, 3 * 16, dtype=np.float32),
                    oracle.h2f(_rand16(72, 3 * 16, 0.1))], -1).astype(np.float32)
    g = torch.empty(16 * T, dtype=torch.float32, device=dev)
    beta = torch.empty(16 * T, dtype=torch.float32, device=dev)
    da, db, dalb = _h(a, dev), _h(b, dev), _f(alb, dev)  # held until the kernels have run
    _lib.check(_lib.lib().spk_deltanet_prefill_gbeta(da.data_ptr(), db.data_ptr(), 16, dalb.data_ptr(), layer, T,
                                                     g.data_ptr(), beta.data_ptr(), _stream()), "gbeta")
    core = np.random.default_rng(3).standard_normal((16, T, 128)).astype(np.float32)
    z = _rand16(73, T * 2048)
    nw = np.random.default_rng(4).uniform(0.5, 1.5, 128).astype(np.float32)
    out = torch.empty(T * 2048, dtype=torch.float16, device=dev)
    dcore, dz, dnw = _f(core, dev), _h(z, dev), _f(nw, dev)
    _lib.check(_lib.lib().spk_deltanet_norm_gate(dcore.data_ptr(), T, dz.data_ptr(), 2048, dnw.data_ptr(), 1e-6, T,
                                                 out.data_ptr(), 2048, _stream()), "norm gate")
    torch.cuda.synchronize()
    # g / beta: the decode shader's formula, one IEEE fp32 operation at a time
    av = oracle.h2f(a).reshape(T, 16).T
    bv = oracle.h2f(b).reshape(T, 16).T
    al = alb.reshape(3, 16, 2)[layer]
    f32 = np.float32
    sp = oracle.logf((f32(1.0) + oracle.expf((av + al[:, 1:2]).astype(f32))).astype(f32))
    eg = -oracle.expf(al[:, 0:1].astype(f32)) * sp
    eb = f32(1.0) / (f32(1.0) + oracle.expf(-bv))
    assert np.array_equal(g.cpu().numpy().reshape(16, T).view(np.uint32), eg.astype(f32).view(np.uint32))
    assert np.array_equal(beta.cpu().numpy().reshape(16, T).view(np.uint32), eb.astype(f32).view(np.uint32))
    # gated norm: 128-wide tree, fp16(w * o * r), then * silu(z)
    s = (core * core).astype(f32)
    for stride in (64, 32, 16, 8, 4, 2, 1):
        s = (s[..., :stride] + s[..., stride:2 * stride]).astype(f32)
    r = (f32(1.0) / np.sqrt((s[..., 0] / f32(128.0) + f32(1e-6)).astype(f32))).astype(f32)
    weighted = oracle.h2f(oracle.f2h((nw * (core * r[..., None]).astype(f32)).astype(f32)))
    zz = oracle.h2f(z).reshape(T, 16, 128).transpose(1, 0, 2)
    silu = (zz / (f32(1.0) + oracle.expf(-zz))).astype(f32)
    exp = oracle.f2h((weighted * silu).astype(f32)).transpose(1, 0, 2).reshape(-1)
    assert np.array_equal(_u16(out), exp)


@pytest.mark.parametrize("case", ["capture", "normal", "tiny", "large", "zero_rows"])
def test_deltanet_norm_gate_f16_bitexact(dev, oracle, case):
    """spk_deltanet_norm_gate_f16 (deltanet_norm_gate.comp, fp16 rows in
    place) against orc_norm_gate_f16: the reference capture's core / z (with
    the weight they imply; head 0 is fp16-subnormal there), random rows at
    three magnitudes (subnormal, unit, near the fp16 range whose squares
    stay finite in fp32), and heads that are exactly zero."""
    from conftest import GOLDEN
    from spock_amd import _lib
    f32 = np.float32
    nh = 16
    nw = np.random.default_rng(5).uniform(0.5, 1.5, 128).astype(f32)
    if case == "capture":
        d = GOLDEN / "ref_data"
        core = np.fromfile(d / "layer0_step1_dn_core_2048.fp16", np.uint16)
        z = np.fromfile(d / "layer0_step1_dn_z_2048.fp16", np.uint16)
    else:
        std = {"normal": 1.0, "tiny": 2e-6, "large": 3000.0, "zero_rows": 1.0}[case]
        core = _rand16(80, nh * 128, std)
        z = _rand16(81, nh * 128, 4.0)
        if case == "zero_rows":
            core.reshape(nh, 128)[::3] = 0
    io = _h(core, dev)
    dz, dnw = _h(z, dev), _f(nw, dev)
    _lib.check(_lib.lib().spk_deltanet_norm_gate_f16(io.data_ptr(), dz.data_ptr(), dnw.data_ptr(), nh, 128, 1e-6,
                                                     _stream()), "norm gate f16")
    torch.cuda.synchronize()
    assert np.array_equal(_u16(io), oracle.norm_gate_f16(core, z, nw))


@pytest.mark.parametrize("M,N,K,res", [(512, 6144, 1024, False), (37, 16, 1024, False), (100, 1000, 64, True),
                                       (70, 1024, 3584, True), (512, 1024, 2048, True), (512, 3584, 1024, False),
                                       (33, 40, 96, True), (300, 6000, 96, False), (512, 2048, 1024, True),
                                       (2048, 4096, 64, False)])
def test_gemm_f16_against_fp64(dev, M, N, K, res):
    from spock_amd import _lib
    print(f"[gemm {M}x{N}x{K}]", flush=True)
    A = _rand16(80, M * K).reshape(M, K)
    W = _rand16(81, N * K, 0.02).reshape(N, K)
    R = _rand16(82, M * N)
    dA, dW = _h(A, dev), _h(W, dev)
    C_ = _h(R, dev) if res else torch.empty(M * N, dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().spk_gemm_f16(dA.data_ptr(), K, dW.data_ptr(), K, C_.data_ptr(), N,
                                       C_.data_ptr() if res else None, M, N, K, _stream()), "spk_gemm_f16")
    torch.cuda.synchronize()
    a64 = A.view(np.float16).astype(np.float64)
    w64 = W.view(np.float16).astype(np.float64)
    dot = a64 @ w64.T
    # fp32 accumulation in any order: |acc - dot| <= K 2^-24 sum|a w|; then one
    # fp16 rounding of the product and, with a residual, one of the sum
    bound = K * 2.0 ** -24 * (np.abs(a64) @ np.abs(w64).T)
    ulp = lambda v: 2.0 ** (np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** -14))) - 10)
    r16 = lambda v: v.astype(np.float16).astype(np.float64)
    got = _u16(C_).reshape(M, N).view(np.float16).astype(np.float64)
    want = r16(dot)
    tol = bound + ulp(dot)
    if res:
        r = R.view(np.float16).reshape(M, N).astype(np.float64)
        want = r16(r + want)
        tol = tol + ulp(r + dot)
    assert np.all(np.abs(got - (r + dot if res else dot)) <= tol), "outside the accumulation error bound"
    # and the typical element equals the correctly rounded value
    assert np.mean(got == want) > 0.95


@pytest.mark.parametrize("rows,out_dim,in_dim,res", [(1, 6144, 1024, False), (70, 1000, 2048, True),
                                                     (133, 16, 1024, False), (65, 1024, 3584, True),
                                                     (200, 6144, 1024, True), (300, 2600, 1024, False),
                                                     (300, 1000, 2048, False), (260, 1024, 3584, True)])
def test_matvec_rows_bitexact(dev, rows, out_dim, in_dim, res):
    """spk_matvec_f16_rows: each row bit-identical to the decode matvec order."""
    from spock_amd import _lib
    print(f"[matvec rows {rows}x{out_dim}x{in_dim}]", flush=True)
    W = _rand16(90, out_dim * in_dim, 0.02).reshape(out_dim, in_dim)
    X = _rand16(91, rows * in_dim).reshape(rows, in_dim)
    R = _rand16(92, rows * out_dim).reshape(rows, out_dim)
    dW, dX = _h(W, dev), _h(X, dev)
    Y = _h(R, dev) if res else torch.empty(rows * out_dim, dtype=torch.float16, device=dev)
    _lib.check(_lib.lib().spk_matvec_f16_rows(dW.data_ptr(), dX.data_ptr(), in_dim, Y.data_ptr(), out_dim,
                                              Y.data_ptr() if res else None, rows, out_dim, in_dim, _stream()),
               "spk_matvec_f16_rows")
    torch.cuda.synchronize()
    exp = np.zeros((rows, out_dim), np.uint16)
    _om().orc_matmul_rows(_p(W), _p(X), _p(exp), out_dim, in_dim, rows)
    if res:
        e2 = np.zeros_like(exp)
        _om().orc_residual_add(_p(R), _p(exp), _p(e2), exp.size)
        exp = e2
    assert np.array_equal(_u16(Y).reshape(rows, out_dim), exp)


@pytest.mark.parametrize("T,f16,l2,init", [(104, False, False, False), (64, True, False, True),
                                          (1, False, True, True), (200, True, False, True),
                                          (520, True, True, True)])
def test_chunk_prefill_ordered_bitexact(dev, oracle, T, f16, l2, init):
    """spk_chunk_prefill_ordered: run_deltanet_chunk_rule's loops with the
    deterministic exp, bit-identical to orc_chunk_rule_det."""
    import ctypes as C_
    from spock_amd import _lib, synth
    print(f"[ordered chunk T={T} f16={f16} l2={l2} init={init}]", flush=True)
    H = 16
    inp = synth.chunk_inputs(H, T, seed=T, l2=not l2)
    if f16:
        for n in ("q", "k", "v"):
            inp[n] = inp[n].astype(np.float16).astype(np.float32)
    st0 = (np.random.default_rng(T).standard_normal((H, 128, 128)) * 0.05).astype(np.float32) if init else None
    L = oracle.lib()
    L.orc_chunk_rule_det.restype = C_.c_int
    L.orc_chunk_rule_det.argtypes = [C_.c_size_t] * 5 + [C_.c_int] + [C_.c_void_p] * 8
    ec = np.zeros((H, T, 128), np.float32)
    es = np.zeros((H, 128, 128), np.float32)
    rc = L.orc_chunk_rule_det(H, T, 128, 128, 64, 1 if l2 else 0, _p(inp["q"]), _p(inp["k"]), _p(inp["v"]),
                              _p(inp["g"]), _p(inp["beta"]), None if st0 is None else _p(st0), _p(ec), _p(es))
    assert rc == 0
    cvt = (lambda a: _h(a.astype(np.float16).view(np.uint16), dev)) if f16 else (lambda a: _f(a, dev))
    dq, dk, dv = cvt(inp["q"]), cvt(inp["k"]), cvt(inp["v"])
    dg, db = _f(inp["g"], dev), _f(inp["beta"], dev)
    dinit = _f(st0, dev) if init else None
    core = torch.empty(H * T * 128, dtype=torch.float32, device=dev)
    state = torch.empty(H * 128 * 128, dtype=torch.float32, device=dev)
    wsb = int(_lib.lib().spk_chunk_prefill_ordered_workspace_size(H, T))
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    a = _lib.SpkChunkArgs()
    a.num_heads, a.total_tokens, a.key_dim, a.value_dim, a.chunk_size = H, T, 128, 128, 64
    a.use_qk_l2norm, a.q_scale, a.input_dtype = 1 if l2 else 0, 0.0, _lib.SPK_F16 if f16 else _lib.SPK_F32
    a.q, a.k, a.v, a.g, a.beta = dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dg.data_ptr(), db.data_ptr()
    a.initial_state = dinit.data_ptr() if init else None
    a.out_core, a.out_state, a.num_seqs = core.data_ptr(), state.data_ptr(), 1
    a.workspace, a.workspace_bytes = ws.data_ptr(), wsb
    _lib.check(_lib.lib().spk_chunk_prefill_ordered(C.byref(a), _stream()), "spk_chunk_prefill_ordered")
    torch.cuda.synchronize()
    assert np.array_equal(core.cpu().numpy().view(np.uint32), ec.reshape(-1).view(np.uint32))
    assert np.array_equal(state.cpu().numpy().view(np.uint32), es.reshape(-1).view(np.uint32))


def test_gemv_silu_pair_bitexact(dev):
    """gate/up projections with silu_gate.comp fused: fp16(silu(fp16(Wg.x)) * fp16(Wu.x))."""
    from spock_amd import _lib
    n = 3584
    h = _rand16(95, 1024)
    w = _rand16(96, 1024, 0.02)
    Wg = _rand16(97, n * 1024, 0.02).reshape(n, 1024)
    Wu = _rand16(98, n * 1024, 0.02).reshape(n, 1024)
    dh, dw, dWg, dWu = _h(h, dev), _h(w, dev), _h(Wg, dev), _h(Wu, dev)
    y = torch.empty(n, dtype=torch.float16, device=dev)
    inp = _lib.SpkGemvInput()
    inp.kind, inp.in_dim, inp.x, inp.x2 = _lib.SPK_GEMV_IN_RMSNORM, 1024, dh.data_ptr(), dw.data_ptr()
    arr = (_lib.SpkGemvOutput * 1)()
    arr[0].W, arr[0].y, arr[0].out_dim, arr[0].W_up = dWg.data_ptr(), y.data_ptr(), n, dWu.data_ptr()
    _lib.check(_lib.lib().spk_gemv_fused(C.byref(inp), arr, 1, _stream()), "spk_gemv_fused pair")
    torch.cuda.synchronize()
    xn = np.zeros(1024, np.uint16)
    _om().orc_rmsnorm1024(_p(h), _p(w), _p(xn))
    g, u = _orc_matvec(Wg, xn), _orc_matvec(Wu, xn)
    exp = np.zeros(n, np.uint16)
    _om().orc_silu_gate(_p(g), _p(u), _p(exp), n)
    assert np.array_equal(_u16(y), exp)


@pytest.mark.parametrize("pos", [0, 5, 64, 700, 1023, 1024, 2047, 2048, 3000, 4095])
def test_attention_decode_oproj_equals_two_step(dev, pos):
    """spk_attention_decode_oproj (blocks, then o_proj + residual with the
    blocks' combine and sigmoid gate in its prologue) gives the bits of
    spk_attention_decode followed by spk_gemv_fused over its output; past
    1024 positions the prologue loads partials beyond its prefetch, past 2048
    it runs more than one chunk of 32 blocks."""
    from spock_amd import _lib
    print(f"[attention decode + o_proj pos={pos}]", flush=True)
    L = _lib.lib()
    max_seq = 4096
    rope, kv, qg, k, v, qn, kn = _attn_inputs(300 + pos, max_seq, pos)
    Wo = _rand16(77, 1024 * 2048, 0.02)
    res = _rand16(78, 1024)
    dWo = _h(Wo, dev)
    outs = []
    for fused in (False, True):
        a, d = _attn_args(dev, rope, kv, qg, k, v, qn, kn, max_seq, 1, max_seq)
        dpos = torch.tensor([pos], dtype=torch.int32, device=dev)
        a.pos_dev = dpos.data_ptr()
        y = _h(res, dev)
        o = _lib.SpkGemvOutput()
        o.W, o.y, o.residual, o.out_dim, o.W_up = dWo.data_ptr(), y.data_ptr(), y.data_ptr(), 1024, None
        if fused:
            _lib.check(L.spk_attention_decode_oproj(C.byref(a), C.byref(o), _stream()), "spk_attention_decode_oproj")
        else:
            _lib.check(L.spk_attention_decode(C.byref(a), _stream()), "spk_attention_decode")
            gi = _lib.SpkGemvInput()
            gi.kind, gi.in_dim, gi.x = _lib.SPK_GEMV_IN_PLAIN, 2048, d["out"].data_ptr()
            _lib.check(L.spk_gemv_fused(C.byref(gi), C.byref(o), 1, _stream()), "spk_gemv_fused")
        torch.cuda.synchronize()
        outs.append((_u16(y), _u16(d["kv"])))
    assert np.array_equal(outs[1][1], outs[0][1])
    assert np.array_equal(outs[1][0], outs[0][0])
