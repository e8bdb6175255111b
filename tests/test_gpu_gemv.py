"""GPU parity of the decode GEMVs, lm_head and argmax against the oracle.

Bar: bit-exact fp16 outputs and argmax indices (the oracle restates
lm_head_tiled.comp's, matvec_tiled.comp's and matvec.comp's summation orders
and argmax.comp's tie rule)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

CHAIN = [(6144, 1024), (2048, 1024), (1024, 2048), (3584, 1024), (3584, 1024), (1024, 3584)]


def _t(dev, a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.float16)).to(dev)


@pytest.mark.parametrize("out_dim,in_dim", CHAIN + [(16, 1024), (7, 64), (300, 192), (40000, 512)])
def test_matvec_bitexact(dev, oracle, out_dim, in_dim):
    from spock_amd import ops, synth
    W = synth.gemv_weights(out_dim, in_dim, seed=out_dim * 7 + in_dim)
    x = synth.gemv_input(in_dim, seed=in_dim)
    y = ops.matvec_f16(_t(dev, W), _t(dev, x))
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16(W, x))


@pytest.mark.parametrize("order", ["strided", "serial", "spans"])
@pytest.mark.parametrize("out_dim,in_dim", CHAIN[:3] + [(1024, 3584), (7, 64), (300, 192), (37, 200),
                                                         (260, 1000), (5, 1), (40000, 512)])
def test_matvec_order_bitexact(dev, oracle, order, out_dim, in_dim):
    if order == "spans" and in_dim % 64:
        pytest.skip("lm_head_tiled.comp's order needs in_dim % 64 == 0")
    from spock_amd import ops, synth
    W = synth.gemv_weights(out_dim, in_dim, seed=out_dim * 5 + in_dim)
    x = synth.gemv_input(in_dim, seed=in_dim + 1)
    y = ops.matvec_f16_order(_t(dev, W), _t(dev, x), order)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16_order(W, x, order))


@pytest.mark.parametrize("order", ["strided", "serial", "spans"])
def test_matvec_order_lm_head_size(dev, oracle, order):
    """508.6 MB: above 128 MB the spans and strided orders stream their rows
    with non-temporal loads (spans: dense loads regrouped through LDS)."""
    from spock_amd import ops, synth
    V, Hd = 248320, 1024
    W = synth.gemv_weights(V, Hd, seed=41)
    x = synth.gemv_input(Hd, seed=42)
    y = ops.matvec_f16_order(_t(dev, W), _t(dev, x), order)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16_order(W, x, order))


@pytest.mark.parametrize("order", ["spans", "strided", "serial"])
@pytest.mark.parametrize("out_dim,in_dim", [(131072, 512), (16384, 4096)])
def test_matvec_order_128mb_edges(dev, oracle, order, out_dim, in_dim):
    """128 MB, the smallest size on the streaming paths, at one and eight
    16-byte pieces per lane of the span order (in_dim 512 and 4096)."""
    from spock_amd import ops, synth
    W = synth.gemv_weights(out_dim, in_dim, seed=in_dim + 7)
    x = synth.gemv_input(in_dim, seed=in_dim + 8)
    y = ops.matvec_f16_order(_t(dev, W), _t(dev, x), order)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16_order(W, x, order))


def test_matvec_order_unaligned_and_cancellation(dev, oracle):
    """x and W 2-byte offset (the serial order's generic kernel), and rows
    that only one summation order sums exactly."""
    from spock_amd import ops, synth
    from test_oracle_decode_gemv import _cancel_rows
    W = synth.gemv_weights(70, 1024, seed=3)
    x = synth.gemv_input(1024, seed=4)
    Wb = torch.empty(70 * 1024 + 1, dtype=torch.float16, device=dev)
    xb = torch.empty(1024 + 1, dtype=torch.float16, device=dev)
    Wb[1:] = _t(dev, W.reshape(-1))
    xb[1:] = _t(dev, x)
    for order in ("strided", "serial"):
        y = ops.matvec_f16_order(Wb[1:].view(70, 1024), xb[1:], order)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16_order(W, x, order))
    for in_dim in (256, 200, 1024):
        rows = _cancel_rows(in_dim)
        Wc = np.stack([w.astype(np.float16) for w in rows.values()]).view(np.uint16)
        xc = np.full(in_dim, np.float16(1.0)).view(np.uint16)
        for order in rows:
            y = ops.matvec_f16_order(_t(dev, Wc), _t(dev, xc), order)
            torch.cuda.synchronize()
            assert np.array_equal(y.cpu().numpy().view(np.uint16), oracle.matvec_f16_order(Wc, xc, order))


def test_matvec_batched_equals_single(dev):
    from spock_amd import ops, synth
    items, singles = [], []
    for i, (o, n) in enumerate(CHAIN):
        W = _t(dev, synth.gemv_weights(o, n, seed=i))
        x = _t(dev, synth.gemv_input(n, seed=50 + i))
        items.append((W, x, torch.empty(o, dtype=torch.float16, device=dev)))
        singles.append(ops.matvec_f16(W, x))
    ops.matvec_f16_batched(items)
    torch.cuda.synchronize()
    for (_, _, y), s in zip(items, singles):
        assert torch.equal(y, s)


def test_lm_head_argmax_config3(dev, oracle):
    from spock_amd import ops, synth
    V, Hd = 248320, 1024
    W = synth.gemv_weights(V, Hd, seed=31)
    x = synth.gemv_input(Hd, seed=32)
    logits = torch.empty(V, dtype=torch.float16, device=dev)
    idx = ops.lm_head_argmax(_t(dev, W), _t(dev, x), logits=logits)
    torch.cuda.synchronize()
    e_idx, e_logits = oracle.lm_head_argmax(W, x)
    assert np.array_equal(logits.cpu().numpy().view(np.uint16), e_logits)
    assert int(idx.cpu()[0]) == e_idx
    # without the logits buffer
    idx2 = ops.lm_head_argmax(_t(dev, W), _t(dev, x))
    torch.cuda.synchronize()
    assert int(idx2.cpu()[0]) == e_idx


def _tie_patterns():
    n = 248320
    E = (n + 255) // 256
    pats = []
    v = np.zeros(n, np.float16)
    v[[E * 64, E * 128]] = 3.0  # argmax.comp's tree keeps lane 128's (bit-reversed order)
    pats.append(v)
    v = np.full(n, -1.0, np.float16)
    v[[5, 6, E * 3 + 1]] = 2.0
    pats.append(v)
    v = np.full(n, np.nan, np.float16)
    pats.append(v)
    v = np.full(n, -np.inf, np.float16)
    v[77777] = -65504.0
    pats.append(v)
    v = np.zeros(n, np.float16)
    v[::2] = -0.0
    pats.append(v)
    rng = np.random.default_rng(0)
    v = rng.integers(-3, 4, n).astype(np.float16)  # many ties
    pats.append(v)
    v = np.zeros(1000, np.float16)
    v[[3, 999]] = 1.0
    pats.append(v)
    return pats


@pytest.mark.parametrize("i", range(7))
def test_argmax_tie_rule(dev, oracle, i):
    from spock_amd import ops
    v = _tie_patterns()[i]
    out = ops.argmax_f16(_t(dev, v.view(np.uint16)))
    torch.cuda.synchronize()
    assert int(out.cpu()[0]) == oracle.argmax_f16(v.view(np.uint16))


def _key_path(dev, W, x, norm_w=None, logits=None, one=False):
    """Through the C ABI: spk_lm_head_argmax_key + spk_argmax_key_take, or
    (one=True) spk_lm_head_argmax_take, the same in one launch."""
    from spock_amd import _lib
    lib = _lib.lib()
    s = torch.cuda.current_stream().cuda_stream
    vocab, hidden = W.shape
    idx = torch.full((1,), -1, dtype=torch.int32, device=dev)
    nw = None if norm_w is None else norm_w.data_ptr()
    lg = None if logits is None else logits.data_ptr()
    if one:
        n = lib.spk_lm_head_take_slots(vocab)
        key = torch.zeros(n, dtype=torch.int64, device=dev)
        rc = lib.spk_lm_head_argmax_take(W.data_ptr(), x.data_ptr(), nw, vocab, hidden, lg, key.data_ptr(), n,
                                         idx.data_ptr(), None, None, None, 0, s)
        _lib.check(rc, "spk_lm_head_argmax_take")
    else:
        key = torch.zeros(64, dtype=torch.int64, device=dev)  # SPK_ARGMAX_KEY_WORDS
        rc = lib.spk_lm_head_argmax_key(W.data_ptr(), x.data_ptr(), nw, vocab, hidden, lg, key.data_ptr(), s)
        _lib.check(rc, "spk_lm_head_argmax_key")
        _lib.check(lib.spk_argmax_key_take(key.data_ptr(), vocab, idx.data_ptr(), None, None, None, 0, s),
                   "spk_argmax_key_take")
    torch.cuda.synchronize()
    assert not key.cpu().numpy().any()  # the take leaves the key words / slots at zero
    return int(idx.cpu()[0])


@pytest.mark.parametrize("one", [False, True])
@pytest.mark.parametrize("norm", [False, True])
def test_lm_head_argmax_key_config3(dev, oracle, norm, one):
    """Final norm + lm_head + argmax (device atomic max of the argmax keys,
    then the take; or one launch whose last workgroup takes the per-workgroup
    key slots) against the oracle: bit-exact logits and index."""
    import oracle_model
    from spock_amd import synth
    V, Hd = 248320, 1024
    W = synth.gemv_weights(V, Hd, seed=41)
    h = synth.gemv_input(Hd, seed=42)
    x = h
    nw = None
    if norm:
        nw = synth.f16(synth.normal(43, Hd, std=0.02))
        x = np.empty(Hd, np.uint16)
        oracle_model.lib().orc_rmsnorm1024(h.ctypes.data, nw.ctypes.data, x.ctypes.data)
    e_idx, e_logits = oracle.lm_head_argmax(W, x)
    logits = torch.empty(V, dtype=torch.float16, device=dev)
    Wd = _t(dev, W)
    got = _key_path(dev, Wd, _t(dev, h), None if nw is None else _t(dev, nw), logits, one=one)
    assert np.array_equal(logits.cpu().numpy().view(np.uint16), e_logits)
    assert got == e_idx
    # again without logits (the key words were returned to zero by the take)
    assert _key_path(dev, Wd, _t(dev, h), None if nw is None else _t(dev, nw), one=one) == e_idx


@pytest.mark.parametrize("one", [False, True])
@pytest.mark.parametrize("vocab,hidden", [(1000, 512), (77777, 2048), (4096, 1024), (1, 512), (33, 4096)])
def test_lm_head_argmax_key_ties(dev, oracle, vocab, hidden, one):
    """Rows repeated across the vocabulary make exact logit ties; the key path
    keeps argmax.comp's tie rule (same index as the oracle)."""
    from spock_amd import synth
    base = synth.gemv_weights(37, hidden, seed=vocab)
    W = np.ascontiguousarray(base[np.arange(vocab) % 37])
    x = synth.gemv_input(hidden, seed=hidden)
    e_idx, _ = oracle.lm_head_argmax(W, x)
    assert _key_path(dev, _t(dev, W), _t(dev, x), one=one) == e_idx


def test_lm_head_argmax_take_bookkeeping_and_invalid_rows(dev, oracle):
    """The one-launch form records the token as spk_argmax_key_take does
    (history[count] = index, count += 1, pos += 1; no history write once count
    reaches the capacity), over several calls in a row on one slot array; rows
    whose logits are -inf or NaN never win, and a whole workgroup of them
    still fills its slot."""
    from spock_amd import _lib, synth
    lib = _lib.lib()
    s = torch.cuda.current_stream().cuda_stream
    V, Hd = 5000, 1024
    W = synth.gemv_weights(V, Hd, seed=7)
    W[:600] = np.float16(np.nan).view(np.uint16)  # rows 0..599: NaN logits (whole workgroups)
    W[600:700] = np.float16(-np.inf).view(np.uint16)
    x = synth.gemv_input(Hd, seed=8)
    Wd, xd = _t(dev, W), _t(dev, x)
    n = lib.spk_lm_head_take_slots(V)
    slots = torch.zeros(n, dtype=torch.int64, device=dev)
    idx = torch.full((1,), -1, dtype=torch.int32, device=dev)
    pos = torch.tensor([10], dtype=torch.int32, device=dev)
    hist = torch.full((1 + 3,), -7, dtype=torch.int32, device=dev)  # [count | history of capacity 3]
    hist[0] = 0
    e_idx, _ = oracle.lm_head_argmax(W, x)
    assert e_idx >= 700
    for call in range(5):
        _lib.check(lib.spk_lm_head_argmax_take(Wd.data_ptr(), xd.data_ptr(), None, V, Hd, None, slots.data_ptr(), n,
                                               idx.data_ptr(), pos.data_ptr(), hist.data_ptr(),
                                               hist[1:].data_ptr(), 3, s), "spk_lm_head_argmax_take")
        torch.cuda.synchronize()
        assert int(idx.cpu()[0]) == e_idx
        assert not slots.cpu().numpy().any()
    assert int(pos.cpu()[0]) == 15
    h = hist.cpu().numpy()
    assert h[0] == 5 and list(h[1:]) == [e_idx] * 3
    # too few slot words is an argument error, before any launch
    assert lib.spk_lm_head_argmax_take(Wd.data_ptr(), xd.data_ptr(), None, V, Hd, None, slots.data_ptr(), n - 1,
                                       idx.data_ptr(), None, None, None, 0, s) == -5
