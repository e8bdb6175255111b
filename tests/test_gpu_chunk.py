"""GPU parity of the chunk prefill (spk_chunk_prefill) against the oracle.

Tolerance (north star): fp32 core_attn_out and final_state within a max
relative error of 1e-5, measured as |gpu - cpu| / max(1, |cpu|) like the
reference probes (apps/spock-deltanet-chunk-prefill-tiled-probe.cpp:286).
"""
import json

import numpy as np
import pytest
import torch

import chunk_cases
from conftest import GOLDEN, max_rel

pytestmark = pytest.mark.gpu
TOL = 1e-5


def _to(dev, a, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype)


def _run(dev, inp, init=None, cu=None, l2=False, half=False):
    from spock_amd import ops
    dt = torch.float16 if half else torch.float32
    q, k, v = (_to(dev, inp[n], dt) for n in ("q", "k", "v"))
    g, b = _to(dev, inp["g"]), _to(dev, inp["beta"])
    st = None if init is None else _to(dev, init)
    core, state = ops.chunk_prefill(q, k, v, g, b, initial_state=st, cu_seqlens=cu, use_qk_l2norm=l2)
    torch.cuda.synchronize()
    return core.cpu().numpy(), state.cpu().numpy()


# Keys outside the runtime's domain (not L2-normalised, |k|^2 ~ 43): the WY
# solve is ill-conditioned and the reference algorithm itself is ~9e-5 from
# the exact (fp64) answer, so fp32 results of any summation order differ at
# that level.  There the bar is accuracy against fp64: the GPU must be at
# least as close to the exact result as the reference algorithm is.
ILL_CONDITIONED = {"runtime-range-padded"}


@pytest.mark.parametrize("name", sorted(json.loads((GOLDEN / "chunk_cases.json").read_text())))
def test_chunk_cases(dev, oracle, name):
    print(f"[chunk case {name}]", flush=True)
    inp = chunk_cases.make_inputs(name)
    spec = chunk_cases.CASES[name]
    cc, cs = oracle.chunk_rule(**inp, chunk=spec["C"])
    gc, gs = _run(dev, inp)
    if name in ILL_CONDITIONED:
        c64, s64 = oracle.delta_recurrence_f64(**inp)
        assert max_rel(gc, c64) <= max_rel(cc, c64) * 1.25
        assert max_rel(gs[0], s64) <= max_rel(cs, s64) * 1.25
        return
    assert max_rel(gc, cc) <= TOL
    assert max_rel(gs[0], cs) <= TOL


def test_reference_unit_case_with_init_and_l2(dev, oracle):
    """The reference unit test's shape (H=2,T=5,dk=3,dv=2) zero-padded to the
    kernel's 128-wide heads: zero key dims do not change dot products or
    norms, zero value dims give zero outputs; q_scale keeps 1/sqrt(3)."""
    from spock_amd import ops
    z = np.load(GOLDEN / "chunk_unit_case.npz")
    H, T, dk, dv = (int(x) for x in z["meta"][:4])
    pad = lambda a, w: np.pad(a, [(0, 0)] * (a.ndim - 1) + [(0, w - a.shape[-1])])
    q, k, v = pad(z["q"], 128), pad(z["k"], 128), pad(z["v"], 128)
    init = np.zeros((H, 128, 128), np.float32)
    init[:, :dk, :dv] = z["init"]
    core, state = ops.chunk_prefill(_to(dev, q), _to(dev, k), _to(dev, v), _to(dev, z["g"]),
                                    _to(dev, z["beta"]), initial_state=_to(dev, init),
                                    use_qk_l2norm=True, q_scale=float(np.float32(1) / np.sqrt(np.float32(3))))
    torch.cuda.synchronize()
    core = core.cpu().numpy()
    state = state.cpu().numpy()[0]
    assert np.abs(core[:, :, :dv] - z["core"]).max() <= TOL
    assert np.abs(state[:, :dk, :dv] - z["state"]).max() <= TOL
    assert not core[:, :, dv:].any() and not state[:, dk:, :].any() and not state[:, :, dv:].any()


@pytest.mark.parametrize("T", [1, 63, 64, 65, 104, 257])
@pytest.mark.parametrize("l2,init,half", [(False, False, False), (True, True, False),
                                          (False, True, True), (True, False, True)])
def test_single_sequence(dev, oracle, T, l2, init, half):
    from spock_amd import synth
    inp = synth.chunk_inputs(16, T, seed=T, l2=not l2)
    if half:  # fp16 q/k/v inputs; the oracle sees the same rounded values
        for n in ("q", "k", "v"):
            inp[n] = inp[n].astype(np.float16).astype(np.float32)
    st0 = np.random.default_rng(T).normal(0, 0.05, (16, 128, 128)).astype(np.float32) if init else None
    cc, cs = oracle.chunk_rule(**inp, init=st0, l2=l2)
    gc, gs = _run(dev, inp, init=st0, l2=l2, half=half)
    assert max_rel(gc, cc) <= TOL
    assert max_rel(gs[0], cs) <= TOL


def test_varlen_ragged_with_empty(dev, oracle):
    from spock_amd import synth
    lens = [5, 0, 64, 130, 1, 200]
    cu = synth.cu_seqlens_from(lens)
    inp = synth.chunk_inputs(16, int(cu[-1]), seed=21)
    init = np.random.default_rng(3).normal(0, 0.05, (len(lens), 16, 128, 128)).astype(np.float32)
    cc, cs = oracle.chunk_rule_varlen(**inp, cu=cu, init=init)
    gc, gs = _run(dev, inp, init=init, cu=cu)
    assert max_rel(gc, cc) <= TOL
    assert max_rel(gs, cs) <= TOL
    assert np.array_equal(gs[1], init[1])  # empty sequence: state passes through


def test_reference_output_buffer_layout(dev, oracle):
    """One buffer [H*total_seq*dv | H*dk*dv] as gpu_chunk_prefill_from_gpu_collect
    binds it (vk_session.cpp:4507-4573): core rows strided by total_seq."""
    from spock_amd import ops, synth
    H, T, total = 16, 104, 128
    inp = synth.chunk_inputs(H, T, seed=4)
    buf = torch.full((H * total * 128 + H * 128 * 128,), float("nan"), device=dev)
    core = buf[:H * total * 128].view(H, total, 128)
    state = buf[H * total * 128:].view(1, H, 128, 128)
    ops.chunk_prefill(*(_to(dev, inp[n]) for n in ("q", "k", "v", "g", "beta")), out_core=core,
                      out_state=state, core_head_stride=total)
    torch.cuda.synchronize()
    cc, cs = oracle.chunk_rule(**inp)
    got = buf.cpu().numpy()
    gcore = got[:H * total * 128].reshape(H, total, 128)
    assert max_rel(gcore[:, :T], cc) <= TOL
    assert np.isnan(gcore[:, T:]).all()  # padding rows untouched
    assert max_rel(got[H * total * 128:].reshape(H, 128, 128), cs) <= TOL


def _trunc16(x):
    """fp32 -> fp16 bits rounded toward zero with flush to zero, formed from
    numpy's round-to-nearest cast: where the nearest fp16 lies above |x|,
    step one ulp toward zero; |x| below fp16's smallest normal gives +-0 and
    |x| >= 2^16 gives +-inf (the reference's float_to_half,
    vk_session.cpp:69-89).  Finite inputs only."""
    x = np.asarray(x, np.float32)
    with np.errstate(over="ignore"):
        h = x.astype(np.float16).view(np.uint16).astype(np.int32)
    above = np.abs(h.astype(np.uint16).view(np.float16).astype(np.float64)) > np.abs(x.astype(np.float64))
    h = np.where(above & ((h & 0x7FFF) != 0), h - 1, h)
    sign = (x.view(np.uint32) >> 16).astype(np.int32) & 0x8000
    h = np.where(np.abs(x) < np.float32(2.0 ** -14), sign, h)
    h = np.where(np.abs(x) >= np.float32(65536.0), sign | 0x7C00, h)
    return h.astype(np.uint16)


def _oracle_pack_threads(oracle, inp, cu):
    """The oracle's chunk rule for every (sequence, head) of a pack, split
    over the host's threads (ctypes releases the GIL during each call)."""
    import os
    from concurrent.futures import ThreadPoolExecutor
    S = len(cu) - 1
    H = inp["q"].shape[0]
    jobs = [(s, h) for s in range(S) for h in range(H)]

    def one(job):
        s, h = job
        t0, t1 = int(cu[s]), int(cu[s + 1])
        sub = {n: np.ascontiguousarray(a[h:h + 1, t0:t1]) for n, a in inp.items()}
        return oracle.chunk_rule(**sub)

    try:
        nt = len(os.sched_getaffinity(0))
    except AttributeError:
        nt = os.cpu_count() or 1
    with ThreadPoolExecutor(max(1, min(16, nt))) as ex:
        res = list(ex.map(one, jobs))
    core = np.empty((H, int(cu[-1]), 128), np.float32)
    state = np.empty((S, H, 128, 128), np.float32)
    for (s, h), (c, st) in zip(jobs, res):
        core[h, int(cu[s]):int(cu[s + 1])] = c[0]
        state[s, h] = st[0]
    return core, state


def test_config2_full_size_against_oracle(dev, oracle):
    """Config 2 at full size (8 sequences, lengths U[512, 8192], fp16 q/k/v,
    34,878 tokens): every sequence of the packed call, the 124-chunk one
    included, against the oracle's chunk rule (deltanet_chunk.cpp:53-284) run
    per (sequence, head), to the north-star bar on the floored metric; the
    pure relative error |g - c| / |c| is reported beside it.  The packed
    result also equals the single-sequence call bit for bit (shortest and
    longest), and the last-token fp16 hand-off of every sequence equals the
    truncated last row (deltanet_chunk_last_to_fp16.comp:70-76)."""
    from spock_amd import ops, synth
    lens = synth.ragged_lengths(8, 512, 8192, seed=2024)
    cu = synth.cu_seqlens_from(lens)
    N = int(cu[-1])
    inp = synth.chunk_inputs(16, N, seed=2)
    for n in ("q", "k", "v"):
        inp[n] = inp[n].astype(np.float16).astype(np.float32)
    dt = torch.float16
    q, k, v = (_to(dev, inp[n], dt) for n in ("q", "k", "v"))
    core_d, state_d = ops.chunk_prefill(q, k, v, _to(dev, inp["g"]), _to(dev, inp["beta"]), cu_seqlens=cu)
    torch.cuda.synchronize()
    gc, gs = core_d.cpu().numpy(), state_d.cpu().numpy()
    assert np.isfinite(gc).all() and np.isfinite(gs).all()
    print(f"[config 2 oracle: lens {list(map(int, lens))}]", flush=True)
    cc, cs = _oracle_pack_threads(oracle, inp, cu)
    for s in range(len(lens)):
        t0, t1 = int(cu[s]), int(cu[s + 1])
        ec, es = max_rel(gc[:, t0:t1], cc[:, t0:t1]), max_rel(gs[s], cs[s])
        a, b = gc[:, t0:t1].astype(np.float64), cc[:, t0:t1].astype(np.float64)
        nz = b != 0
        pure_c = float(np.max(np.abs(a - b)[nz] / np.abs(b)[nz]))
        nzs = cs[s] != 0
        pure_s = float(np.max(np.abs(gs[s].astype(np.float64) - cs[s])[nzs] / np.abs(cs[s].astype(np.float64))[nzs]))
        print(f"  seq {s} len {t1 - t0} ({(t1 - t0 + 63) // 64} chunks): floored core {ec:.2e} state {es:.2e}; "
              f"pure relative core {pure_c:.2e} state {pure_s:.2e}", flush=True)
        assert ec <= TOL and es <= TOL, (s, ec, es)
        # last-token hand-off: row (h*N + t1 - 1) of every head
        last = ops.chunk_last_to_fp16(core_d, seq_len=t1, total_seq=N)
        torch.cuda.synchronize()
        assert np.array_equal(last.cpu().numpy().view(np.uint16), _trunc16(gc[:, t1 - 1, :]).reshape(-1)), s
    order = np.argsort(lens)
    for s in (order[0], order[-1]):
        t0, L = int(cu[s]), int(lens[s])
        sub = {k_: v_[:, t0:t0 + L] for k_, v_ in inp.items()}
        c1, s1 = _run(dev, sub, half=True)
        assert np.array_equal(c1, gc[:, t0:t0 + L]) and np.array_equal(s1[0], gs[s])


@pytest.mark.parametrize("half", [False, True])
def test_small_launch_paths_equal_packed(dev, half):
    """Alone, a 104-token sequence (2 chunks x 16 heads) runs the intra kernel
    as 8 workgroups per (chunk, head), a 192-token one (3 chunks) as 4 and a
    300-token one (5 chunks) as 2; the scan runs two workgroups per CU and
    skips the first chunk's S products (no initial state).  Packed with longer
    sequences the same sequences run one workgroup per (chunk, head) and, for
    fp16, the three-per-CU scan.  Every output must be the same bits."""
    from spock_amd import synth
    lens = np.array([104, 192, 300, 300, 4096])
    cu = synth.cu_seqlens_from(lens)
    inp = synth.chunk_inputs(16, int(cu[-1]), seed=11)
    if half:
        for n in ("q", "k", "v"):
            inp[n] = inp[n].astype(np.float16).astype(np.float32)
    gc, gs = _run(dev, inp, cu=cu, half=half)
    for s in (0, 1, 2):
        t0, L = int(cu[s]), int(lens[s])
        c1, s1 = _run(dev, {k_: v_[:, t0:t0 + L] for k_, v_ in inp.items()}, half=half)
        assert np.array_equal(c1, gc[:, t0:t0 + L]) and np.array_equal(s1[0], gs[s])


def test_collect_and_last_to_fp16(dev, oracle):
    from spock_amd import ops, synth
    H, T = 16, 9
    rng = np.random.default_rng(0)
    qo, ko, vo = (np.zeros((H, T, 128), np.float32) for _ in range(3))
    go = np.zeros((H, T), np.float32)
    bo = np.zeros((H, T), np.float32)
    dq = [torch.zeros((H, T, 128), device=dev) for _ in range(3)] + [torch.zeros((H, T), device=dev) for _ in range(2)]
    for t in range(T):
        qkv = synth.f16(rng.normal(size=6144).astype(np.float32))
        gb = rng.normal(size=32).astype(np.float32)
        oracle.prefill_collect(qkv, gb, H, T, t, (qo, ko, vo, go, bo))
        ops.prefill_collect(_to(dev, qkv.view(np.float16), torch.float16), _to(dev, gb), dq, T, t)
    torch.cuda.synchronize()
    for a, b in zip(dq, (qo, ko, vo, go, bo)):
        assert np.array_equal(a.cpu().numpy(), b)
    src = rng.normal(size=(H * 128 * 128,)).astype(np.float32) * 1e3
    src[:50] = 1e-7  # flush-to-zero region
    out = ops.chunk_last_to_fp16(_to(dev, src), seq_len=100, total_seq=128)
    torch.cuda.synchronize()
    exp = oracle.chunk_last_to_fp16(src, H, 128, 100, 128)
    assert np.array_equal(out.cpu().numpy().view(np.uint16), exp)


def test_chunk_prefill_rejects_inconsistent_arguments(dev):
    """The Python mirror checks every operand the kernels index from N, S and
    cu_seqlens before a launch (no kernel runs for these calls)."""
    from spock_amd import ops
    from spock_amd._lib import SpockError
    H, N = 2, 100
    f = lambda *s, dt=torch.float32: torch.zeros(*s, dtype=dt, device=dev)
    q, k, v, g, b = f(H, N, 128), f(H, N, 128), f(H, N, 128), f(H, N), f(H, N)
    cu = [0, 40, 100]
    bad = [
        dict(k=f(H, N - 1, 128)), dict(v=f(H + 1, N, 128)), dict(g=f(H, N + 1)), dict(beta=f(N)),
        dict(initial_state=f(1, H, 128, 128), cu_seqlens=cu),
        dict(initial_state=f(2, H, 128, 128, dt=torch.float16), cu_seqlens=cu),
        dict(out_state=f(1, H, 128, 128), cu_seqlens=cu),
        dict(out_core=f(H, N - 1, 128)),
        dict(out_core=f(H, N, 128), core_head_stride=N + 5),
        dict(cu_seqlens=cu, cu_seqlens_dev=torch.tensor(cu, dtype=torch.int64, device=dev)),
        dict(cu_seqlens=cu, cu_seqlens_dev=torch.tensor([0, 50, 100], dtype=torch.int32, device=dev)),
        dict(cu_seqlens=cu, cu_seqlens_dev=torch.tensor([0, 100], dtype=torch.int32, device=dev)),
        dict(cu_seqlens_dev=torch.tensor(cu, dtype=torch.int32, device=dev)),
    ]
    for kw in bad:
        args = dict(q=q, k=k, v=v, g=g, beta=b)
        args.update(kw)
        with pytest.raises(SpockError):
            ops.chunk_prefill(**args)
    torch.cuda.synchronize()
    # the consistent call still runs
    ops.chunk_prefill(q, k, v, g, b, cu_seqlens=cu,
                      cu_seqlens_dev=torch.tensor(cu, dtype=torch.int32, device=dev))
    torch.cuda.synchronize()


def test_packed_prefill_graph_replays_equal_eager(dev):
    """A ragged pack (host sequence tables, longest first) captured into a HIP
    graph: every replay, with eager work and synchronisations in between,
    gives the eager bits."""
    from spock_amd import ops, synth
    lens = [3000, 200, 2900, 700, 64, 1500]
    cu = synth.cu_seqlens_from(lens)
    N = int(cu[-1])
    inp = synth.chunk_inputs(16, N, seed=12)
    q, k, v = (_to(dev, inp[n], torch.float16) for n in ("q", "k", "v"))
    g, b = _to(dev, inp["g"]), _to(dev, inp["beta"])
    cu_dev = torch.from_numpy(np.asarray(cu, np.int32)).to(dev)
    core = torch.empty((16, N, 128), device=dev)
    state = torch.empty((len(lens), 16, 128, 128), device=dev)
    ws = torch.empty(ops.chunk_workspace_bytes(16, N, len(lens)), dtype=torch.uint8, device=dev)
    call = lambda: ops.chunk_prefill(q, k, v, g, b, cu_seqlens=cu, cu_seqlens_dev=cu_dev, out_core=core,
                                     out_state=state, workspace=ws)
    call()
    torch.cuda.synchronize()
    ref_c, ref_s = core.cpu().numpy(), state.cpu().numpy()
    gr = torch.cuda.CUDAGraph()
    with torch.cuda.graph(gr):
        call()
    for _ in range(3):
        core.fill_(float("nan"))
        state.fill_(float("nan"))
        torch.cuda.synchronize()
        gr.replay()
        torch.cuda.synchronize()
        assert np.array_equal(core.cpu().numpy(), ref_c)
        assert np.array_equal(state.cpu().numpy(), ref_s)


def test_many_sequences_device_table_path(dev, oracle):
    """More sequences than the host tables hold (32): the kernels find the
    chunks from the device cu_seqlens, with the same results."""
    from spock_amd import synth
    rng = np.random.default_rng(5)
    lens = [int(x) for x in rng.integers(1, 150, 40)]
    cu = synth.cu_seqlens_from(lens)
    inp = synth.chunk_inputs(4, int(cu[-1]), seed=22)
    cc, cs = oracle.chunk_rule_varlen(**inp, cu=cu)
    gc, gs = _run(dev, inp, cu=cu)
    assert max_rel(gc, cc) <= TOL
    assert max_rel(gs, cs) <= TOL


def _random_case(i):
    """Seeded random pack: head count, ragged lengths (empty, sub-chunk and
    chunk-boundary lengths included), input dtype, L2 inside the kernel or
    not, initial state or not."""
    rng = np.random.default_rng(1000 + i)
    H = int(rng.choice([1, 2, 3, 5, 8, 16]))
    S = int(rng.integers(1, 7))
    choices = [0, 1, 2, 31, 63, 64, 65, 127, 128, 129, 191, 200, 256, 300]
    lens = [int(rng.choice(choices)) if rng.random() < 0.5 else int(rng.integers(1, 320)) for _ in range(S)]
    if sum(lens) == 0:
        lens[0] = 17
    return H, lens, bool(rng.random() < 0.5), bool(rng.random() < 0.5), bool(rng.random() < 0.5)


@pytest.mark.parametrize("i", range(20))
def test_random_packs_against_oracle(dev, oracle, i):
    """Seeded random packs through the packed launch (host sequence table,
    split intra parts for the small ones) against the oracle's per-sequence
    chunk rule, to the north-star tolerance."""
    from spock_amd import synth
    H, lens, l2, init, half = _random_case(i)
    print(f"[random pack {i}: H={H} lens={lens} l2={l2} init={init} half={half}]", flush=True)
    cu = synth.cu_seqlens_from(lens)
    inp = synth.chunk_inputs(H, int(cu[-1]), seed=300 + i, l2=not l2)
    if half:
        for n in ("q", "k", "v"):
            inp[n] = inp[n].astype(np.float16).astype(np.float32)
    st0 = (np.random.default_rng(i).normal(0, 0.05, (len(lens), H, 128, 128)).astype(np.float32)
           if init else None)
    cc, cs = oracle.chunk_rule_varlen(**inp, cu=cu, init=st0, l2=l2)
    gc, gs = _run(dev, inp, init=st0, cu=cu, l2=l2, half=half)
    assert max_rel(gc, cc) <= TOL
    assert max_rel(gs, cs) <= TOL


def _poisoned(dev, a, dtype, fill, extra_rows=64):
    """`a` [H][N][128] copied to the front of a larger device buffer whose
    remaining `extra_rows` rows hold `fill` (NaN or Inf): a row read past the
    tensor's end returns that value instead of finite garbage."""
    H, N, D = a.shape
    buf = torch.full((H * N * D + extra_rows * D,), fill, dtype=dtype, device=dev)
    buf[:H * N * D] = torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype).reshape(-1)
    return buf[:H * N * D].view(H, N, D)


@pytest.mark.parametrize("half", [False, True])
@pytest.mark.parametrize("last", [1, 17, 63])
def test_padding_rows_never_read_past_the_chunk(dev, oracle, half, last):
    """The last chunk of a sequence is zero padded to 64 rows.  The kernels
    must not read the padding rows from memory: q/k/v are placed at the front
    of larger buffers whose tail holds NaN (q, v) and Inf (k), the pack's last
    sequence ends on a partial chunk of `last` rows, so its padding rows fall
    past the tensor's end.  One head alone (H=1) and 16 heads, packed after a
    ragged sequence, must match the oracle and stay finite (NaN or Inf read
    into U, W or S would spread through 0 * Inf into every output row)."""
    from spock_amd import ops, synth
    dt = torch.float16 if half else torch.float32
    for H, lens in ((1, [last]), (16, [130, 64 + last])):
        print(f"[poisoned tail H={H} lens={lens} half={half}]", flush=True)
        cu = synth.cu_seqlens_from(lens)
        inp = synth.chunk_inputs(H, int(cu[-1]), seed=40 + last)
        if half:
            for n in ("q", "k", "v"):
                inp[n] = inp[n].astype(np.float16).astype(np.float32)
        q = _poisoned(dev, inp["q"], dt, float("nan"))
        k = _poisoned(dev, inp["k"], dt, float("inf"))
        v = _poisoned(dev, inp["v"], dt, float("nan"))
        core, state = ops.chunk_prefill(q, k, v, _to(dev, inp["g"]), _to(dev, inp["beta"]),
                                        cu_seqlens=cu)
        torch.cuda.synchronize()
        gc, gs = core.cpu().numpy(), state.cpu().numpy()
        assert np.isfinite(gc).all() and np.isfinite(gs).all()
        cc, cs = oracle.chunk_rule_varlen(**inp, cu=cu)
        assert max_rel(gc, cc) <= TOL
        assert max_rel(gs, cs) <= TOL
