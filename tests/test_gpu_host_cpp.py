"""The C++ host layer on the GPU, through its command-line drivers:
run_deltanet_chunk_rule (the reference's CPU interface, deltanet_chunk.hpp:39-40)
and DeltaNetSession (the DeltaNet part of DecodeSession), checked against the
oracle and the reference's own unit case."""
import json
import subprocess

import numpy as np
import pytest

import host_cli as HC
from conftest import GOLDEN, max_rel
from spock_amd import synth

pytestmark = pytest.mark.gpu


def test_reference_unit_case_through_cli(dev, tmp_path, oracle):
    """tests/run_deltanet_chunk_unit.py:104-170: H=2, T=5, dk=3, dv=2, C=4,
    L2 on, initial state; |diff| <= 1e-5 against the reference rule's outputs
    (golden, from oracle/_ref) and against the fp64 recurrence."""
    z = np.load(GOLDEN / "chunk_unit_case.npz")
    H, T, dk, dv, C, l2 = (int(x) for x in z["meta"])
    fx = HC.chunk_fixture(z["q"], z["k"], z["v"], z["g"], z["beta"], init=z["init"], chunk_size=C, l2=bool(l2))
    r = HC.run_chunk_cli(tmp_path, fx)
    assert r.returncode == 0, r.stderr
    core, state = HC.parse_chunk_output(r.stdout, H, T, dk, dv)
    assert np.abs(core - z["core"]).max() <= 1e-5
    assert np.abs(state - z["state"]).max() <= 1e-5
    c64, s64 = oracle.delta_recurrence_f64(z["q"], z["k"], z["v"], z["g"], z["beta"], init=z["init"], l2=True)
    assert np.abs(core - c64).max() <= 1e-5 and np.abs(state - s64).max() <= 1e-5


@pytest.mark.parametrize("H,T,dk,dv,l2,init", [(4, 104, 128, 128, False, False),
                                                (3, 130, 128, 128, True, True),
                                                (2, 70, 64, 32, True, True),
                                                (1, 1, 128, 128, False, True)])
def test_chunk_cli_vs_oracle(dev, tmp_path, oracle, H, T, dk, dv, l2, init):
    inp = synth.chunk_inputs(H, T, dk=dk, dv=dv, seed=40 + T, l2=not l2)
    st0 = (synth.normal(99 + T, H * dk * dv, std=0.05).reshape(H, dk, dv) if init else None)
    r = HC.run_chunk_cli(tmp_path, HC.chunk_fixture(**inp, init=st0, l2=l2))
    assert r.returncode == 0, r.stderr
    core, state = HC.parse_chunk_output(r.stdout, H, T, dk, dv)
    # the CLI prints 9 significant digits: exact for fp32 round trips
    cc, cs = oracle.chunk_rule(**inp, init=st0, l2=l2)
    assert max_rel(core, cc) <= 1e-5 and max_rel(state, cs) <= 1e-5


def test_chunk_size_is_the_kernel_blocking(dev, tmp_path, oracle):
    """run_deltanet_chunk_rule validates chunk_size and then runs the kernels'
    64-token blocking: C = 4, 16 and 64 give the same bits, each within 1e-5
    of the reference rule at its own C."""
    inp = synth.chunk_inputs(2, 37, dk=128, dv=128, seed=17)
    outs = []
    for C in (4, 16, 64):
        r = HC.run_chunk_cli(tmp_path, HC.chunk_fixture(**inp, chunk_size=C, l2=False))
        assert r.returncode == 0, r.stderr
        core, state = HC.parse_chunk_output(r.stdout, 2, 37, 128, 128)
        cc, cs = oracle.chunk_rule(**inp, chunk=C, l2=False)
        assert max_rel(core, cc) <= 1e-5 and max_rel(state, cs) <= 1e-5
        outs.append((core, state))
    for core, state in outs[1:]:
        assert np.array_equal(core, outs[0][0]) and np.array_equal(state, outs[0][1])


def _session_inputs(L, T, D, V, hidden, seed):
    CD, NH = 6144, 16
    pre_qkv = np.empty((L, T, CD), dtype=np.uint16)
    pre_gb = np.empty((L, T, 2 * NH), dtype=np.float32)
    for l in range(L):
        c = synth.chunk_inputs(NH, T, seed=seed + l)
        # token-major dn_qkv [Q h*128+d | K | V] in fp16, g/beta [g H | beta H]
        pre_qkv[l, :, :2048] = synth.f16(c["q"].transpose(1, 0, 2).reshape(T, 2048))
        pre_qkv[l, :, 2048:4096] = synth.f16(c["k"].transpose(1, 0, 2).reshape(T, 2048))
        pre_qkv[l, :, 4096:] = synth.f16(c["v"].transpose(1, 0, 2).reshape(T, 2048))
        pre_gb[l, :, :NH] = c["g"].T
        pre_gb[l, :, NH:] = c["beta"].T
    d = synth.decode_inputs(D * L, seed=seed + 100, layers=L)
    conv = synth.decode_inputs(L, seed=seed + 200, layers=L)["conv_state"]
    conv_w = np.stack([synth.gemv_weights(CD, 4, seed=seed + 300 + l) for l in range(L)])
    norm_w = (1.0 + synth.normal(seed + 400, 128, std=0.1)).astype(np.float32)
    return {
        "prefill_qkv.u16": pre_qkv, "prefill_gbeta.f32": pre_gb,
        "a_log_bias.f32": d["a_log_bias"], "conv_state.u16": conv, "conv_weight.u16": conv_w,
        "norm_weight.f32": norm_w,
        "decode_qkv.u16": d["qkv"].reshape(D, L, CD), "decode_a.u16": d["a"].reshape(D, L, NH),
        "decode_b.u16": d["b"].reshape(D, L, NH), "decode_z.u16": d["z"].reshape(D, L, 2048),
        "lm_weight.u16": synth.gemv_weights(V, hidden, seed=seed + 500),
        "lm_x.u16": synth.gemv_input(hidden, seed=seed + 501),
    }


@pytest.mark.parametrize("L,T,D", [(2, 100, 3), (1, 128, 2)])
def test_session_flow_vs_oracle(dev, tmp_path, oracle, L, T, D):
    V, hidden = 4096, 1024
    inp = _session_inputs(L, T, D, V, hidden, seed=7 * T + L)
    ind, outd = tmp_path / "in", tmp_path / "out"
    ind.mkdir()
    outd.mkdir()
    (ind / "meta.json").write_text(json.dumps({"layers": L, "prompt_len": T, "decode_steps": D,
                                               "vocab": V, "hidden": hidden}))
    for name, arr in inp.items():
        np.ascontiguousarray(arr).tofile(ind / name)
    r = subprocess.run([str(HC.SESSION_CLI), "--input", str(ind), "--output", str(outd)],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    rd = lambda n, dt: np.fromfile(outd / n, dtype=dt)
    SF = 16 * 128 * 128 + 32
    core = rd("prefill_core.f32", np.float32).reshape(L, 16, T, 128)
    attn = rd("chunk_attn_out.u16", np.uint16).reshape(L, 2048)
    pstate = rd("prefill_state.f32", np.float32).reshape(L, SF)
    for l in range(L):
        # collect (deltanet_prefill_collect.comp) is exact: fp16 -> fp32
        qkv = inp["prefill_qkv.u16"][l].view(np.float16).astype(np.float32)
        q = qkv[:, :2048].reshape(T, 16, 128).transpose(1, 0, 2)
        k = qkv[:, 2048:4096].reshape(T, 16, 128).transpose(1, 0, 2)
        v = qkv[:, 4096:].reshape(T, 16, 128).transpose(1, 0, 2)
        g = inp["prefill_gbeta.f32"][l, :, :16].T
        beta = inp["prefill_gbeta.f32"][l, :, 16:].T
        cc, cs = oracle.chunk_rule(q, k, v, g, beta, l2=False)
        assert max_rel(core[l], cc) <= 1e-5, l
        assert max_rel(pstate[l, :SF - 32].reshape(16, 128, 128), cs) <= 1e-5, l
        assert not pstate[l, SF - 32:].any()  # g/beta tail untouched (zero after reset)
        total = (T + 63) // 64 * 64
        padded = np.zeros((16, total, 128), dtype=np.float32)
        padded[:, :T] = core[l]
        assert np.array_equal(attn[l], oracle.chunk_last_to_fp16(padded, 16, 128, T, total))
    # decode: oracle steps from the device's post-prefill state, bit-exact
    st = [pstate[l][None].copy() for l in range(L)]
    cs_ = [inp["conv_state.u16"][l][None].copy() for l in range(L)]
    dec = rd("decode_out.u16", np.uint16).reshape(D, L, 6144)
    for d in range(D):
        for l in range(L):
            step = {"state": st[l], "conv_state": cs_[l], "qkv": inp["decode_qkv.u16"][d, l][None],
                    "z": inp["decode_z.u16"][d, l][None], "a": inp["decode_a.u16"][d, l][None],
                    "b": inp["decode_b.u16"][d, l][None], "a_log_bias": inp["a_log_bias.f32"],
                    "conv_w": inp["conv_weight.u16"][l], "norm_w": inp["norm_weight.f32"]}
            oq, cs_[l], st[l] = oracle.decode_step(step, layer_idx=l)
            assert np.array_equal(dec[d, l], oq[0]), (d, l)
    fstate = rd("final_state.f32", np.float32).reshape(L, SF)
    fconv = rd("final_conv_state.u16", np.uint16).reshape(L, 6144, 4)
    for l in range(L):
        assert np.array_equal(fstate[l].view(np.uint32), st[l][0].view(np.uint32)), l
        assert np.array_equal(fconv[l], cs_[l][0]), l
    tok = json.loads((outd / "token.json").read_text())["token"]
    assert tok == oracle.lm_head_argmax(inp["lm_weight.u16"], inp["lm_x.u16"])[0]
