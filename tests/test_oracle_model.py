"""Pinning of the full-model oracle (oracle/model.h) on the CPU.

* residual_add / silu_gate against the reference's own GPU captures
  (tests/data/layer0_step1_*.fp16 of the real model, copied to
  tests/golden/ref_data): residual bit-exact, SiLU gate within the reference's
  2-ulp fp16 policy (diary/0089; GLSL exp differs from ours);
* RMSNorm, per-head norm, RoPE and attention against float64 formulas;
* the deterministic-exp chunk rule against the reference-exact one;
* the whole model against an independent float64 numpy forward of the same
  architecture (HF semantics, the token recurrence instead of the chunk rule,
  fp16 storage at the same points) on a small seeded artifact.
"""
import ctypes as C

import numpy as np
import pytest

from conftest import GOLDEN, fp16_ulp

REF = GOLDEN / "ref_data"


def _p(a):
    return a.ctypes.data


def _om():
    import oracle_model
    return oracle_model.lib()


def _fx(name):
    return np.fromfile(REF / f"layer0_step1_{name}.fp16", dtype=np.uint16)


def test_residual_add_matches_reference_capture():
    for a, b, want in (("input_hidden_1024", "mixer_output_1024", "mixer_residual_1024"),
                       ("mixer_residual_1024", "down_output_1024", "post_mlp_1024")):
        x, y, w = _fx(a), _fx(b), _fx(want)
        out = np.zeros_like(w)
        _om().orc_residual_add(_p(x), _p(y), _p(out), out.size)
        assert np.array_equal(out, w), (a, b)


def test_silu_gate_matches_reference_capture():
    g, u, want = _fx("mlp_gate_3584"), _fx("mlp_up_3584"), _fx("mlp_product_3584")
    out = np.zeros_like(want)
    _om().orc_silu_gate(_p(g), _p(u), _p(out), out.size)
    assert int(fp16_ulp(out, want).max()) <= 2


def _h(n, seed, std=1.0):
    from spock_amd import synth
    return synth.f16(synth.normal(seed, n, std=std))


def _f(h):
    return np.asarray(h, np.uint16).view(np.float16).astype(np.float64)


def test_rmsnorms_against_fp64():
    x, w = _h(1024, 1), _h(1024, 2, 0.02)
    y = np.zeros(1024, np.uint16)
    _om().orc_rmsnorm1024(_p(x), _p(w), _p(y))
    xf = _f(x)
    ref = xf / np.sqrt(np.mean(xf * xf) + 1e-6) * (1 + _f(w))
    assert int(fp16_ulp(y, ref.astype(np.float16).view(np.uint16)).max()) <= 1
    x2, w2 = _h(256, 3), _h(256, 4, 0.02)
    y2 = np.zeros(256, np.uint16)
    _om().orc_head_rmsnorm256(_p(x2), _p(w2), _p(y2))
    xf = _f(x2)
    ref = xf / np.sqrt(np.mean(xf * xf) + 1e-6) * (1 + _f(w2))
    assert int(fp16_ulp(y2, ref.astype(np.float16).view(np.uint16)).max()) <= 1


def test_rope_against_fp64_rotation():
    pos, heads = 517, 3
    table = np.zeros((pos + 1) * 64, np.float32)
    _om().orc_rope_table(pos + 1, _p(table))
    i = np.arange(32)
    ang = pos * 1e7 ** (-(2.0 * i) / 64.0)
    assert np.max(np.abs(table[pos * 64::2][:32] - np.cos(ang))) < 1e-7
    x = _h(heads * 256, 5)
    y = x.copy()
    _om().orc_rope_apply(_p(y), heads, _p(np.ascontiguousarray(table[pos * 64:pos * 64 + 64])))
    xf = _f(x).reshape(heads, 256)
    ref = xf.copy()
    c, s = np.cos(ang), np.sin(ang)
    ref[:, :32] = xf[:, :32] * c - xf[:, 32:64] * s      # rotate_half on the first 64 dims
    ref[:, 32:64] = xf[:, 32:64] * c + xf[:, :32] * s
    got = _f(y).reshape(heads, 256)
    assert np.array_equal(got[:, 64:], xf[:, 64:])
    assert np.max(np.abs(got - ref) / np.maximum(1e-3, np.abs(ref))) < 2e-3


@pytest.mark.parametrize("npos", [1, 63, 64, 65, 300])
def test_attention_against_fp64_softmax(npos):
    kv = _h(npos * 1024, 6).reshape(npos, 1024)
    q = _h(256, 7)
    out = np.zeros(256, np.uint16)
    _om().orc_attend(_p(q), _p(np.ascontiguousarray(kv)), 1, npos, _p(out))
    K = _f(kv[:, 256:512])
    V = _f(kv[:, 512 + 256:512 + 512])
    sc = K @ _f(q) / 16.0
    w = np.exp(sc - sc.max())
    ref = (w @ V) / w.sum()
    assert np.max(np.abs(_f(out) - ref)) <= 2e-3 * max(1.0, np.max(np.abs(ref)))


def test_deterministic_exp_chunk_rule_close_to_reference_exact(oracle):
    from spock_amd import synth
    L = oracle.lib()
    L.orc_chunk_rule_det.restype = C.c_int
    L.orc_chunk_rule_det.argtypes = [C.c_size_t] * 5 + [C.c_int] + [C.c_void_p] * 8
    inp = synth.chunk_inputs(4, 150, seed=9)
    c1, s1 = oracle.chunk_rule(**inp)
    c2 = np.zeros_like(c1)
    s2 = np.zeros_like(s1)
    assert L.orc_chunk_rule_det(4, 150, 128, 128, 64, 0, *[_p(inp[n]) for n in ("q", "k", "v", "g", "beta")],
                                None, _p(c2), _p(s2)) == 0
    rel = lambda a, b: float(np.max(np.abs(a - b) / np.maximum(1.0, np.abs(b))))
    assert rel(c2, c1) <= 1e-5 and rel(s2, s1) <= 1e-5
    assert not np.array_equal(c1, c2)  # the exp really differs somewhere


# ---- independent float64 forward of the whole model --------------------------

def _r16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


class NumpyModel:
    """HF Qwen3.5 text forward (modeling_qwen3_5.py:387-795) in float64 with
    fp16 storage where the engine stores fp16; DeltaNet by its token
    recurrence.  Written from the architecture, not from the oracle."""

    def __init__(self, art):
        import oracle_model
        self.man, self.w, self.roles = oracle_model.load_artifact(art)
        self.t = lambda role: oracle_model.tensor(self.w, self.roles[role]).astype(np.float64) \
            if self.roles[role]["dtype"] == "fp32" else _f(oracle_model.tensor(self.w, self.roles[role]))
        self.L = self.man["model"]["layers"]

    @staticmethod
    def rms(x, w):
        return _r16(x / np.sqrt(np.mean(x * x, -1, keepdims=True) + 1e-6) * (1 + w))

    def forward(self, tokens):
        T = len(tokens)
        t = self.t
        h = t("global.token_embedding")[tokens]
        ang = np.arange(T)[:, None] * 1e7 ** (-(2.0 * np.arange(32)) / 64.0)
        cos = np.concatenate([np.cos(ang)] * 2, -1)
        sin = np.concatenate([np.sin(ang)] * 2, -1)
        for L in range(self.L):
            r = f"layer.{L}."
            x = self.rms(h, t(r + "input_norm"))
            if L % 4 == 3:
                qg = _r16(x @ t(r + "attn_q").T).reshape(T, 8, 512)
                q, gate = qg[..., :256], qg[..., 256:].reshape(T, 2048)
                k = _r16(x @ t(r + "attn_k").T).reshape(T, 2, 256)
                v = _r16(x @ t(r + "attn_v").T).reshape(T, 2, 256)
                q, k = self.rms(q, t(r + "attn_q_norm")), self.rms(k, t(r + "attn_k_norm"))

                def rope(a):
                    rot = a[..., :64]
                    half = np.concatenate([-rot[..., 32:], rot[..., :32]], -1)
                    return np.concatenate([_r16(rot * cos[:, None] + half * sin[:, None]), a[..., 64:]], -1)
                q, k = rope(q), rope(k)
                out = np.zeros((T, 8, 256))
                for hh in range(8):
                    s = q[:, hh] @ k[:, hh // 4].T / 16.0
                    s = np.where(np.tril(np.ones((T, T))) > 0, s, -np.inf)
                    p = np.exp(s - s.max(-1, keepdims=True))
                    out[:, hh] = _r16((p @ v[:, hh // 4]) / p.sum(-1, keepdims=True))
                att = _r16(out.reshape(T, 2048) / (1 + np.exp(-gate)))
                mix = _r16(att @ t(r + "attn_o").T)
            else:
                qkv = _r16(x @ t(r + "delta_in_proj_qkv").T)
                z = _r16(x @ t(r + "delta_in_proj_z").T)
                a = _r16(x @ t(r + "delta_in_proj_a").T)
                b = _r16(x @ t(r + "delta_in_proj_b").T)
                w = t(r + "delta_conv").reshape(6144, 4)
                pad = np.concatenate([np.zeros((3, 6144)), qkv], 0)
                conv = sum(pad[i:i + T] * w[:, i] for i in range(4))
                y = _r16(conv / (1 + np.exp(-conv)))
                qh, kh, vh = (y[:, i * 2048:(i + 1) * 2048].reshape(T, 16, 128) for i in range(3))
                qh = _r16(qh / np.sqrt((qh * qh).sum(-1, keepdims=True) + 1e-6))
                kh = _r16(kh / np.sqrt((kh * kh).sum(-1, keepdims=True) + 1e-6))
                dt = t(r + "delta_dt_bias")
                g = -np.exp(t(r + "delta_a_log")) * np.log1p(np.exp(a + dt))
                beta = 1 / (1 + np.exp(-b))
                S = np.zeros((16, 128, 128))
                o = np.zeros((T, 16, 128))
                for i in range(T):
                    S = S * np.exp(g[i])[:, None, None]
                    kv_mem = np.einsum("hkv,hk->hv", S, kh[i])
                    delta = (vh[i] - kv_mem) * beta[i][:, None]
                    S = S + kh[i][:, :, None] * delta[:, None, :]
                    o[i] = np.einsum("hkv,hk->hv", S, qh[i] / np.sqrt(128.0))
                nrm = o / np.sqrt(np.mean(o * o, -1, keepdims=True) + 1e-6) * t(r + "delta_norm")
                zz = z.reshape(T, 16, 128)
                gated = _r16(_r16(nrm) * zz / (1 + np.exp(-zz))).reshape(T, 2048)
                mix = _r16(gated @ t(r + "delta_out_proj").T)
            h = _r16(h + mix)
            x = self.rms(h, t(r + "post_norm"))
            gt, up = _r16(x @ t(r + "mlp_gate").T), _r16(x @ t(r + "mlp_up").T)
            m = _r16(gt / (1 + np.exp(-gt)) * up)
            h = _r16(h + _r16(m @ t(r + "mlp_down").T))
        hn = self.rms(h[-1], t("global.final_norm"))
        return _r16(hn @ t("global.token_embedding").T)


def test_whole_model_against_independent_fp64_forward(tmp_path):
    """The numpy forward tracks the oracle to ~0.003 in the logits; planted
    bugs in it (GQA head mapping, RoPE sign, attention scale, conv tap order,
    dropped beta / decay / q scale, q-gate split) move them by 0.15-3.2."""
    import oracle_model
    from spock_amd import model, synth
    art = model.write_synthetic_artifact(tmp_path / "a", layers=4, vocab=2048, seed=21)
    tokens = (synth.splitmix64(8, 40) % np.uint64(2048)).astype(np.int32)
    om = oracle_model.OracleModel(art, max_seq=64)
    tok, logits, _ = om.prefill(tokens, want_logits=True)
    ref = NumpyModel(art).forward(tokens)
    got = _f(logits)
    assert np.max(np.abs(got - ref)) <= 0.01 * max(1.0, np.max(np.abs(ref)))
    order = np.argsort(-ref)
    if ref[order[0]] - ref[order[1]] > 0.02:
        assert tok == int(order[0])
    # one decode step against the forward of the extended prompt
    tok2, logits2, _ = om.decode(tok, want_logits=True)
    ref2 = NumpyModel(art).forward(np.concatenate([tokens, [tok]]).astype(np.int64))
    assert np.max(np.abs(_f(logits2) - ref2)) <= 0.01 * max(1.0, np.max(np.abs(ref2)))
