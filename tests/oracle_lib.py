"""ctypes binding of the CPU oracle (oracle/liboracle.so) and of the reference's
own compiled chunk rule (oracle/_ref/libref_chunk.so).  TEST INFRASTRUCTURE:
imported by tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
only, always as the checker."""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
ORACLE_SO = ROOT / "oracle" / "liboracle.so"
REF_SO = ROOT / "oracle" / "_ref" / "libref_chunk.so"

_c = ctypes
_sz = _c.c_size_t
_p = _c.c_void_p


def _ptr(a):
    return None if a is None else a.ctypes.data_as(_p)


def _load_oracle():
    if not ORACLE_SO.exists():
        raise RuntimeError(f"oracle library missing: {ORACLE_SO} (run __graft_entry__.build())")
    lib = _c.CDLL(str(ORACLE_SO))
    lib.orc_h2f.restype = _c.c_float
    lib.orc_h2f.argtypes = [_c.c_uint16]
    lib.orc_f2h_rne.restype = _c.c_uint16
    lib.orc_f2h_rne.argtypes = [_c.c_float]
    lib.orc_f2h_trunc.restype = _c.c_uint16
    lib.orc_f2h_trunc.argtypes = [_c.c_float]
    for n in ("orc_expf", "orc_logf", "orc_rsqrtf"):
        getattr(lib, n).restype = _c.c_float
        getattr(lib, n).argtypes = [_c.c_float]
    for n in ("orc_h2f_array", "orc_f2h_rne_array", "orc_expf_array", "orc_logf_array"):
        getattr(lib, n).restype = None
        getattr(lib, n).argtypes = [_p, _p, _sz]
    lib.orc_chunk_rule.restype = _c.c_int
    lib.orc_chunk_rule.argtypes = [_sz] * 5 + [_c.c_int] + [_p] * 8
    lib.orc_chunk_rule_varlen.restype = _c.c_int
    lib.orc_chunk_rule_varlen.argtypes = [_sz] * 5 + [_c.c_int, _p, _sz] + [_p] * 8
    lib.orc_delta_recurrence_f64.restype = None
    lib.orc_delta_recurrence_f64.argtypes = [_sz] * 4 + [_c.c_int] + [_p] * 8
    lib.orc_prefill_collect.restype = None
    lib.orc_prefill_collect.argtypes = [_sz] * 5 + [_p] * 7
    lib.orc_chunk_last_to_fp16.restype = None
    lib.orc_chunk_last_to_fp16.argtypes = [_sz] * 4 + [_p, _p]
    lib.orc_conv_l2_qk.restype = None
    lib.orc_conv_l2_qk.argtypes = [_sz] * 4 + [_p] * 3
    lib.orc_recurrent_gbeta_norm_gate.restype = None
    lib.orc_recurrent_gbeta_norm_gate.argtypes = [_sz, _sz, _c.c_float, _c.c_float] + [_p] * 8
    lib.orc_gbeta.restype = None
    lib.orc_gbeta.argtypes = [_c.c_float] * 4 + [_p, _p]
    lib.orc_norm_gate_row.restype = None
    lib.orc_norm_gate_row.argtypes = [_p, _p, _p, _c.c_float, _p]
    lib.orc_norm_gate_f16.restype = None
    lib.orc_norm_gate_f16.argtypes = [_sz, _c.c_float, _p, _p, _p]
    lib.orc_recurrent.restype = None
    lib.orc_recurrent.argtypes = [_sz, _c.c_float, _p, _p]
    lib.orc_decode_step.restype = None
    lib.orc_decode_step.argtypes = [_sz, _sz, _sz, _c.c_float, _c.c_float,
                                    _p, _sz, _p, _sz, _p, _p, _p, _sz, _p, _p, _sz, _p, _sz, _p]
    lib.orc_matvec_f16.restype = _c.c_int
    lib.orc_matvec_f16.argtypes = [_p, _p, _p, _sz, _sz]
    for name in ("orc_matvec_f16_strided", "orc_matvec_f16_serial"):
        getattr(lib, name).restype = _c.c_int
        getattr(lib, name).argtypes = [_p, _p, _p, _sz, _sz]
    lib.orc_argmax_f16.restype = _c.c_uint32
    lib.orc_argmax_f16.argtypes = [_p, _sz]
    lib.orc_lm_head_argmax.restype = _c.c_uint32
    lib.orc_lm_head_argmax.argtypes = [_p, _p, _sz, _sz, _p]
    return lib


_LIB = None
_REF = None


def lib():
    global _LIB
    if _LIB is None:
        _LIB = _load_oracle()
    return _LIB


def ref_available() -> bool:
    return REF_SO.exists()


def ref():
    global _REF
    if _REF is None:
        if not REF_SO.exists():
            raise RuntimeError(f"reference chunk rule not built: {REF_SO}")
        r = _c.CDLL(str(REF_SO))
        r.ref_chunk_rule.restype = _c.c_int
        r.ref_chunk_rule.argtypes = [_sz] * 5 + [_c.c_int] + [_p] * 8
        _REF = r
    return _REF


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


# ---- numerics ---------------------------------------------------------------
def expf(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_expf_array(_ptr(x), _ptr(out), x.size)
    return out


def logf(x):
    x = _f32(x)
    out = np.empty_like(x)
    lib().orc_logf_array(_ptr(x), _ptr(out), x.size)
    return out


def h2f(h):
    h = _u16(h)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_h2f_array(_ptr(h), _ptr(out), h.size)
    return out


def f2h(x):
    x = _f32(x)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f2h_rne_array(_ptr(x), _ptr(out), x.size)
    return out


# ---- chunk rule -------------------------------------------------------------
def chunk_rule(q, k, v, g, beta, init=None, chunk=64, l2=False, use_ref=False):
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    H, T, dk = q.shape
    dv = v.shape[2]
    init = None if init is None else _f32(init)
    core = np.empty((H, T, dv), dtype=np.float32)
    state = np.empty((H, dk, dv), dtype=np.float32)
    fn = ref().ref_chunk_rule if use_ref else lib().orc_chunk_rule
    rc = fn(H, T, dk, dv, chunk, int(l2), _ptr(q), _ptr(k), _ptr(v), _ptr(g), _ptr(beta),
            _ptr(init), _ptr(core), _ptr(state))
    if rc != 0:
        raise RuntimeError(f"chunk rule rc={rc}")
    return core, state


def chunk_rule_varlen(q, k, v, g, beta, cu, init=None, chunk=64, l2=False):
    q, k, v, g, beta = map(_f32, (q, k, v, g, beta))
    cu = np.ascontiguousarray(cu, dtype=np.int32)
    H, N, dk = q.shape
    dv = v.shape[2]
    S = len(cu) - 1
    init = None if init is None else _f32(init)
    core = np.empty((H, N, dv), dtype=np.float32)
    state = np.empty((S, H, dk, dv), dtype=np.float32)
    rc = lib().orc_chunk_rule_varlen(H, N, dk, dv, chunk, int(l2), _ptr(cu), S, _ptr(q), _ptr(k),
                                     _ptr(v), _ptr(g), _ptr(beta), _ptr(init), _ptr(core),
                                     _ptr(state))
    if rc != 0:
        raise RuntimeError(f"chunk rule varlen rc={rc}")
    return core, state


def delta_recurrence_f64(q, k, v, g, beta, init=None, l2=False):
    c = lambda a: np.ascontiguousarray(a, dtype=np.float64)
    q, k, v, g, beta = map(c, (q, k, v, g, beta))
    H, T, dk = q.shape
    dv = v.shape[2]
    init = None if init is None else c(init)
    core = np.empty((H, T, dv))
    state = np.empty((H, dk, dv))
    lib().orc_delta_recurrence_f64(H, T, dk, dv, int(l2), _ptr(q), _ptr(k), _ptr(v), _ptr(g),
                                   _ptr(beta), _ptr(init), _ptr(core), _ptr(state))
    return core, state


# ---- collect / last-token ---------------------------------------------------
def prefill_collect(dn_qkv, g_beta, H, T, tok, bufs, dk=128, dv=128):
    qo, ko, vo, go, bo = bufs
    lib().orc_prefill_collect(H, T, tok, dk, dv, _ptr(_u16(dn_qkv)), _ptr(_f32(g_beta)),
                              _ptr(qo), _ptr(ko), _ptr(vo), _ptr(go), _ptr(bo))


def chunk_last_to_fp16(src, H, dv, T, total):
    src = _f32(src)
    dst = np.empty(H * dv, dtype=np.uint16)
    lib().orc_chunk_last_to_fp16(H, dv, T, total, _ptr(src), _ptr(dst))
    return dst


# ---- decode step ------------------------------------------------------------
def decode_step(inp: dict, layer_idx=0, q_scale=None, eps=1e-6):
    """Runs the fused decode step on copies of the mutable inputs; returns
    (qkv, conv_state, state) after the step."""
    qkv = _u16(inp["qkv"]).copy()
    cs = _u16(inp["conv_state"]).copy()
    st = _f32(inp["state"]).copy()
    B = qkv.shape[0]
    nh = inp["a"].shape[1]
    qs = np.float32(1.0) / np.sqrt(np.float32(128.0)) if q_scale is None else q_scale
    lib().orc_decode_step(B, nh, layer_idx, float(qs), float(eps), _ptr(qkv), qkv.shape[1],
                          _ptr(cs), cs.shape[1] * cs.shape[2], _ptr(_u16(inp["conv_w"])),
                          _ptr(_u16(inp["a"])), _ptr(_u16(inp["b"])), nh,
                          _ptr(_f32(inp["a_log_bias"])), _ptr(st), st[0].size,
                          _ptr(_u16(inp["z"])), inp["z"].shape[1], _ptr(_f32(inp["norm_w"])))
    return qkv, cs, st


def conv_l2_qk(qkv, conv_state, conv_w, nh=16):
    """One deltanet_conv_l2_qk step on copies; returns (qkv, conv_state)."""
    qkv = _u16(qkv).copy()
    cs = _u16(conv_state).copy()
    lib().orc_conv_l2_qk(qkv.size, 4, nh * 128, nh, _ptr(qkv), _ptr(cs), _ptr(_u16(conv_w)))
    return qkv, cs


def gbeta(a, b, a_log, dt_bias):
    """(g, beta) per element of equally shaped fp32 arrays (orc_gbeta)."""
    a, b, a_log, dt_bias = (np.broadcast_to(_f32(x), np.broadcast(a, b, a_log, dt_bias).shape).ravel()
                            for x in (a, b, a_log, dt_bias))
    g = np.empty(a.size, np.float32)
    beta = np.empty(a.size, np.float32)
    gp, bp = _c.c_float(), _c.c_float()
    f = lib().orc_gbeta
    for i in range(a.size):
        f(float(a[i]), float(b[i]), float(a_log[i]), float(dt_bias[i]), _c.byref(gp), _c.byref(bp))
        g[i], beta[i] = gp.value, bp.value
    return g, beta


def norm_gate_f16(core, z, norm_w, eps=1e-6):
    """deltanet_norm_gate.comp over fp16 rows core [nh][128] (orc_norm_gate_f16)."""
    io = _u16(core).copy()
    lib().orc_norm_gate_f16(io.size // 128, float(eps), _ptr(io), _ptr(_u16(z)), _ptr(_f32(norm_w)))
    return io


def norm_gate_row(o, z, norm_w, eps=1e-6):
    """The fused decode's gated RMSNorm of one fp32 row of 128 (orc_norm_gate_row)."""
    out = np.empty(128, np.uint16)
    lib().orc_norm_gate_row(_ptr(_f32(o)), _ptr(_u16(z)), _ptr(_f32(norm_w)), float(eps), _ptr(out))
    return out


def recurrent(qkv, state_with_tail, nh=16, q_scale=None):
    qkv = _u16(qkv).copy()
    st = _f32(state_with_tail).copy()
    qs = np.float32(1.0) / np.sqrt(np.float32(128.0)) if q_scale is None else q_scale
    lib().orc_recurrent(nh, float(qs), _ptr(qkv), _ptr(st))
    return qkv, st


# ---- matvec / lm_head / argmax ----------------------------------------------
def matvec_f16(W, x):
    W = _u16(W)
    x = _u16(x)
    y = np.empty(W.shape[0], dtype=np.uint16)
    rc = lib().orc_matvec_f16(_ptr(W), _ptr(x), _ptr(y), W.shape[0], W.shape[1])
    if rc != 0:
        raise RuntimeError("in_dim must be a multiple of 64")
    return y


def matvec_f16_order(W, x, order):
    """order: "spans" (orc_matvec_f16), "strided" or "serial"."""
    if order == "spans":
        return matvec_f16(W, x)
    W = _u16(W)
    x = _u16(x)
    y = np.empty(W.shape[0], dtype=np.uint16)
    fn = {"strided": lib().orc_matvec_f16_strided, "serial": lib().orc_matvec_f16_serial}[order]
    if fn(_ptr(W), _ptr(x), _ptr(y), W.shape[0], W.shape[1]) != 0:
        raise RuntimeError("in_dim must be positive")
    return y


def argmax_f16(vals):
    vals = _u16(vals)
    return int(lib().orc_argmax_f16(_ptr(vals), vals.size))


def lm_head_argmax(W, x):
    W = _u16(W)
    x = _u16(x)
    logits = np.empty(W.shape[0], dtype=np.uint16)
    idx = lib().orc_lm_head_argmax(_ptr(W), _ptr(x), W.shape[0], W.shape[1], _ptr(logits))
    return int(idx), logits
