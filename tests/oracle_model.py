"""ctypes binding of the CPU oracle's full-model restatement (oracle/model.h)
over a repacked artifact directory.  TEST INFRASTRUCTURE: imported by tests/,
smoke() and bench.py's cpu_baseline leg only, as the checker."""
from __future__ import annotations

import ctypes as C
import json
from pathlib import Path

import numpy as np

import oracle_lib

_p = C.c_void_p
_i32 = C.c_int32
MAX_LAYERS = 64


class OrcLayer(C.Structure):
    _fields_ = [("kind", _i32), ("sub_idx", _i32)] + [
        (n, _p) for n in ("input_norm", "post_norm", "mlp_gate", "mlp_up", "mlp_down",
                          "dn_qkv", "dn_z", "dn_a", "dn_b", "dn_conv", "dn_out", "dn_dt_bias",
                          "dn_a_log", "dn_norm",
                          "attn_q", "attn_k", "attn_v", "attn_o", "attn_q_norm", "attn_k_norm")]


class OrcModel(C.Structure):
    _fields_ = [("n_layers", _i32), ("vocab", _i32), ("max_seq", _i32), ("n_dn", _i32), ("n_attn", _i32),
                ("pad_", _i32), ("embed", _p), ("final_norm", _p), ("layers", OrcLayer * MAX_LAYERS)]


class OrcModelState(C.Structure):
    _fields_ = [("dn_state", _p), ("conv_state", _p), ("kv_cache", _p), ("a_log_bias", _p), ("rope", _p),
                ("pos", _i32)]


_ROLE_FIELDS = {
    "input_norm": "input_norm", "post_norm": "post_norm", "mlp_gate": "mlp_gate", "mlp_up": "mlp_up",
    "mlp_down": "mlp_down", "delta_in_proj_qkv": "dn_qkv", "delta_in_proj_z": "dn_z",
    "delta_in_proj_a": "dn_a", "delta_in_proj_b": "dn_b", "delta_conv": "dn_conv",
    "delta_out_proj": "dn_out", "delta_dt_bias": "dn_dt_bias", "delta_a_log": "dn_a_log",
    "delta_norm": "dn_norm", "attn_q": "attn_q", "attn_k": "attn_k", "attn_v": "attn_v",
    "attn_o": "attn_o", "attn_q_norm": "attn_q_norm", "attn_k_norm": "attn_k_norm",
}

_LIB = None


def lib():
    global _LIB
    if _LIB is None:
        l = oracle_lib.lib()
        l.orc_model_init_state.restype = None
        l.orc_model_init_state.argtypes = [_p, _p]
        l.orc_model_prefill.restype = C.c_uint32
        l.orc_model_prefill.argtypes = [_p, _p, _p, _i32, _p, _p]
        l.orc_model_decode.restype = C.c_uint32
        l.orc_model_decode.argtypes = [_p, _p, _i32, _p, _p]
        l.orc_model_generate.restype = None
        l.orc_model_generate.argtypes = [_p, _p, _p, _i32, _i32, _p]
        l.orc_model_set_variant.restype = None
        l.orc_model_set_variant.argtypes = [_i32, _i32]
        l.orc_rope_table.restype = None
        l.orc_rope_table.argtypes = [_i32, _p]
        l.orc_rmsnorm1024.restype = None
        l.orc_rmsnorm1024.argtypes = [_p, _p, _p]
        l.orc_head_rmsnorm256.restype = None
        l.orc_head_rmsnorm256.argtypes = [_p, _p, _p]
        l.orc_rope_apply.restype = None
        l.orc_rope_apply.argtypes = [_p, _i32, _p]
        l.orc_attend.restype = None
        l.orc_attend.argtypes = [_p, _p, _i32, _i32, _p]
        for n in ("orc_silu_gate", "orc_sigmoid_gate", "orc_residual_add"):
            getattr(l, n).restype = None
            getattr(l, n).argtypes = [_p, _p, _p, C.c_size_t]
        l.orc_matmul_rows.restype = None
        l.orc_matmul_rows.argtypes = [_p, _p, _p, C.c_size_t, C.c_size_t, C.c_size_t]
        _LIB = l
    return _LIB


def load_artifact(path):
    """(manifest dict, weights memmap uint8, {role: tensor dict})"""
    path = Path(path)
    man = json.loads((path / "text_repack_manifest.json").read_text())
    w = np.memmap(path / "text_weights.bin", dtype=np.uint8, mode="r")
    return man, w, {t["role_path"]: t for t in man["tensors"]}


def tensor(w, t):
    a = w[t["offset"]: t["offset"] + t["nbytes"]]
    return a.view(np.float32 if t["dtype"] == "fp32" else np.uint16).reshape(t["shape"])


class OracleModel:
    """The oracle's model over an artifact, with its own state."""

    def __init__(self, artifact_dir, max_seq: int = 2048):
        self.man, self.w, self.roles = load_artifact(artifact_dir)
        self.n_layers = self.man["model"]["layers"]
        self.vocab = self.man["model"]["vocab"]
        self.max_seq = max_seq
        m = OrcModel()
        m.n_layers, m.vocab, m.max_seq = self.n_layers, self.vocab, max_seq
        base = self.w.ctypes.data if hasattr(self.w, "ctypes") else None
        base = np.frombuffer(self.w, dtype=np.uint8).ctypes.data if base is None else base
        self._base = base
        addr = lambda role: base + self.roles[role]["offset"]
        m.embed = addr("global.token_embedding")
        m.final_norm = addr("global.final_norm")
        n_dn = n_attn = 0
        for L in range(self.n_layers):
            ly = m.layers[L]
            attn = (L % 4 == 3)
            ly.kind = 1 if attn else 0
            ly.sub_idx = n_attn if attn else n_dn
            if attn:
                n_attn += 1
            else:
                n_dn += 1
            for role, field in _ROLE_FIELDS.items():
                key = f"layer.{L}.{role}"
                if key in self.roles:
                    setattr(ly, field, addr(key))
        m.n_dn, m.n_attn = n_dn, n_attn
        self.n_dn, self.n_attn = n_dn, n_attn
        self.model = m
        self.dn_state = np.zeros(max(1, n_dn) * 16 * 128 * 128, dtype=np.float32)
        self.conv = np.zeros(max(1, n_dn) * 6144 * 4, dtype=np.uint16)
        self.kv = np.zeros(max(1, n_attn) * max_seq * 1024, dtype=np.uint16)
        self.alb = np.zeros(max(1, n_dn) * 32, dtype=np.float32)
        self.rope = np.zeros(max_seq * 64, dtype=np.float32)
        st = OrcModelState()
        st.dn_state, st.conv_state, st.kv_cache = self.dn_state.ctypes.data, self.conv.ctypes.data, self.kv.ctypes.data
        st.a_log_bias, st.rope = self.alb.ctypes.data, self.rope.ctypes.data
        self.state = st
        self.reset()

    def reset(self):
        lib().orc_model_init_state(C.byref(self.model), C.byref(self.state))

    @property
    def pos(self):
        return self.state.pos

    def prefill(self, tokens, want_logits=False):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        logits = np.zeros(self.vocab, dtype=np.uint16) if want_logits else None
        hidden = np.zeros(1024, dtype=np.uint16)
        tok = lib().orc_model_prefill(C.byref(self.model), C.byref(self.state), t.ctypes.data, len(t),
                                      None if logits is None else logits.ctypes.data, hidden.ctypes.data)
        return (int(tok), logits, hidden) if want_logits else int(tok)

    def decode(self, token, want_logits=False):
        logits = np.zeros(self.vocab, dtype=np.uint16) if want_logits else None
        hidden = np.zeros(1024, dtype=np.uint16)
        tok = lib().orc_model_decode(C.byref(self.model), C.byref(self.state), int(token),
                                     None if logits is None else logits.ctypes.data, hidden.ctypes.data)
        return (int(tok), logits, hidden) if want_logits else int(tok)

    def generate(self, prompt, n_new):
        self.reset()
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(n_new, dtype=np.int32)
        lib().orc_model_generate(C.byref(self.model), C.byref(self.state), p.ctypes.data, len(p), n_new,
                                 out.ctypes.data)
        return out

    def snapshot(self):
        return {"dn_state": self.dn_state[: self.n_dn * 16 * 128 * 128].copy(),
                "conv": self.conv[: self.n_dn * 6144 * 4].copy(),
                "kv": self.kv[: self.n_attn * self.max_seq * 1024].copy(), "pos": self.pos}


def set_variant(gemm_f64=False, chunk_f64=False):
    lib().orc_model_set_variant(1 if gemm_f64 else 0, 1 if chunk_f64 else 0)
