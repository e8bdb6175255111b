"""ctypes binding of the gfx950 library's C ABI (include/spock_hip.h).

Loading fails loudly when libspock_hip.so is missing: there is no CPU
fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libspock_hip.so"

_p = C.c_void_p
_i32 = C.c_int32
_i64 = C.c_int64
_f32 = C.c_float
_sz = C.c_size_t

# Exported entry points and their C signatures (restype, argtypes).
SIGNATURES = {
    "spk_last_error": (C.c_char_p, []),
    "spk_abi_version": (C.c_uint32, []),
    "spk_chunk_prefill_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "spk_chunk_prefill": (C.c_int, [_p, _p]),
    "spk_prefill_collect": (C.c_int, [_p] * 7 + [_i32] * 5 + [_p]),
    "spk_chunk_last_to_fp16": (C.c_int, [_p, _p] + [_i32] * 4 + [_p]),
    "spk_deltanet_decode_step": (C.c_int, [_p, _p]),
    "spk_deltanet_conv_l2_qk": (C.c_int, [_p, _p]),
    "spk_deltanet_recurrent_gbeta_norm_gate": (C.c_int, [_p, _p]),
    "spk_deltanet_recurrent": (C.c_int, [_p, _p]),
    "spk_matvec_f16": (C.c_int, [_p, _p, _p, _i32, _i32, _p]),
    "spk_matvec_f16_batched": (C.c_int, [_p, _i32, _p]),
    "spk_matvec_f16_order": (C.c_int, [_p, _p, _p, _i32, _i32, _i32, _p]),
    "spk_argmax_f16": (C.c_int, [_p, _i32, _p, _p]),
    "spk_lm_head_workspace_size": (_sz, [_i32]),
    "spk_lm_head_argmax": (C.c_int, [_p, _p, _i32, _i32, _p, _p, _p, _sz, _p]),
    "spk_lm_head_argmax_noalloc": (C.c_int, [_p, _p, _i32, _i32, _p, _p, _p]),
    "spk_selftest_numerics": (C.c_int, [_p, _i32, _p, _p]),
    "spk_selftest_mfma_peak": (C.c_int, [_i32, _i32, _p, _p]),
    "spk_selftest_xcc_ids": (C.c_int, [_i32, _p, _p]),
    "spk_selftest_stream_read": (C.c_int, [_p, _sz, _i32, _i32, _p, _p]),
    # Qwen3.5 model kernels
    "spk_gemv_fused": (C.c_int, [_p, _p, _i32, _p]),
    "spk_attention_workspace_size": (_sz, [_i32, _i32]),
    "spk_attention_decode": (C.c_int, [_p, _p]),
    "spk_attention_prefill": (C.c_int, [_p, _i32, _i32, _p]),
    "spk_attention_decode_oproj": (C.c_int, [_p, _p, _p]),
    "spk_rmsnorm_f16": (C.c_int, [_p, _p, _p, _i32, _i32, _p]),
    "spk_silu_gate_f16": (C.c_int, [_p, _p, _p, _i64, _p]),
    "spk_residual_add_f16": (C.c_int, [_p, _p, _p, _i64, _p]),
    "spk_embedding_f16": (C.c_int, [_p, _p, _i32, _i32, _p, _p]),
    "spk_add_i32": (C.c_int, [_p, _i32, _p]),
    "spk_record_token": (C.c_int, [_p, _p, _p, _p, _i32, _p]),
    "spk_lm_head_argmax_key": (C.c_int, [_p, _p, _p, _i32, _i32, _p, _p, _p]),
    "spk_argmax_key_take": (C.c_int, [_p, _i32, _p, _p, _p, _p, _i32, _p]),
    "spk_lm_head_take_slots": (_sz, [_i32]),
    "spk_lm_head_argmax_take": (C.c_int, [_p, _p, _p, _i32, _i32, _p, _p, _sz, _p, _p, _p, _p, _i32, _p]),
    "spk_gemm_f16": (C.c_int, [_p, _i64, _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _p]),
    "spk_deltanet_prefill_conv": (C.c_int, [_p, _i64, _p, _p, _i32, _p, _p, _p, _p]),
    "spk_deltanet_prefill_gbeta": (C.c_int, [_p, _p, _i64, _p, _i32, _i32, _p, _p, _p]),
    "spk_deltanet_norm_gate": (C.c_int, [_p, _i64, _p, _i64, _p, _f32, _i32, _p, _i64, _p]),
    "spk_deltanet_norm_gate_f16": (C.c_int, [_p, _p, _p, _i32, _i32, _f32, _p]),
    "spk_deltanet_inproj_step": (C.c_int, [_p, _p, _p, _p, _p]),
    "spk_attention_inproj": (C.c_int, [_p, _p, _p, _p]),
    "spk_matvec_f16_rows": (C.c_int, [_p, _p, _i64, _p, _i64, _p, _i32, _i32, _i32, _p]),
    "spk_chunk_prefill_ordered_workspace_size": (_sz, [_i32, _i32]),
    "spk_chunk_prefill_ordered": (C.c_int, [_p, _p]),
}


class SpkChunkArgs(C.Structure):
    _fields_ = [
        ("num_heads", _i32), ("total_tokens", _i32), ("key_dim", _i32), ("value_dim", _i32),
        ("chunk_size", _i32), ("use_qk_l2norm", _i32), ("q_scale", _f32), ("input_dtype", _i32),
        ("q", _p), ("k", _p), ("v", _p), ("g", _p), ("beta", _p), ("initial_state", _p),
        ("out_core", _p), ("core_head_stride", _i64), ("out_state", _p),
        ("cu_seqlens", _p), ("cu_seqlens_host", _p), ("num_seqs", _i32),
        ("workspace", _p), ("workspace_bytes", _sz),
    ]


class SpkDecodeArgs(C.Structure):
    _fields_ = [
        ("batch", _i32), ("num_heads", _i32), ("layer_idx", _i32), ("q_scale", _f32),
        ("rms_eps", _f32),
        ("qkv", _p), ("qkv_stride", _i64),
        ("conv_state", _p), ("conv_state_stride", _i64),
        ("conv_weight", _p),
        ("a", _p), ("b", _p), ("ab_stride", _i64),
        ("a_log_bias", _p),
        ("state", _p), ("state_stride", _i64),
        ("z", _p), ("z_stride", _i64),
        ("norm_weight", _p),
    ]


SPK_GEMV_IN_PLAIN, SPK_GEMV_IN_RMSNORM, SPK_GEMV_IN_SILU_GATE = 0, 1, 2


class SpkGemvInput(C.Structure):
    _fields_ = [("kind", _i32), ("in_dim", _i32), ("x", _p), ("x2", _p), ("token", _p),
                ("token_rows", _i32), ("h_out", _p)]


class SpkGemvOutput(C.Structure):
    _fields_ = [("W", _p), ("y", _p), ("residual", _p), ("out_dim", _i32), ("W_up", _p)]


class SpkAttnArgs(C.Structure):
    _fields_ = [("qg", _p), ("k", _p), ("v", _p), ("q_norm_w", _p), ("k_norm_w", _p), ("rope", _p),
                ("kv_cache", _p), ("max_seq", _i32), ("pos_dev", _p), ("out", _p), ("workspace", _p),
                ("workspace_bytes", _sz)]


class SpkMatvecDesc(C.Structure):
    _fields_ = [("W", _p), ("x", _p), ("y", _p), ("out_dim", _i32), ("in_dim", _i32)]


SPK_F32 = 0
SPK_F16 = 1

_LIB = None


class SpockError(RuntimeError):
    pass


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            raise SpockError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                             "(there is no CPU fallback)")
        l = C.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = l
    return _LIB


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().spk_last_error().decode(errors="replace")
        raise SpockError(f"{what} failed ({rc}): {msg}")
