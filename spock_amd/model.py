"""Python binding of the Qwen3.5-0.8B-shaped decode session
(libspock_hip_host.so, include/spock_model.h): the reference's
DecodeSession(repack_dir) / decode(prompt, max_new) / reset() surface
(src/runtime/vk_session.hpp:22-46).  Host pointers only; the session owns its
device memory.  Loading fails loudly when the library is missing.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HOST_LIB_PATH = Path(__file__).resolve().parent / "libspock_hip_host.so"

_p = C.c_void_p
_i32 = C.c_int32
_sz = C.c_size_t


SPK_MODEL_NO_GRAPH = 1
SPK_MODEL_MATRIX_PREFILL = 2
SPK_MODEL_GPU_TIMESTAMPS = 4
SPK_MODEL_GPU_REGIONS = 8
SPK_MODEL_LMHEAD_ONE_LAUNCH = 16
SPK_MODEL_LMHEAD_KEY_TAKE = 64
SPK_MODEL_SPLIT_DN_STEP = 32


class SpkGenerateStats(C.Structure):
    _fields_ = [("prefill_ms", C.c_double), ("decode_ms", C.c_double), ("gpu_prefill_ms", C.c_double),
                ("gpu_decode_ms", C.c_double), ("decode_steps", _i32), ("used_graph", _i32)]


SIGNATURES = {
    "spk_model_last_error": (C.c_char_p, []),
    "spk_model_open": (_p, [C.c_char_p, _i32, _i32]),
    "spk_model_close": (None, [_p]),
    "spk_model_info": (C.c_int, [_p, _p, _p, _p]),
    "spk_model_reset": (C.c_int, [_p]),
    "spk_model_generate": (C.c_int, [_p, _p, _i32, _i32, _p, _p]),
    "spk_model_gpu_token_us": (C.c_int, [_p, _p, _i32, _p]),
    "spk_model_gpu_region_count": (C.c_int, [_p, _p]),
    "spk_model_gpu_region": (C.c_int, [_p, _i32, _p, _p]),
    "spk_model_prefill": (C.c_int, [_p, _p, _i32, _p]),
    "spk_model_decode": (C.c_int, [_p, _i32, _p]),
    "spk_model_state_sizes": (C.c_int, [_p, _p, _p, _p]),
    "spk_model_get_state": (C.c_int, [_p, _p, _p, _p, _p, _p]),
    "spk_model_set_state": (C.c_int, [_p, _p, _p, _p, _i32, _i32]),
    "spk_model_last_output": (C.c_int, [_p, _p, _p]),
    "spk_artifact_write_synthetic": (C.c_int, [C.c_char_p, _i32, _i32, C.c_uint64]),
}

_LIB = None


class ModelError(RuntimeError):
    pass


def lib():
    global _LIB
    if _LIB is None:
        if not HOST_LIB_PATH.exists():
            raise ModelError(f"{HOST_LIB_PATH} is missing: build it with __graft_entry__.build()")
        l = C.CDLL(str(HOST_LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(l, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = l
    return _LIB


def _check(rc: int, what: str) -> None:
    if rc != 0:
        raise ModelError(f"{what}: {lib().spk_model_last_error().decode(errors='replace')}")


def write_synthetic_artifact(path, layers: int = 24, vocab: int = 248320, seed: int = 0) -> Path:
    """Seeded random-init Qwen3.5-0.8B-shaped artifact (text_repack_manifest.json
    + text_weights.bin)."""
    path = Path(path)
    _check(lib().spk_artifact_write_synthetic(str(path).encode(), layers, vocab, seed),
           "spk_artifact_write_synthetic")
    return path


@dataclass
class GenerateResult:
    tokens: np.ndarray
    prefill_ms: float
    decode_ms: float
    gpu_prefill_ms: float
    gpu_decode_ms: float
    decode_steps: int
    used_graph: bool
    # with gpu_timestamps (DecodeResult::per_token_gpu_us / gpu_region_us)
    per_token_gpu_us: Optional[np.ndarray] = None
    gpu_region_us: Optional[dict] = None


class Session:
    """DecodeSession on one MI355X: construct from a repack directory, then
    generate(prompt, max_new) (= decode()), reset(), prefill/decode steps.
    matrix_prefill=True runs the prompt on the matrix cores; the default runs
    it in the CPU restatement's order (bit-identical).  gpu_timestamps: 0 off,
    1 GPU time per decode step, 2 also per region of the step (layer_i,
    lm_head, argmax; the step's kernels are then launched one by one).
    lm_head_one_launch=False runs the final norm + lm_head + argmax as the key
    launch then the take instead of one launch (same tokens).
    fused_dn_step=False runs each DeltaNet layer's input projections and
    decode step as two launches instead of one (same tokens)."""

    def __init__(self, repack_dir, max_seq: int = 2048, use_graph: bool = True, matrix_prefill: bool = False,
                 gpu_timestamps: int = 0, lm_head_one_launch: bool = True, fused_dn_step: bool = True):
        if gpu_timestamps not in (0, 1, 2):
            raise ModelError(f"gpu_timestamps must be 0, 1 or 2, got {gpu_timestamps}")
        flags = (0 if use_graph else SPK_MODEL_NO_GRAPH) | (SPK_MODEL_MATRIX_PREFILL if matrix_prefill else 0)
        flags |= 0 if lm_head_one_launch else SPK_MODEL_LMHEAD_KEY_TAKE
        flags |= 0 if fused_dn_step else SPK_MODEL_SPLIT_DN_STEP
        flags |= (0, SPK_MODEL_GPU_TIMESTAMPS, SPK_MODEL_GPU_REGIONS)[gpu_timestamps]
        self._h = lib().spk_model_open(str(repack_dir).encode(), max_seq, flags)
        if not self._h:
            raise ModelError(f"spk_model_open: {lib().spk_model_last_error().decode(errors='replace')}")
        layers, vocab, ms = _i32(), _i32(), _i32()
        _check(lib().spk_model_info(self._h, C.byref(layers), C.byref(vocab), C.byref(ms)), "spk_model_info")
        self.layers, self.vocab, self.max_seq = layers.value, vocab.value, ms.value

    def close(self):
        if self._h:
            lib().spk_model_close(self._h)
            self._h = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def reset(self):
        _check(lib().spk_model_reset(self._h), "spk_model_reset")

    def generate(self, prompt: Sequence[int], max_new: int) -> GenerateResult:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        out = np.zeros(max(1, max_new), dtype=np.int32)
        st = SpkGenerateStats()
        _check(lib().spk_model_generate(self._h, p.ctypes.data, len(p), max_new, out.ctypes.data, C.byref(st)),
               "spk_model_generate")
        res = GenerateResult(out[:max_new].copy(), st.prefill_ms, st.decode_ms, st.gpu_prefill_ms,
                             st.gpu_decode_ms, st.decode_steps, bool(st.used_graph))
        n = _i32()
        _check(lib().spk_model_gpu_token_us(self._h, None, 0, C.byref(n)), "spk_model_gpu_token_us")
        if n.value:
            us = np.zeros(n.value, dtype=np.float64)
            _check(lib().spk_model_gpu_token_us(self._h, us.ctypes.data, n.value, C.byref(n)),
                   "spk_model_gpu_token_us")
            res.per_token_gpu_us = us
        _check(lib().spk_model_gpu_region_count(self._h, C.byref(n)), "spk_model_gpu_region_count")
        if n.value:
            regions = {}
            name, us1 = C.c_char_p(), C.c_double()
            for i in range(n.value):
                _check(lib().spk_model_gpu_region(self._h, i, C.byref(name), C.byref(us1)), "spk_model_gpu_region")
                regions[name.value.decode()] = us1.value
            res.gpu_region_us = regions
        return res

    def prefill(self, prompt: Sequence[int]) -> int:
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        tok = _i32()
        _check(lib().spk_model_prefill(self._h, p.ctypes.data, len(p), C.byref(tok)), "spk_model_prefill")
        return tok.value

    def decode(self, n_steps: int) -> np.ndarray:
        out = np.zeros(max(1, n_steps), dtype=np.int32)
        _check(lib().spk_model_decode(self._h, n_steps, out.ctypes.data), "spk_model_decode")
        return out[:n_steps].copy()

    def state_sizes(self):
        a, b, c = _sz(), _sz(), _sz()
        _check(lib().spk_model_state_sizes(self._h, C.byref(a), C.byref(b), C.byref(c)), "spk_model_state_sizes")
        return a.value, b.value, c.value

    def get_state(self):
        a, b, c = self.state_sizes()
        dn = np.zeros(a // 4, dtype=np.float32)
        conv = np.zeros(b // 2, dtype=np.uint16)
        kv = np.zeros(c // 2, dtype=np.uint16)
        pos, tok = _i32(), _i32()
        _check(lib().spk_model_get_state(self._h, dn.ctypes.data, conv.ctypes.data, kv.ctypes.data,
                                         C.byref(pos), C.byref(tok)), "spk_model_get_state")
        return {"dn_state": dn, "conv": conv, "kv": kv, "pos": pos.value, "last_token": tok.value}

    def set_state(self, dn_state: np.ndarray, conv: np.ndarray, kv: np.ndarray, pos: int, last_token: int):
        a, b, c = self.state_sizes()
        dn = np.ascontiguousarray(dn_state, dtype=np.float32)
        cv = np.ascontiguousarray(conv, dtype=np.uint16)
        kvv = np.ascontiguousarray(kv, dtype=np.uint16)
        if dn.nbytes != a or cv.nbytes != b or kvv.nbytes != c:
            raise ModelError("set_state: state sizes do not match the session")
        _check(lib().spk_model_set_state(self._h, dn.ctypes.data, cv.ctypes.data, kvv.ctypes.data, pos, last_token),
               "spk_model_set_state")

    def last_output(self):
        logits = np.zeros(self.vocab, dtype=np.uint16)
        hidden = np.zeros(1024, dtype=np.uint16)
        _check(lib().spk_model_last_output(self._h, logits.ctypes.data, hidden.ctypes.data), "spk_model_last_output")
        return logits, hidden
