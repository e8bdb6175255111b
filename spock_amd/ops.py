"""Python host side of the MI355X hot path: thin wrappers that hand device
tensors (torch, ROCm) to the C ABI on the current HIP stream.

torch is only plumbing here (device memory, streams); every computation is a
hand-written gfx950 kernel behind include/spock_hip.h.
"""
from __future__ import annotations

import ctypes as C
from typing import Optional, Sequence

import numpy as np
import torch

from . import _lib
from ._lib import SpkChunkArgs, SpkDecodeArgs, SpkMatvecDesc, check, lib

KEY_DIM = 128
VALUE_DIM = 128
CHUNK = 64


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _dev(t: torch.Tensor, dtype=None) -> torch.Tensor:
    if not t.is_cuda:
        raise _lib.SpockError("expected a device tensor")
    if dtype is not None and t.dtype != dtype:
        raise _lib.SpockError(f"expected {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise _lib.SpockError("expected a contiguous tensor")
    return t


# ----------------------------------------------------------------------------
# chunk prefill
# ----------------------------------------------------------------------------
_CU_CHECKED: dict = {}


def _check_cu_dev(cu_dev: torch.Tensor, cu_host: np.ndarray, dev) -> None:
    """The launch is sized from the host copy; for packs of more than 32
    sequences the kernels find the sequences through the device copy, so the
    two must agree (the kernels keep every access in bounds either way, but a
    differing copy gives wrong results).  The comparison reads the device
    tensor back once per (buffer, torch version counter, host offsets) and is
    cached, so repeated calls stay asynchronous: offsets rewritten behind
    torch's back (through a raw pointer, without a version bump) are not seen
    again, and must not be."""
    if cu_dev.device != dev or cu_dev.dtype != torch.int32 or not cu_dev.is_contiguous():
        raise _lib.SpockError("chunk_prefill: cu_seqlens_dev must be a contiguous int32 tensor on q's device")
    if cu_dev.numel() != cu_host.size:
        raise _lib.SpockError(f"chunk_prefill: cu_seqlens_dev has {cu_dev.numel()} entries, cu_seqlens {cu_host.size}")
    key = (cu_dev.data_ptr(), cu_dev._version, cu_host.tobytes())
    if key in _CU_CHECKED:
        return
    if not np.array_equal(cu_dev.cpu().numpy(), cu_host):
        raise _lib.SpockError("chunk_prefill: cu_seqlens_dev differs from cu_seqlens")
    if len(_CU_CHECKED) > 64:
        _CU_CHECKED.clear()
    _CU_CHECKED[key] = True


def chunk_workspace_bytes(num_heads: int, total_tokens: int, num_seqs: int = 1) -> int:
    return int(lib().spk_chunk_prefill_workspace_size(num_heads, total_tokens, num_seqs, CHUNK))


def chunk_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, g: torch.Tensor,
                  beta: torch.Tensor, initial_state: Optional[torch.Tensor] = None,
                  cu_seqlens: Optional[Sequence[int]] = None, use_qk_l2norm: bool = False,
                  q_scale: float = 0.0, out_core: Optional[torch.Tensor] = None,
                  out_state: Optional[torch.Tensor] = None,
                  workspace: Optional[torch.Tensor] = None, core_head_stride: int = 0,
                  cu_seqlens_dev: Optional[torch.Tensor] = None):
    """Gated-DeltaNet chunk prefill (spk_chunk_prefill).

    q, k: [H][N][128], v: [H][N][128] (float32 or float16, device);
    g, beta: [H][N] float32; cu_seqlens: host sequence offsets (None = one
    sequence; cu_seqlens_dev optionally holds the same offsets already on the
    device, int32).  Returns (core [H][N][128] f32, state [S][H][128][128] f32).
    """
    if q.dim() != 3:
        raise _lib.SpockError(f"chunk_prefill: q must be [H][N][128], got {tuple(q.shape)}")
    H, N, dk = q.shape
    if dk != KEY_DIM:
        raise _lib.SpockError("chunk_prefill: key_dim and value_dim must be 128")
    for name, t in (("k", k), ("v", v)):
        if tuple(t.shape) != (H, N, KEY_DIM):
            raise _lib.SpockError(f"chunk_prefill: {name} shape {tuple(t.shape)} != q shape {(H, N, KEY_DIM)}")
    for name, t in (("g", g), ("beta", beta)):
        if tuple(t.shape) != (H, N):
            raise _lib.SpockError(f"chunk_prefill: {name} shape {tuple(t.shape)} != {(H, N)}")
    dtype = q.dtype
    if dtype not in (torch.float32, torch.float16):
        raise _lib.SpockError("chunk_prefill: q/k/v must be float32 or float16")
    for t in (q, k, v):
        _dev(t, dtype)
    _dev(g, torch.float32)
    _dev(beta, torch.float32)
    dev = q.device
    if cu_seqlens is None:
        S = 1
        cu_dev = None
        cu_host = None
        if cu_seqlens_dev is not None:
            raise _lib.SpockError("chunk_prefill: cu_seqlens_dev given without cu_seqlens")
    else:
        cu_host = np.ascontiguousarray(np.asarray(cu_seqlens, dtype=np.int32))
        S = len(cu_host) - 1
        if cu_seqlens_dev is not None:
            _check_cu_dev(cu_seqlens_dev, cu_host, dev)
            cu_dev = cu_seqlens_dev
        else:
            cu_dev = torch.from_numpy(cu_host.copy()).to(dev)
    state_elems = S * H * KEY_DIM * VALUE_DIM
    if initial_state is not None:
        _dev(initial_state, torch.float32)
        if initial_state.numel() != state_elems:
            raise _lib.SpockError(f"chunk_prefill: initial_state must hold [S={S}][H={H}][128][128] "
                                  f"= {state_elems} floats, got {initial_state.numel()}")
    hs = core_head_stride or N
    if out_core is None:
        if hs != N:
            raise _lib.SpockError("chunk_prefill: core_head_stride needs an out_core buffer")
        out_core = torch.empty((H, N, VALUE_DIM), dtype=torch.float32, device=dev)
    else:
        _dev(out_core, torch.float32)
        if hs < N or out_core.numel() < ((H - 1) * hs + N) * VALUE_DIM:
            raise _lib.SpockError(f"chunk_prefill: out_core holds {out_core.numel()} floats, "
                                  f"rows (h*{hs} + t) for H={H}, N={N} need {((H - 1) * hs + N) * VALUE_DIM}")
    if out_state is None:
        out_state = torch.empty((S, H, KEY_DIM, VALUE_DIM), dtype=torch.float32, device=dev)
    else:
        _dev(out_state, torch.float32)
        if out_state.numel() < state_elems:
            raise _lib.SpockError(f"chunk_prefill: out_state holds {out_state.numel()} floats, need {state_elems}")
    need = chunk_workspace_bytes(H, N, S)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(max(need, 256), dtype=torch.uint8, device=dev)
    a = SpkChunkArgs()
    a.num_heads, a.total_tokens, a.key_dim, a.value_dim, a.chunk_size = H, N, KEY_DIM, VALUE_DIM, CHUNK
    a.use_qk_l2norm = int(bool(use_qk_l2norm))
    a.q_scale = float(q_scale)
    a.input_dtype = _lib.SPK_F32 if dtype == torch.float32 else _lib.SPK_F16
    a.q, a.k, a.v, a.g, a.beta = map(_ptr, (q, k, v, g, beta))
    a.initial_state = _ptr(initial_state)
    a.out_core = _ptr(out_core)
    a.core_head_stride = core_head_stride
    a.out_state = _ptr(out_state)
    a.cu_seqlens = _ptr(cu_dev)
    a.cu_seqlens_host = None if cu_host is None else cu_host.ctypes.data
    a.num_seqs = S
    a.workspace = _ptr(workspace)
    a.workspace_bytes = workspace.numel() * workspace.element_size()
    check(lib().spk_chunk_prefill(C.byref(a), _stream()), "spk_chunk_prefill")
    return out_core, out_state


def prefill_collect(dn_qkv: torch.Tensor, g_beta: torch.Tensor, bufs, seq_len: int, token_idx: int,
                    num_heads: int = 16) -> None:
    qo, ko, vo, go, bo = bufs
    check(lib().spk_prefill_collect(_ptr(dn_qkv), _ptr(g_beta), _ptr(qo), _ptr(ko), _ptr(vo),
                                    _ptr(go), _ptr(bo), num_heads, seq_len, token_idx, KEY_DIM,
                                    VALUE_DIM, _stream()), "spk_prefill_collect")


def chunk_last_to_fp16(src: torch.Tensor, seq_len: int, total_seq: int, num_heads: int = 16,
                       out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty(num_heads * VALUE_DIM, dtype=torch.float16, device=src.device)
    check(lib().spk_chunk_last_to_fp16(_ptr(src), _ptr(out), num_heads, VALUE_DIM, seq_len,
                                       total_seq, _stream()), "spk_chunk_last_to_fp16")
    return out


# ----------------------------------------------------------------------------
# decode step
# ----------------------------------------------------------------------------
_DECODE_FNS = {
    "fused": "spk_deltanet_decode_step",
    "conv_l2_qk": "spk_deltanet_conv_l2_qk",
    "gbeta_norm_gate": "spk_deltanet_recurrent_gbeta_norm_gate",
    "recurrent": "spk_deltanet_recurrent",
}


def decode_step(qkv: torch.Tensor, state: torch.Tensor, conv_state: Optional[torch.Tensor] = None,
                conv_weight: Optional[torch.Tensor] = None, a: Optional[torch.Tensor] = None,
                b: Optional[torch.Tensor] = None, a_log_bias: Optional[torch.Tensor] = None,
                z: Optional[torch.Tensor] = None, norm_weight: Optional[torch.Tensor] = None,
                layer_idx: int = 0, q_scale: float = 0.0, rms_eps: float = 0.0,
                variant: str = "fused", num_heads: int = 16) -> None:
    """In-place batched DeltaNet decode step over the leading batch dim of
    qkv [B][6144] fp16, state [B][...] fp32, conv_state [B][6144][4] fp16,
    a/b [B][16] fp16, z [B][2048] fp16."""
    B = qkv.shape[0]
    d = SpkDecodeArgs()
    d.batch, d.num_heads, d.layer_idx = B, num_heads, layer_idx
    d.q_scale, d.rms_eps = float(q_scale), float(rms_eps)
    d.qkv, d.qkv_stride = _ptr(qkv), qkv[0].numel() if B else 0
    if conv_state is not None:
        d.conv_state, d.conv_state_stride = _ptr(conv_state), conv_state[0].numel()
    d.conv_weight = _ptr(conv_weight)
    if a is not None:
        d.a, d.b, d.ab_stride = _ptr(a), _ptr(b), a[0].numel()
    d.a_log_bias = _ptr(a_log_bias)
    d.state, d.state_stride = _ptr(state), state[0].numel() if B else 0
    if z is not None:
        d.z, d.z_stride = _ptr(z), z[0].numel()
    d.norm_weight = _ptr(norm_weight)
    name = _DECODE_FNS[variant]
    check(getattr(lib(), name)(C.byref(d), _stream()), name)


# ----------------------------------------------------------------------------
# GEMV / lm_head / argmax
# ----------------------------------------------------------------------------
def matvec_f16(W: torch.Tensor, x: torch.Tensor, y: Optional[torch.Tensor] = None) -> torch.Tensor:
    out_dim, in_dim = W.shape
    if y is None:
        y = torch.empty(out_dim, dtype=torch.float16, device=W.device)
    check(lib().spk_matvec_f16(_ptr(W), _ptr(x), _ptr(y), out_dim, in_dim, _stream()),
          "spk_matvec_f16")
    return y


MATVEC_ORDERS = {"spans": 0, "strided": 1, "serial": 2}


def matvec_f16_order(W: torch.Tensor, x: torch.Tensor, order: str,
                     y: Optional[torch.Tensor] = None) -> torch.Tensor:
    """spk_matvec_f16_order: "spans" (lm_head_tiled.comp), "strided"
    (matvec_tiled.comp) or "serial" (matvec.comp) summation order."""
    out_dim, in_dim = W.shape
    if y is None:
        y = torch.empty(out_dim, dtype=torch.float16, device=W.device)
    check(lib().spk_matvec_f16_order(_ptr(W), _ptr(x), _ptr(y), out_dim, in_dim,
                                     MATVEC_ORDERS[order], _stream()),
          "spk_matvec_f16_order")
    return y


def matvec_f16_batched(items) -> None:
    """items: sequence of (W, x, y) device tensors; one call."""
    arr = (SpkMatvecDesc * len(items))()
    for i, (W, x, y) in enumerate(items):
        arr[i].W, arr[i].x, arr[i].y = _ptr(W), _ptr(x), _ptr(y)
        arr[i].out_dim, arr[i].in_dim = W.shape[0], W.shape[1]
    check(lib().spk_matvec_f16_batched(arr, len(items), _stream()), "spk_matvec_f16_batched")


def argmax_f16(vals: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=vals.device)
    check(lib().spk_argmax_f16(_ptr(vals), vals.numel(), _ptr(out), _stream()), "spk_argmax_f16")
    return out


def lm_head_workspace_bytes(vocab: int) -> int:
    return int(lib().spk_lm_head_workspace_size(vocab))


def lm_head_argmax(W: torch.Tensor, x: torch.Tensor, logits: Optional[torch.Tensor] = None,
                   out: Optional[torch.Tensor] = None,
                   workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
    vocab, hidden = W.shape
    if out is None:
        out = torch.empty(1, dtype=torch.int32, device=W.device)
    need = lm_head_workspace_bytes(vocab)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=W.device)
    check(lib().spk_lm_head_argmax(_ptr(W), _ptr(x), vocab, hidden, _ptr(logits), _ptr(out),
                                   _ptr(workspace), workspace.numel() * workspace.element_size(),
                                   _stream()), "spk_lm_head_argmax")
    return out
