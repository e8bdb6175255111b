"""Seeded synthetic inputs for the DeltaNet hot path (host side, numpy).

One portable generator for every tensor: SplitMix64 -> uniform in [0,1) from the
top 53 bits -> Box-Muller in float64 -> float32.  Each tensor gets its own seed,
so CPU and GPU legs, tests and bench.py all see identical inputs.

The shapes and distributions are those of the synthetic configs the bench
reports on (chunk prefill, batched decode step, decode GEMV chain); the
reference's own probes use fixed seeds the same way
(apps/spock-deltanet-chunk-prefill-tiled-probe.cpp:140-160).
"""
from __future__ import annotations

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def splitmix64(seed: int, n: int) -> np.ndarray:
    """n successive SplitMix64 outputs from state `seed` (uint64 array)."""
    with np.errstate(over="ignore"):
        idx = np.arange(1, n + 1, dtype=np.uint64)
        z = np.uint64(seed & 0xFFFFFFFFFFFFFFFF) + idx * _GOLDEN
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
        return z ^ (z >> np.uint64(31))


def uniform(seed: int, n: int, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    u = (splitmix64(seed, n) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    return (lo + u * (hi - lo)).astype(np.float32)


def normal(seed: int, n: int, std: float = 1.0, mean: float = 0.0) -> np.ndarray:
    m = (n + 1) // 2
    u = (splitmix64(seed, 2 * m) >> np.uint64(11)).astype(np.float64) * (1.0 / 9007199254740992.0)
    u1 = 1.0 - u[0::2]  # (0, 1]
    u2 = u[1::2]
    r = np.sqrt(-2.0 * np.log(u1))
    z = np.empty(2 * m, dtype=np.float64)
    z[0::2] = r * np.cos(2.0 * np.pi * u2)
    z[1::2] = r * np.sin(2.0 * np.pi * u2)
    return (mean + std * z[:n]).astype(np.float32)


def softplus64(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.float64)
    return np.where(x > 20.0, x, np.log1p(np.exp(np.minimum(x, 20.0))))


def l2_normalize_rows(x: np.ndarray, eps: float = 1e-6) -> np.ndarray:
    """x / sqrt(sum x^2 + eps) over the last axis, float32 (deltanet_chunk.cpp:27-39)."""
    x = x.astype(np.float32)
    ss = np.sum(x.astype(np.float64) ** 2, axis=-1, keepdims=True)
    return (x / np.sqrt(ss + eps)).astype(np.float32)


def chunk_inputs(H: int, T: int, dk: int = 128, dv: int = 128, seed: int = 0,
                 l2: bool = True) -> dict:
    """Chunk-prefill inputs in the reference layout [H][T][d], g/beta [H][T].

    q, k ~ N(0,1) then L2 per (head, token); v ~ N(0,1);
    g = -softplus(N(0,1)); beta = sigmoid(N(0,1)).
    """
    q = normal(seed * 16 + 1, H * T * dk).reshape(H, T, dk)
    k = normal(seed * 16 + 2, H * T * dk).reshape(H, T, dk)
    v = normal(seed * 16 + 3, H * T * dv).reshape(H, T, dv)
    g = (-softplus64(normal(seed * 16 + 4, H * T))).astype(np.float32).reshape(H, T)
    beta = (1.0 / (1.0 + np.exp(-normal(seed * 16 + 5, H * T).astype(np.float64)))).astype(
        np.float32).reshape(H, T)
    if l2:
        q = l2_normalize_rows(q)
        k = l2_normalize_rows(k)
    return {"q": np.ascontiguousarray(q), "k": np.ascontiguousarray(k),
            "v": np.ascontiguousarray(v), "g": g, "beta": beta}


def ragged_lengths(num_seqs: int, lo: int, hi: int, seed: int) -> np.ndarray:
    u = (splitmix64(seed, num_seqs) % np.uint64(hi - lo + 1)).astype(np.int64)
    return (lo + u).astype(np.int32)


def cu_seqlens_from(lengths) -> np.ndarray:
    cu = np.zeros(len(lengths) + 1, dtype=np.int32)
    cu[1:] = np.cumsum(np.asarray(lengths, dtype=np.int64))
    return cu


def f16(x: np.ndarray) -> np.ndarray:
    """float32 -> IEEE half (round to nearest even), returned as uint16 bits."""
    return np.asarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def decode_inputs(B: int, seed: int = 0, num_heads: int = 16, layers: int = 18) -> dict:
    """Batched decode-step inputs (per-sequence state, conv history, token).

    state fp32 N(0,0.02); conv history fp16 N(0,1) stored [6144][4]
    (channel-major as the reference, vk_session.cpp:365); qkv, z, a, b fp16
    N(0,1); A_log U(-1,1); dt_bias N(0,0.1) rounded through fp16; conv weight
    fp16 N(0,0.02); norm weight 1.0.
    """
    conv_dim = 3 * num_heads * 128
    st = normal(seed * 16 + 1, B * num_heads * 128 * 128, std=0.02).reshape(B, num_heads, 128, 128)
    conv = f16(normal(seed * 16 + 2, B * conv_dim * 4)).reshape(B, conv_dim, 4)
    qkv = f16(normal(seed * 16 + 3, B * conv_dim)).reshape(B, conv_dim)
    z = f16(normal(seed * 16 + 4, B * num_heads * 128)).reshape(B, num_heads * 128)
    a = f16(normal(seed * 16 + 5, B * num_heads)).reshape(B, num_heads)
    b = f16(normal(seed * 16 + 6, B * num_heads)).reshape(B, num_heads)
    a_log = uniform(seed * 16 + 7, layers * num_heads, -1.0, 1.0)
    dt_bias = f16(normal(seed * 16 + 8, layers * num_heads, std=0.1)).view(np.float16).astype(np.float32)
    alb = np.stack([a_log, dt_bias], axis=-1).reshape(layers, num_heads, 2).astype(np.float32)
    conv_w = f16(normal(seed * 16 + 9, conv_dim * 4, std=0.02)).reshape(conv_dim, 4)
    norm_w = np.ones(128, dtype=np.float32)
    return {"state": np.ascontiguousarray(st, dtype=np.float32), "conv_state": conv, "qkv": qkv,
            "z": z, "a": a, "b": b, "a_log_bias": alb, "conv_w": conv_w, "norm_w": norm_w}


def gemv_weights(out_dim: int, in_dim: int, seed: int) -> np.ndarray:
    return f16(normal(seed, out_dim * in_dim, std=0.02)).reshape(out_dim, in_dim)


def gemv_input(n: int, seed: int) -> np.ndarray:
    return f16(normal(seed, n))
