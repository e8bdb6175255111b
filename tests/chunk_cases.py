"""Deterministic chunk-rule test cases (inputs regenerated bit-for-bit).

Probe cases restate the table of apps/spock-deltanet-chunk-prefill-probe.cpp:62-84
(name, heads, seq_len, k_dim, v_dim, chunk, value ranges, generator flags) and
its input generators (:213-298): xorshift32 `bounded_rand` with the fixed seeds
0xDEADBEEF/0xCAFEBABE/0xDECAFBAD/0xABADCAFE/0xBEEFCACE, the linear `bounded`
ramp, per-head repetition, and the probe's L2 step (x /= sqrt(sum x^2 + 1e-6)).
All arithmetic is float32 in the probe's operation order, so inputs are exact.
"config0" is the north-star config 0 (H=16, T=104, seeded N(0,1) data).
"""
from __future__ import annotations

import hashlib

import numpy as np

from spock_amd import synth

_SEEDS = (0xDEADBEEF, 0xCAFEBABE, 0xDECAFBAD, 0xABADCAFE, 0xBEEFCACE)


def _spec(H, T, dk, dv, C, q, k, v, g, b, repeat=False, prandom=False, l2=False):
    return {"H": H, "T": T, "dk": dk, "dv": dv, "C": C, "q": q, "k": k, "v": v, "g": g,
            "beta": b, "repeat": repeat, "prandom": prandom, "l2": l2}


CASES = {
    "real-width": _spec(1, 4, 128, 128, 4, (-0.01, 0.01), (-0.01, 0.01), (-0.01, 0.01),
                        (-0.04, -0.01), (0.1, 0.4)),
    "real-chunk": _spec(1, 64, 128, 128, 64, (-0.005, 0.005), (-0.005, 0.005), (-0.005, 0.005),
                        (-0.015, -0.002), (0.05, 0.2)),
    "two-chunks": _spec(1, 128, 128, 128, 64, (-0.003, 0.003), (-0.003, 0.003), (-0.003, 0.003),
                        (-0.012, -0.0015), (0.04, 0.16)),
    "multi-head": _spec(16, 64, 128, 128, 64, (-0.002, 0.002), (-0.002, 0.002), (-0.002, 0.002),
                        (-0.010, -0.001), (0.03, 0.12)),
    "multi-head-repeat": _spec(16, 64, 128, 128, 64, (-0.002, 0.002), (-0.002, 0.002),
                               (-0.002, 0.002), (-0.010, -0.001), (0.03, 0.12), repeat=True),
    "multi-head-padded": _spec(16, 104, 128, 128, 64, (-0.002, 0.002), (-0.002, 0.002),
                               (-0.002, 0.002), (-0.010, -0.001), (0.03, 0.12)),
    "runtime-range-padded": _spec(16, 104, 128, 128, 64, (-1.0, 1.0), (-1.0, 1.0), (-20.0, 20.0),
                                  (-9.0, -1e-6), (0.0, 1.0), prandom=True),
    "runtime-l2-padded": _spec(16, 104, 128, 128, 64, (-1.0, 1.0), (-1.0, 1.0), (-20.0, 20.0),
                               (-9.0, -1e-6), (0.0, 1.0), prandom=True, l2=True),
    "config0": {"H": 16, "T": 104, "dk": 128, "dv": 128, "C": 64, "synth_seed": 0},
}


def xorshift32_stream(seed: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.uint32)
    s = seed & 0xFFFFFFFF
    for i in range(n):
        s ^= (s << 13) & 0xFFFFFFFF
        s ^= s >> 17
        s ^= (s << 5) & 0xFFFFFFFF
        out[i] = s
    return out


def bounded_rand(n, lo, hi, seed):
    t = xorshift32_stream(seed, n).astype(np.float32) * np.float32(1.0 / 4294967296.0)
    lo32, hi32 = np.float32(lo), np.float32(hi)
    return (lo32 + t * (hi32 - lo32)).astype(np.float32)


def bounded(n, lo, hi):
    lo32, hi32 = np.float32(lo), np.float32(hi)
    if n == 1:
        return np.array([lo32], dtype=np.float32)
    step = (hi32 - lo32) / np.float32(n - 1)
    return (lo32 + step * np.arange(n, dtype=np.float32)).astype(np.float32)


def _probe_l2(x, H, T, d):
    x = x.reshape(H, T, d)
    nrm = np.cumsum(x * x, axis=-1, dtype=np.float32)[..., -1]  # sequential float32 sum
    nrm = np.sqrt(nrm + np.float32(1e-6)).astype(np.float32)
    return (x / nrm[..., None]).astype(np.float32).reshape(-1)


def make_inputs(name: str) -> dict:
    spec = CASES[name]
    H, T, dk, dv = spec["H"], spec["T"], spec["dk"], spec["dv"]
    if "synth_seed" in spec:
        return synth.chunk_inputs(H, T, dk, dv, seed=spec["synth_seed"])
    if spec["prandom"]:
        q = bounded_rand(H * T * dk, *spec["q"], _SEEDS[0])
        k = bounded_rand(H * T * dk, *spec["k"], _SEEDS[1])
        v = bounded_rand(H * T * dv, *spec["v"], _SEEDS[2])
        g = bounded_rand(H * T, *spec["g"], _SEEDS[3])
        b = bounded_rand(H * T, *spec["beta"], _SEEDS[4])
        if spec["l2"]:
            q = _probe_l2(q, H, T, dk)
            k = _probe_l2(k, H, T, dk)
    elif spec["repeat"]:
        q = np.tile(bounded(T * dk, *spec["q"]), H)
        k = np.tile(bounded(T * dk, *spec["k"]), H)
        v = np.tile(bounded(T * dv, *spec["v"]), H)
        g = np.tile(bounded(T, *spec["g"]), H)
        b = np.tile(bounded(T, *spec["beta"]), H)
    else:
        q = bounded(H * T * dk, *spec["q"])
        k = bounded(H * T * dk, *spec["k"])
        v = bounded(H * T * dv, *spec["v"])
        g = bounded(H * T, *spec["g"])
        b = bounded(H * T, *spec["beta"])
    return {"q": q.reshape(H, T, dk), "k": k.reshape(H, T, dk), "v": v.reshape(H, T, dv),
            "g": g.reshape(H, T), "beta": b.reshape(H, T)}


def inputs_digest(inp: dict) -> str:
    h = hashlib.sha256()
    for key in ("q", "k", "v", "g", "beta"):
        h.update(np.ascontiguousarray(inp[key], dtype=np.float32).tobytes())
    return h.hexdigest()
