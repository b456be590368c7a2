"""Seeded synthetic inputs of the benchmark workloads (numpy, CPU).

All draws come from ``numpy.random.Generator(PCG64(seed))``, so the same seed
gives the same bits regardless of thread count.  Distributions:

* activations ~ N(0, 1), rounded RTE to the DT;
* ternary weights with p(-1, 0, +1) = (0.25, 0.5, 0.25), drawn bitwise as the
  reference drivers do (int2_fp16_upcvt/main.cpp:238-242: low bit = r1,
  high bit = r1 & r2, per 2-bit field) -> codes {0, 1, 3};
* per-128-group scales ~ U[0.005, 0.02];
* BITCOS weights at zero density z, non-zeros +/-1 equiprobable;
* MoE routing: each token picks topk distinct experts uniformly at random; its
  gate weights are the softmax of topk logits ~N(0, 1) (fp32, then DT).
"""
from __future__ import annotations

import numpy as np

from .formats import bitcos_pack, f32_to_dt

_M55 = np.uint32(0x55555555)


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def activations(g: np.random.Generator, shape, bf16: bool, sigma: float = 1.0) -> np.ndarray:
    return f32_to_dt(g.standard_normal(shape, dtype=np.float32) * np.float32(sigma), bf16)


def int2_weights(g: np.random.Generator, K: int, N: int) -> np.ndarray:
    """B uint32 [K/16, N], codes {0: 1/2, 1: 1/4, 3: 1/4}."""
    r1 = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    r2 = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    lo = r1 & _M55
    hi = (r1 & r2) & _M55
    return lo | (hi << np.uint32(1))


def scales(g: np.random.Generator, K: int, N: int, bf16: bool, lo=0.005, hi=0.02) -> np.ndarray:
    return f32_to_dt(g.uniform(lo, hi, size=(K // 128, N)).astype(np.float32), bf16)


def ternary_codes(g: np.random.Generator, K: int, N: int, z: float) -> np.ndarray:
    """int8 [K, N]: 0 with probability z, else +/-1 equiprobable."""
    u = g.random((K, N), dtype=np.float32)
    s = g.integers(0, 2, size=(K, N), dtype=np.int8) * 2 - 1
    return np.where(u < z, 0, s).astype(np.int8)


def bitcos_weights(g: np.random.Generator, K: int, N: int, z: float):
    codes = ternary_codes(g, K, N, z)
    return bitcos_pack(codes), codes


def moe_routing(g: np.random.Generator, T: int, E: int, topk: int, bf16: bool):
    """ids int32 [T*topk] (distinct experts per token, uniform) and RW DT [T*topk]."""
    ids = np.argsort(g.random((T, E), dtype=np.float32), axis=1)[:, :topk].astype(np.int32)
    logits = g.standard_normal((T, topk), dtype=np.float32)
    w = np.exp(logits - logits.max(axis=1, keepdims=True))
    w = (w / w.sum(axis=1, keepdims=True)).astype(np.float32)
    return ids.reshape(-1), f32_to_dt(w.reshape(-1), bf16)
