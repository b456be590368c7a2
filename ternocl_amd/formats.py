"""Host-side weight formats (numpy): the packers that sit before the kernels.

* int2: ``uint32 [K/16, N]``, word (kp, n) bits 2j..2j+1 = code of row 16kp+j,
  codes {0, 1, 3} = {0, +1, -1} (int2_fp16_upcvt/int2_fp16_upcvt.cl:6-19).
* BITCOS: one uint32 buffer, bitmap [K/32][N] | offsets [N] | per-column sign
  streams (1 = -1, tail bits zero) | 4 pad words (common/bitcos.hpp:1-27), and
  slice ranks [LS-1][N] (common/bitcos.hpp:81-94).
* DT: fp16 / bf16 raw bits (uint16), converted with round-to-nearest-even
  (bf16 NaN quieted as common/dt16.hpp:34).
"""
from __future__ import annotations

import numpy as np

BITCOS_PAD = 4  # common/bitcos.hpp:27


# ---- DT ----------------------------------------------------------------------

def f32_to_dt(x, bf16: bool) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    if not bf16:
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r = np.where(nan, ((u >> 16) | 0x40) & 0xFFFF, r)
    return r.astype(np.uint16)


def dt_to_f32(h, bf16: bool) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    if not bf16:
        return h.view(np.float16).astype(np.float32)
    return (h.astype(np.uint32) << 16).view(np.float32)


# ---- int2 --------------------------------------------------------------------

_CODE_OF = {0: 0, 1: 1, -1: 3}


def pack_int2(codes) -> np.ndarray:
    """codes int8 [K, N] in {-1, 0, +1} -> B uint32 [K/16, N]."""
    codes = np.asarray(codes)
    K, N = codes.shape
    if K % 16:
        raise ValueError("K must be a multiple of 16")
    c = np.where(codes < 0, 3, codes).astype(np.uint32).reshape(K // 16, 16, N)
    sh = (2 * np.arange(16, dtype=np.uint32))[None, :, None]
    return np.bitwise_or.reduce(c << sh, axis=1).astype(np.uint32)


def unpack_int2(B, K: int) -> np.ndarray:
    """B uint32 [K/16, N] -> int8 [K, N] signed values (2-bit two's complement:
    code 2 reads as -2, as code_to_value of int2_fp16_upcvt/main.cpp:76)."""
    B = np.asarray(B, dtype=np.uint32)
    sh = (2 * np.arange(16, dtype=np.uint32))[None, :, None]
    c = ((B[:, None, :] >> sh) & 3).astype(np.int8)
    v = np.where(c >= 2, c - 4, c).astype(np.int8)
    return v.reshape(K, B.shape[1])


# ---- BITCOS ------------------------------------------------------------------

def bitcos_pack(codes) -> np.ndarray:
    """codes int8 [K, N] in {-1, 0, +1} -> BITCOS buffer (uint32)."""
    codes = np.asarray(codes, dtype=np.int8)
    K, N = codes.shape
    if K % 32:
        raise ValueError("K must be a multiple of 32")
    nz = codes != 0
    bits = nz.reshape(K // 32, 32, N).astype(np.uint64)
    bitmap = (bits << np.arange(32, dtype=np.uint64)[None, :, None]).sum(axis=1).astype(np.uint32)
    nnz = nz.sum(axis=0).astype(np.int64)
    words = (nnz + 31) // 32
    off = np.concatenate([[0], np.cumsum(words)[:-1]]).astype(np.uint32)
    total_signs = int(words.sum())
    signs = np.zeros(total_signs, np.uint32)
    neg = codes < 0
    for n in range(N):  # column-major sign streams
        s = neg[nz[:, n], n]
        if s.size:
            padded = np.zeros(words[n] * 32, np.uint8)
            padded[: s.size] = s
            w = np.packbits(padded.reshape(-1, 32)[:, ::-1], axis=1).view(">u4").astype(np.uint32)
            signs[off[n]: off[n] + words[n]] = w.ravel()
    return np.concatenate([bitmap.ravel(), off, signs, np.zeros(BITCOS_PAD, np.uint32)])


def bitcos_slice_ranks(buf, K: int, N: int, ls: int) -> np.ndarray:
    """Non-zeros of column n above each slice boundary s*ceil(K/ls) (s = 1..ls-1),
    counted over whole 32-row bitmap words, as common/bitcos.hpp:81-94."""
    if ls <= 1:
        return np.zeros(0, np.uint32)
    bm = np.asarray(buf[: K // 32 * N], dtype=np.uint32).reshape(K // 32, N)
    pc = np.unpackbits(bm.view(np.uint8).reshape(K // 32, N, 4), axis=2).sum(axis=2)
    csum = np.concatenate([np.zeros((1, N), np.int64), np.cumsum(pc, axis=0)])
    slice_k = (K + ls - 1) // ls
    rows = [csum[(s * slice_k) // 32] for s in range(1, ls)]
    return np.stack(rows).astype(np.uint32).ravel()


def bitcos_bytes(buf) -> int:
    return int(np.asarray(buf).size) * 4
