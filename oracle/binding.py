"""numpy wrappers of the CPU oracle (test infrastructure only).

``orc`` functions wrap ``liboracle.so`` (the C restatement); ``ref`` functions
wrap ``_ref/libternocl_ref.so`` (the reference's own host code), which exists
only where it was built from a reference tree (``ref_available()``).
DT arrays are ``np.uint16`` raw bits; ``bf16`` selects bf16 over fp16.
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ORC_PATH = HERE / "liboracle.so"
REF_PATH = HERE / "_ref" / "libternocl_ref.so"

_orc = None
_ref = None


def build_oracle() -> None:
    """Compile the C oracle (and the reference shim where the tree exists)."""
    subprocess.run(["make", "-s", "-C", str(HERE), "all"], check=True)


def _p(a):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def orc() -> C.CDLL:
    global _orc
    if _orc is None:
        if not ORC_PATH.exists():
            build_oracle()
        _orc = C.CDLL(str(ORC_PATH))
        _orc.orc_tof.restype = C.c_float
        _orc.orc_tof.argtypes = [C.c_uint16, C.c_int]
        _orc.orc_fromf.restype = C.c_uint16
        _orc.orc_fromf.argtypes = [C.c_float, C.c_int]
        _orc.orc_sigmoid.restype = C.c_float
        _orc.orc_sigmoid.argtypes = [C.c_float]
        _orc.orc_fwht_scale.restype = C.c_float
        _orc.orc_bitcos_words.restype = C.c_size_t
        _orc.orc_bitcos_pack.restype = C.c_size_t
        _orc.orc_fwht.restype = C.c_int
        _orc.orc_ldsa.restype = C.c_int
    return _orc


def ref_available() -> bool:
    return REF_PATH.exists()


def ref() -> C.CDLL:
    global _ref
    if _ref is None:
        _ref = C.CDLL(str(REF_PATH))
        _ref.ref_tof.restype = C.c_float
        _ref.ref_tof.argtypes = [C.c_uint16]
        _ref.ref_fromf.restype = C.c_uint16
        _ref.ref_fromf.argtypes = [C.c_float]
        _ref.ref_sigmoid.restype = C.c_float
        _ref.ref_sigmoid.argtypes = [C.c_float]
        _ref.ref_bitcos_random_words.restype = C.c_size_t
        _ref.ref_bitcos_random_words.argtypes = [C.c_int, C.c_int, C.c_double, C.c_uint64]
        _ref.ref_bitcos_random.argtypes = [C.c_int, C.c_int, C.c_double, C.c_uint64, C.c_void_p]
        _ref.ref_bitcos_slice_ranks.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_void_p]
        _ref.ref_bitcos_decode_col.argtypes = [C.c_void_p, C.c_size_t, C.c_int, C.c_int, C.c_int, C.c_void_p]
        _ref.ref_bitcos_gold.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_void_p, C.c_void_p,
                                         C.c_int, C.c_int, C.c_int]
    return _ref


def _u16(a):
    return np.ascontiguousarray(a, dtype=np.uint16)


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


# ---- conversions -----------------------------------------------------------

def tof(h, bf16: bool) -> np.ndarray:
    h = _u16(h)
    f = np.empty(h.shape, np.float32)
    orc().orc_tof_n(_p(h), _p(f), C.c_size_t(h.size), int(bf16))
    return f


def fromf(f, bf16: bool) -> np.ndarray:
    f = np.ascontiguousarray(f, dtype=np.float32)
    h = np.empty(f.shape, np.uint16)
    orc().orc_fromf_n(_p(f), _p(h), C.c_size_t(f.size), int(bf16))
    return h


# ---- int2 ------------------------------------------------------------------

def int2_gold(A, B, S, M, K, N, bf16: bool) -> np.ndarray:
    C_ = np.empty((M, N), np.float32)
    orc().orc_int2_gold(int(bf16), _p(_u16(A)), _p(_u32(B)), _p(_u16(S)), _p(C_), M, K, N)
    return C_


def int2_dequant(B, S, K, N) -> np.ndarray:
    W = np.empty((K, N), np.uint16)
    orc().orc_int2_dequant(_p(_u32(B)), _p(_u16(S)), _p(W), K, N)
    return W


def epilogue(acc, other, bias, postop: int, out_f32: bool, bf16: bool) -> np.ndarray:
    acc = np.ascontiguousarray(acc, np.float32)
    M, N = acc.shape
    out = np.empty((M, N), np.float32 if out_f32 else np.uint16)
    o = None if other is None else _u16(other)
    b = None if bias is None else np.ascontiguousarray(bias)
    orc().orc_epilogue(int(bf16), postop, int(out_f32), _p(acc), _p(o), _p(b), _p(out), M, N)
    return out


# ---- int8 ------------------------------------------------------------------

def ldsa(M: int) -> int:
    return (M + 31) & ~31


def scale_a(A, M, K, bf16: bool) -> np.ndarray:
    SA = np.zeros((K // 128, ldsa(M)), np.uint16)
    orc().orc_scale_a(int(bf16), _p(_u16(A)), _p(SA), M, K)
    return SA


def quant_a(A, SA, M, K, bf16: bool) -> np.ndarray:
    Aq = np.empty((M, K), np.int8)
    orc().orc_quant_a(int(bf16), _p(_u16(A)), _p(_u16(SA)), _p(Aq), M, K)
    return Aq


def int8_gold(A, B, SA, SB, M, K, N, bf16: bool) -> np.ndarray:
    C_ = np.empty((M, N), np.float32)
    orc().orc_int8_gold(int(bf16), _p(_u16(A)), _p(_u32(B)), _p(_u16(SA)), _p(_u16(SB)), _p(C_), M, K, N)
    return C_


# ---- BITCOS ----------------------------------------------------------------

def bitcos_pack(codes) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.int8)
    K, N = codes.shape
    n = orc().orc_bitcos_words(_p(codes), K, N)
    buf = np.empty(n, np.uint32)
    orc().orc_bitcos_pack(_p(codes), K, N, _p(buf))
    return buf


def bitcos_slice_ranks(buf, K, N, ls) -> np.ndarray:
    sr = np.zeros(max(ls - 1, 0) * N, np.uint32)
    if ls > 1:
        orc().orc_bitcos_slice_ranks(_p(_u32(buf)), K, N, ls, _p(sr))
    return sr


def bitcos_decode(buf, K, N) -> np.ndarray:
    out = np.empty((K, N), np.int8)
    col = np.empty(K, np.int8)
    b = _u32(buf)
    for n in range(N):
        orc().orc_bitcos_decode_col(_p(b), K, N, n, _p(col))
        out[:, n] = col
    return out


def bitcos_gold(A, buf, S, M, K, N, bf16: bool) -> np.ndarray:
    C_ = np.empty((M, N), np.float32)
    orc().orc_bitcos_gold(int(bf16), _p(_u16(A)), _p(_u32(buf)), _p(_u16(S)), _p(C_), M, K, N)
    return C_


def bitcos_dequant(buf, S, K, N) -> np.ndarray:
    W = np.empty((K, N), np.uint16)
    orc().orc_bitcos_dequant(_p(_u32(buf)), _p(_u16(S)), _p(W), K, N)
    return W


# ---- FWHT ------------------------------------------------------------------

def fwht(x, signs, rows, K, HB, use_signs: bool, bf16: bool) -> np.ndarray:
    y = np.empty((rows, K), np.uint16)
    s = None if signs is None else np.ascontiguousarray(signs, np.int8)
    rc = orc().orc_fwht(int(bf16), _p(_u16(x)), _p(s), _p(y), rows, K, HB, int(use_signs))
    if rc != 0:
        raise ValueError("orc_fwht: unsupported HB / K")
    return y


def fwht_scale(n: int) -> float:
    return orc().orc_fwht_scale(n)


# ---- MoE -------------------------------------------------------------------

def moe_route(ids, E, rows_per_tile):
    ids = np.ascontiguousarray(ids, np.int32)
    G = ids.size
    meta = np.empty(2 * E + 2, np.int32)
    perm = np.empty(G, np.int32)
    inv = np.empty(G, np.int32)
    orc().orc_moe_route(_p(ids), G, E, rows_per_tile, _p(meta), _p(perm), _p(inv))
    return meta, perm, inv


def moe_gather(X, perm, topk):
    X = _u16(X)
    T, K = X.shape
    perm = np.ascontiguousarray(perm, np.int32)
    Xs = np.empty((perm.size, K), np.uint16)
    orc().orc_moe_gather(_p(X), _p(perm), _p(Xs), perm.size, K, topk)
    return Xs


def moe_combine(Y, inv, RW, T, topk, N, bf16: bool):
    O = np.empty((T, N), np.uint16)
    orc().orc_moe_combine(int(bf16), _p(np.ascontiguousarray(Y, np.float32)),
                          _p(np.ascontiguousarray(inv, np.int32)), _p(_u16(RW)), _p(O), T, topk, N)
    return O


def moe_ref_tokens(X, ids, RW, T0, T1, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16: bool,
                   round_up: bool = True):
    """round_up: the prefill check (up rounded to DT first, int2_moe/prefill.cpp:306);
    False: the decode check (int2_moe/main.cpp:280)."""
    O = np.empty((T1 - T0, H), np.float64)
    orc().orc_moe_ref_tokens(int(bf16), _p(_u16(X)), _p(np.ascontiguousarray(ids, np.int32)),
                             _p(_u16(RW)), T0, T1, topk, H, I, _p(_u32(Bg)), _p(_u16(Sg)),
                             _p(_u32(Bu)), _p(_u16(Su)), _p(_u32(Bd)), _p(_u16(Sd)), _p(O), int(round_up))
    return O


def set_threads(n: int) -> None:
    """OpenMP threads of the oracle's and (where built) the compiled reference's loops."""
    orc().orc_set_threads(int(n))
    if ref_available():
        ref().ref_set_threads(int(n))


def max_threads() -> int:
    return int(orc().orc_max_threads())


# ---- the compiled reference (oracle/_ref) ------------------------------------

def ref_int2_gold(A, B, S, M, K, N, bf16: bool) -> np.ndarray:
    r = ref()
    r.ref_set_bf16(int(bf16))
    C_ = np.empty((M, N), np.float32)
    r.ref_int2_gold(_p(_u16(A)), _p(_u32(B)), _p(_u16(S)), _p(C_), M, K, N)
    return C_


def ref_epilogue(acc, other, bias, postop, out_f32, bf16):
    r = ref()
    r.ref_set_bf16(int(bf16))
    acc = np.ascontiguousarray(acc, np.float32)
    M, N = acc.shape
    out = np.empty((M, N), np.float32 if out_f32 else np.uint16)
    o = None if other is None else _u16(other)
    b = None if bias is None else np.ascontiguousarray(bias)
    r.ref_epilogue(postop, int(out_f32), _p(acc), _p(o), _p(b), _p(out), M, N)
    return out


def ref_scale_a(A, M, K, bf16):
    r = ref()
    r.ref_set_bf16(int(bf16))
    SA = np.zeros((K // 128, ldsa(M)), np.uint16)
    r.ref_scale_a(_p(_u16(A)), _p(SA), M, K)
    return SA


def ref_int8_gold(A, B, SA, SB, M, K, N, bf16):
    r = ref()
    r.ref_set_bf16(int(bf16))
    C_ = np.empty((M, N), np.float32)
    r.ref_int8_gold(_p(_u16(A)), _p(_u32(B)), _p(_u16(SA)), _p(_u16(SB)), _p(C_), M, K, N)
    return C_


def ref_bitcos_random(K, N, z, seed) -> np.ndarray:
    r = ref()
    n = r.ref_bitcos_random_words(K, N, z, seed)
    buf = np.empty(n, np.uint32)
    r.ref_bitcos_random(K, N, z, seed, _p(buf))
    return buf


def ref_bitcos_slice_ranks(buf, K, N, ls):
    sr = np.zeros(max(ls - 1, 0) * N, np.uint32)
    b = _u32(buf)
    ref().ref_bitcos_slice_ranks(_p(b), b.size, K, N, ls, _p(sr))
    return sr


def ref_bitcos_decode(buf, K, N):
    b = _u32(buf)
    out = np.empty((K, N), np.int8)
    col = np.empty(K, np.int8)
    for n in range(N):
        ref().ref_bitcos_decode_col(_p(b), b.size, K, N, n, _p(col))
        out[:, n] = col
    return out


def ref_bitcos_gold(A, buf, S, M, K, N, bf16):
    r = ref()
    r.ref_set_bf16(int(bf16))
    b = _u32(buf)
    C_ = np.empty((M, N), np.float32)
    r.ref_bitcos_gold(_p(_u16(A)), _p(b), b.size, _p(_u16(S)), _p(C_), M, K, N)
    return C_
