"""ternocl_amd -- MI355X (gfx950) ternary GEMV/GEMM library, Python mirror.

The product is the C ABI in ``include/ternocl_amd.h`` (shared library
``ternocl_amd/_lib/libternocl_amd.so``).  This module is a thin ctypes mirror of
the reference's kernel interface: the same kernel names and argument order as
TernOCL's OpenCL kernels, with torch tensors (device memory) in place of
``cl_mem`` buffers.  It never falls back to a CPU path: if the library is
missing, every call raises.

Errors: the reference's host drivers print and exit on a shape violation
(e.g. ``int2_fp16_upcvt/main.cpp:159``); here every check happens on the host
before any launch and raises :class:`TernoclError` carrying the C status.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

from . import _abi

__all__ = [
    "TernoclError", "lib", "library_path", "FP16", "BF16", "WS_HEADER_BYTES",
    "int2_gemm_ws_bytes", "workspace_zero", "int2_fp16_upcvt_gemm", "int2_dequant",
    "int2_gemv_decode", "int2_gemv_stream_probe", "stream_read_probe", "gemv_tile", "GemvTile", "VALU", "MFMA", "GEMM",
    "int2_pack", "int2_unpack", "bitcos_pack", "bitcos_unpack", "bitcos_slice_ranks_host",
    "ldsa", "quant_a", "int2_int8_gemm", "int2_int8_gemm_ws_bytes", "int2_s8_decode",
    "bitcos_fp16_upcvt_gemm", "bitcos_fwht_gemm", "bitcos_gemv_ws_bytes", "bitcos_slice_ranks", "bitcos_pick_ls", "bitcos_dequant",
    "hadamard_fwht",
    "moe_tile_rows", "int2_moe_route", "int2_moe_gather", "int2_moe_gemm", "int2_moe_combine",
    "int2_moe_prefill_ws_bytes", "int2_moe_prefill", "int2_moe_prefill_int8_ws_bytes", "int2_moe_prefill_int8",
]

FP16, BF16 = 0, 1
# TERNOCL_WS_HEADER_BYTES: the front of every workspace, where the K splits keep
# their counters (zero between calls); all other workspace data lies after it.
WS_HEADER_BYTES = 64 << 10
_LIB_PATH = Path(__file__).resolve().parent / "_lib" / "libternocl_amd.so"
_lib = None


class TernoclError(RuntimeError):
    """A C-ABI call returned a non-OK status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} (status {status})")
        self.status = status


def library_path() -> Path:
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    """Load the HIP library (once).  Raises if it has not been built."""
    global _lib
    if _lib is None:
        path = Path(os.environ.get("TERNOCL_AMD_LIB", _LIB_PATH))
        if not path.exists():
            raise TernoclError(-1, f"{path} is missing: run `python -m ternocl_amd.build` first")
        _lib = ctypes.CDLL(str(path))
        _abi.declare(_lib)
    return _lib


def _check(status: int) -> None:
    if status != 0:
        L = lib()
        raise TernoclError(status, f"{L.ternocl_status_string(status).decode()}: "
                                   f"{L.ternocl_last_error().decode()}")


def _ptr(x) -> int | None:
    """Device pointer of a torch tensor (None -> NULL, int passes through)."""
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream(stream) -> int | None:
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def _dtype_of(t) -> int:
    import torch
    if t.dtype == torch.float16:
        return FP16
    if t.dtype == torch.bfloat16:
        return BF16
    raise TernoclError(1, f"activations must be float16 or bfloat16, got {t.dtype}")


def _nbytes(t) -> int:
    return 0 if t is None else t.numel() * t.element_size()


# ---- int2 upcvt (int2_fp16_upcvt/int2_fp16_upcvt.cl) --------------------

def int2_gemm_ws_bytes(M: int, N: int, K: int) -> int:
    """Workspace bytes of ``int2_fp16_upcvt_gemm`` (0 when none is needed)."""
    return lib().ternocl_int2_gemm_ws_bytes(M, N, K)


def workspace_zero(ws, stream=None) -> None:
    """Zero a workspace once before its first use (the library keeps it zeroed)."""
    _check(lib().ternocl_workspace_zero(_ptr(ws), _nbytes(ws), _stream(stream)))


GemvTile = _abi.GemvTile
VALU, MFMA, GEMM, F4, F4MS = 1, 2, 3, 4, 5  # engines: VALU GEMV, MFMA GEMV, MFMA prefill GEMM,
# fp8 x fp4 GEMV, its multi-strip form (M = 1)


def gemv_tile(engine: int = 0, waves: int = 0, cols_per_lane: int = 0, groups_per_wave: int = 0,
              col_lanes: int = 0, k_slices: int = 0) -> "GemvTile":
    """A decode-GEMV tile (0 = automatic for every field)."""
    return GemvTile(engine, waves, cols_per_lane, groups_per_wave, col_lanes, k_slices)


def int2_fp16_upcvt_gemm(A, B, S, C, Other, Bias, M: int, N: int, K: int, postop: int = 0,
                         out_f32: bool = False, ws=None, stream=None, tile=None) -> None:
    """C = ct(epi(A x dequant(B, S))) -- int2_fp16_upcvt_gemm{,_mt}(A, B, S, C, Other,
    Bias, M, N, K) of int2_fp16_upcvt.cl:196 / :341.  ``tile`` (a GemvTile)
    overrides the automatic decode-GEMV tile."""
    L = lib()
    args = (_dtype_of(A), _ptr(A), _ptr(B), _ptr(S), _ptr(C), _ptr(Other), _ptr(Bias), M, N, K,
            postop, int(bool(out_f32)), _ptr(ws), _nbytes(ws))
    if tile is None:
        _check(L.ternocl_int2_fp16_upcvt_gemm(*args, _stream(stream)))
    else:
        _check(L.ternocl_int2_fp16_upcvt_gemm_ex(*args, ctypes.byref(tile), _stream(stream)))


def int2_dequant(B, S, W, K: int, N: int, stream=None) -> None:
    """W = the DT B operand the reference's dq_word builds (+0, +s, s^0x8000)."""
    _check(lib().ternocl_int2_dequant(_dtype_of(W), _ptr(B), _ptr(S), _ptr(W), K, N, _stream(stream)))


def int2_gemv_decode(B, D, K: int, N: int, bf16: bool, engine: int = MFMA, stream=None) -> None:
    """D[word][j] = the packed DT pair j an engine builds from each B word (test hook;
    engine 4 writes its two fp4 dwords per word)."""
    _check(lib().ternocl_int2_gemv_decode(BF16 if bf16 else FP16, engine, _ptr(B), _ptr(D), K, N,
                                          _stream(stream)))


# ---- int2 x int8 (int2_via_int2_x_int8_dpas/int2_int8_dpas.cl) ------------

def stream_read_probe(src, nbytes: int, sink, stream=None) -> None:
    """Plain streaming read of the first nbytes (rounded down to 16) of the device tensor
    src (measurement hook: the per-launch read ceiling; sink: a tensor of >= 4 bytes)."""
    _check(lib().ternocl_stream_read_probe(_ptr(src), nbytes, _ptr(sink), _stream(stream)))


def int2_gemv_stream_probe(B, S, C, M: int, N: int, K: int, stream=None) -> None:
    """The decode GEMV (engine 4) with the decode removed: streams B and S as the GEMV
    does and writes a checksum per column into C (fp32 [M, N]) -- a memory-ceiling
    measurement, not a GEMV.  The dtype comes from S."""
    _check(lib().ternocl_int2_gemv_stream_probe(_dtype_of(S), _ptr(B), _ptr(S), _ptr(C), M, N, K,
                                                 _stream(stream)))


# ---- host packers (CPU, through the C ABI) -----------------------------------

def _host_i8(W, K=None, N=None):
    import numpy as np
    W = np.ascontiguousarray(W, dtype=np.int8)
    if W.ndim != 2:
        raise ValueError("W must be [K, N]")
    return W


def _cptr(a):
    return ctypes.c_void_p(a.ctypes.data)


def int2_pack(W):
    """int8 [K, N] ternary -> B uint32 [K/16, N] (ternocl_int2_pack)."""
    import numpy as np
    W = _host_i8(W)
    K, N = W.shape
    B = np.empty((K // 16, N), np.uint32)
    _check(lib().ternocl_int2_pack(_cptr(W), _cptr(B), K, N))
    return B


def int2_unpack(B, K: int):
    """B uint32 [K/16, N] -> int8 [K, N] (ternocl_int2_unpack)."""
    import numpy as np
    B = np.ascontiguousarray(B, dtype=np.uint32)
    N = B.shape[1]
    W = np.empty((K, N), np.int8)
    _check(lib().ternocl_int2_unpack(_cptr(B), _cptr(W), K, N))
    return W


def bitcos_pack(W):
    """int8 [K, N] ternary -> the BITCOS buffer, uint32 (ternocl_bitcos_pack)."""
    import numpy as np
    W = _host_i8(W)
    K, N = W.shape
    n = lib().ternocl_bitcos_pack_words(_cptr(W), K, N)
    if n == 0:
        raise TernoclError(1, "bitcos_pack: W must be ternary with K % 32 == 0")
    buf = np.empty(n, np.uint32)
    _check(lib().ternocl_bitcos_pack(_cptr(W), K, N, _cptr(buf), n))
    return buf


def bitcos_unpack(buf, K: int, N: int):
    """The BITCOS buffer -> int8 [K, N] ternary (ternocl_bitcos_unpack)."""
    import numpy as np
    buf = np.ascontiguousarray(buf, dtype=np.uint32)
    W = np.empty((K, N), np.int8)
    _check(lib().ternocl_bitcos_unpack(_cptr(buf), buf.size, K, N, _cptr(W)))
    return W


def bitcos_slice_ranks_host(buf, K: int, N: int, ls: int):
    """Slice ranks [ls-1, N] of a BITCOS buffer, on the host (ternocl_bitcos_slice_ranks_host)."""
    import numpy as np
    buf = np.ascontiguousarray(buf, dtype=np.uint32)
    SR = np.zeros(max(ls - 1, 0) * N, np.uint32)
    _check(lib().ternocl_bitcos_slice_ranks_host(_cptr(buf), K, N, ls, _cptr(SR) if SR.size else None))
    return SR


def ldsa(M: int) -> int:
    """Row pitch of SA, (M + 31) & ~31 (LDSA of int2_int8_dpas.cl:58)."""
    return lib().ternocl_ldsa(M)


def quant_a(A, SA, Aq, M: int, K: int, stream=None) -> None:
    """quant_a(A, SA, Aq, M, K) of int2_int8_dpas.cl:105: SA [K/128, ldsa(M)] DT scales
    and Aq [M, K] int8, bit-exact with the reference's host quantization.  Aq=None writes
    SA only (the reference built without WRITE_Q, for the in-GEMM quantization mode)."""
    _check(lib().ternocl_quant_a(_dtype_of(A), _ptr(A), _ptr(SA), _ptr(Aq), M, K, _stream(stream)))


def int2_int8_gemm_ws_bytes(M: int, N: int, K: int) -> int:
    """Scratch bytes of int2_int8_gemm's K-split path (0: none used)."""
    return lib().ternocl_int2_int8_gemm_ws_bytes(M, N, K)


def int2_int8_gemm(A, Aq, SA, B, SB, C, Other, Bias, M: int, N: int, K: int, postop: int = 0,
                   out_f32: bool = False, ws=None, stream=None) -> None:
    """int2_int8_gemm_mt(A, Aq, SA, B, SB, C, Other, Bias, M, N, K) of int2_int8_dpas.cl:316.
    With Aq given: upfront quantization (QMODE 0; A is not read and may be None).  With
    Aq=None: A's tiles are quantized while staged (QMODE 1), bit-identical q.  The dtype
    comes from SB.  ``ws`` (int2_int8_gemm_ws_bytes, zeroed once): the deterministic K split
    where the wide tiles (or, at M <= 4, the GEMV's strips) alone leave CUs idle."""
    _check(lib().ternocl_int2_int8_gemm_ws(_dtype_of(SB), _ptr(A), _ptr(Aq), _ptr(SA), _ptr(B), _ptr(SB),
                                           _ptr(C), _ptr(Other), _ptr(Bias), M, N, K, postop,
                                           int(bool(out_f32)), _ptr(ws), _nbytes(ws), _stream(stream)))


def int2_s8_decode(B, D, K: int, N: int, stream=None) -> None:
    """D[word][i] = the s8 x s2 GEMM's B fragment dwords of each word (test hook)."""
    _check(lib().ternocl_int2_s8_decode(_ptr(B), _ptr(D), K, N, _stream(stream)))


# ---- BITCOS (bitcos_fp16_upcvt/bitcos_fp16_upcvt.cl) ------------------------

def bitcos_gemv_ws_bytes(N: int, ls: int) -> int:
    """Scratch bytes of bitcos_fp16_upcvt_gemm's split launch (0: none)."""
    return lib().ternocl_bitcos_gemv_ws_bytes(N, ls)


def bitcos_fp16_upcvt_gemm(A, B, S, SR, C, Other, Bias, M: int, N: int, K: int, ls: int = 1,
                           postop: int = 0, out_f32: bool = False, ws=None, stream=None) -> None:
    """bitcos_fp16_upcvt_gemv(A, B, S, SR, C, Other, Bias, M, N, K) of
    bitcos_fp16_upcvt.cl:179 with LS = ls K slices (SR computed for that ls).
    ``ws`` (bitcos_gemv_ws_bytes, zeroed once): the launch that spreads a
    strip's slices over several workgroups where that evens out the CUs."""
    if ws is None:
        _check(lib().ternocl_bitcos_fp16_upcvt_gemm(_dtype_of(A), _ptr(A), _ptr(B), _ptr(S), _ptr(SR), ls,
                                                    _ptr(C), _ptr(Other), _ptr(Bias), M, N, K, postop,
                                                    int(bool(out_f32)), _stream(stream)))
    else:
        _check(lib().ternocl_bitcos_fp16_upcvt_gemm_ws(_dtype_of(A), _ptr(A), _ptr(B), _ptr(S), _ptr(SR), ls,
                                                       _ptr(C), _ptr(Other), _ptr(Bias), M, N, K, postop,
                                                       int(bool(out_f32)), _ptr(ws), _nbytes(ws),
                                                       _stream(stream)))


def bitcos_fwht_gemm(x, signs, HB: int, B, S, SR, C, Other, Bias, M: int, N: int, K: int, ls: int = 1,
                     postop: int = 0, out_f32: bool = False, ws=None, use_signs: bool = True, stream=None) -> None:
    """The decode step's sign flip + FWHT (hadamard_fwht.cl:62) and BITCOS GEMV (bitcos_fp16_upcvt.cl:179)
    in one launch: the C of hadamard_fwht(x, signs, y) then bitcos_fp16_upcvt_gemm(y, ...), bit for bit,
    without y.  ``ws``: as bitcos_fp16_upcvt_gemm (bitcos_gemv_ws_bytes, zeroed once)."""
    _check(lib().ternocl_bitcos_fwht_gemm_ws(_dtype_of(x), _ptr(x), _ptr(signs), HB, int(bool(use_signs)), _ptr(B),
                                             _ptr(S), _ptr(SR), ls, _ptr(C), _ptr(Other), _ptr(Bias), M, N, K, postop,
                                             int(bool(out_f32)), _ptr(ws), _nbytes(ws), _stream(stream)))


def bitcos_gemm_mt_ws_bytes(K: int, N: int) -> int:
    return lib().ternocl_bitcos_gemm_mt_ws_bytes(K, N)


def bitcos_fp16_upcvt_gemm_mt(A, B, S, SR, C, Other, Bias, M: int, N: int, K: int, ls: int, ws,
                              postop: int = 0, out_f32: bool = False, stream=None) -> None:
    """bitcos_fp16_upcvt_gemm_mt (bitcos_fp16_upcvt.cl:303): any M, the weights re-packed into
    ws (bitcos_gemm_mt_ws_bytes) and streamed once by the int2 prefill GEMM."""
    _check(lib().ternocl_bitcos_fp16_upcvt_gemm_mt(_dtype_of(A), _ptr(A), _ptr(B), _ptr(S), _ptr(SR), ls,
                                                   _ptr(C), _ptr(Other), _ptr(Bias), M, N, K, postop,
                                                   int(bool(out_f32)), _ptr(ws), _nbytes(ws),
                                                   _stream(stream)))


def bitcos_to_int2(B, SR, ls: int, W2, K: int, N: int, stream=None) -> None:
    """W2 [K/16, N] int2 words of the BITCOS weights (the M-tiled path's re-pack, test hook)."""
    _check(lib().ternocl_bitcos_to_int2(_ptr(B), _ptr(SR), ls, _ptr(W2), K, N, _stream(stream)))


def bitcos_slice_ranks(B, SR, K: int, N: int, ls: int, stream=None) -> None:
    """SR [ls-1, N] slice ranks of a BITCOS buffer (common/bitcos.hpp:81-94), on the device."""
    _check(lib().ternocl_bitcos_slice_ranks(_ptr(B), _ptr(SR), K, N, ls, _stream(stream)))


def bitcos_pick_ls(M: int, N: int, K: int) -> int:
    return lib().ternocl_bitcos_pick_ls(M, N, K)


def bitcos_dequant(B, S, W, K: int, N: int, stream=None) -> None:
    """W = the DT B operand of the BITCOS kernels (0 / S / S^0x8000), test hook."""
    _check(lib().ternocl_bitcos_dequant(_dtype_of(W), _ptr(B), _ptr(S), _ptr(W), K, N, _stream(stream)))


# ---- Hadamard (hadamard/hadamard_fwht.cl) ------------------------------------

def hadamard_fwht(x, signs, y, rows: int, K: int, HB: int, use_signs: bool = True, stream=None) -> None:
    """hadamard_fwht(x, signs, y, K, use_signs) of hadamard_fwht.cl:63 with -DHB=HB over rows rows."""
    _check(lib().ternocl_hadamard_fwht(_dtype_of(x), _ptr(x), _ptr(signs), _ptr(y), rows, K, HB,
                                       int(bool(use_signs)), _stream(stream)))


# ---- int2 MoE prefill (int2_moe/int2_moe_prefill.cl) ---------------------------

def moe_tile_rows() -> int:
    """Rows per tile of meta's row-tile offsets."""
    return lib().ternocl_moe_tile_rows()


def int2_moe_route(ids, meta, perm, inv, G: int, E: int, stream=None) -> None:
    """int2_moe_route(ids, meta, perm, inv, G) of int2_moe_prefill.cl:30 (stable order)."""
    _check(lib().ternocl_int2_moe_route(_ptr(ids), _ptr(meta), _ptr(perm), _ptr(inv), G, E, _stream(stream)))


def int2_moe_gather(X, perm, Xs, G: int, K: int, topk: int, stream=None) -> None:
    """int2_moe_gather(X, perm, Xs, K) of int2_moe_prefill.cl:64."""
    _check(lib().ternocl_int2_moe_gather(_dtype_of(X), _ptr(X), _ptr(perm), _ptr(Xs), G, K, topk,
                                         _stream(stream)))


def int2_moe_gemm(meta, A_all, perm, topk: int, B_all, S_all, C_all, Other_all, E: int, G: int, N: int,
                  K: int, postop: int = 0, out_f32: bool = False, stream=None) -> None:
    """int2_moe_gemm_mt(meta, A_all, B_all, S_all, C_all, Other_all, N, K) of
    int2_moe_prefill.cl:75; A rows through perm / topk when perm is given."""
    _check(lib().ternocl_int2_moe_gemm(_dtype_of(A_all), _ptr(meta), _ptr(A_all), _ptr(perm), topk,
                                       _ptr(B_all), _ptr(S_all), _ptr(C_all), _ptr(Other_all), E, G, N, K,
                                       postop, int(bool(out_f32)), _stream(stream)))


def int2_moe_combine(Y, inv, RW, O, T: int, topk: int, N: int, stream=None) -> None:
    """int2_moe_combine(Y, inv, RW, O, N) of int2_moe_prefill.cl:144."""
    _check(lib().ternocl_int2_moe_combine(_dtype_of(O), _ptr(Y), _ptr(inv), _ptr(RW), _ptr(O), T, topk, N,
                                          _stream(stream)))


def int2_moe_prefill_ws_bytes(T: int, E: int, topk: int, H: int, I: int) -> int:
    return lib().ternocl_int2_moe_prefill_ws_bytes(T, E, topk, H, I)


def int2_moe_prefill(X, ids, RW, T: int, E: int, topk: int, H: int, I: int, Bg, Sg, Bu, Su, Bd, Sd, O,
                     ws, stream=None) -> None:
    """One MoE layer: route, up, gate (silu * up), down, combine (int2_moe/prefill.cpp:268-279)."""
    _check(lib().ternocl_int2_moe_prefill(_dtype_of(X), _ptr(X), _ptr(ids), _ptr(RW), T, E, topk, H, I,
                                          _ptr(Bg), _ptr(Sg), _ptr(Bu), _ptr(Su), _ptr(Bd), _ptr(Sd), _ptr(O),
                                          _ptr(ws), _nbytes(ws), _stream(stream)))


def int2_moe_prefill_int8_ws_bytes(T: int, E: int, topk: int, H: int, I: int) -> int:
    return lib().ternocl_int2_moe_prefill_int8_ws_bytes(T, E, topk, H, I)


def int2_moe_prefill_int8(X, ids, RW, T: int, E: int, topk: int, H: int, I: int, Bg, Sg, Bu, Su, Bd, Sd, O,
                          ws, stream=None) -> None:
    """One MoE prefill layer on the s8 x s2 GEMM: route, gather, quant_a, up, gate (silu * up),
    quant_a, down, combine (int2_moe/int2_moe_prefill_int8.cl, QMODE 1)."""
    _check(lib().ternocl_int2_moe_prefill_int8(_dtype_of(X), _ptr(X), _ptr(ids), _ptr(RW), T, E, topk, H, I,
                                               _ptr(Bg), _ptr(Sg), _ptr(Bu), _ptr(Su), _ptr(Bd), _ptr(Sd),
                                               _ptr(O), _ptr(ws), _nbytes(ws), _stream(stream)))


# ---- int2 MoE decode (int2_moe/int2_moe.cl) -------------------------------------

def int2_moe_decode_ws_bytes(T: int, topk: int, H: int, I: int) -> int:
    return lib().ternocl_int2_moe_decode_ws_bytes(T, topk, H, I)


def int2_moe_decode(X, ids, RW, T: int, E: int, topk: int, H: int, I: int, Bg, Sg, Bu, Su, Bd, Sd, O,
                    ws, stream=None) -> None:
    """One MoE decode layer: gate/up GEMVs with silu * up, down GEMVs, weighted sum over the
    topk experts (int2_moe/int2_moe.cl:61-133, main.cpp:226-261)."""
    _check(lib().ternocl_int2_moe_decode(_dtype_of(X), _ptr(X), _ptr(ids), _ptr(RW), T, E, topk, H, I,
                                         _ptr(Bg), _ptr(Sg), _ptr(Bu), _ptr(Su), _ptr(Bd), _ptr(Sd), _ptr(O),
                                         _ptr(ws), _nbytes(ws), _stream(stream)))
