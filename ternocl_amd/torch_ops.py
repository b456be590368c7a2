"""PyTorch custom operators over the C ABI: ``torch.ops.ternocl.*``.

A serving framework calls the library through these: each operator allocates
its outputs with torch on the inputs' device, takes its workspace (where the C
ABI has one) from a zeroed one kept per device and stream, launches on torch's
current stream, and has a fake (meta)
implementation, so the operators trace under ``torch.compile`` and run inside
captured CUDA/HIP graphs.  They add nothing to the arithmetic: every call is
one call of the ``ternocl_amd`` function of the same name, which raises if the
native library is missing (there is no CPU fallback).

    import ternocl_amd.torch_ops  # registers the operators
    C = torch.ops.ternocl.int2_gemm(A, B, S, None, None, 0, False)

Operators (the reference kernels they stand for, as in the C ABI):
  int2_gemm         int2_fp16_upcvt_gemm{,_mt}            (int2_fp16_upcvt.cl:196, :341)
  quant_a           quant_a                               (int2_int8_dpas.cl:105)
  int2_int8_gemm    int2_int8_gemm_mt, upfront quant      (int2_int8_dpas.cl:316)
  bitcos_gemm       bitcos_fp16_upcvt_gemv / _gemm_mt     (bitcos_fp16_upcvt.cl:179, :303)
  fwht              hadamard_fwht                         (hadamard_fwht.cl:63)
  moe_prefill       the int2 MoE prefill layer            (int2_moe/prefill.cpp:268-279)
  moe_decode        the int2 MoE decode layer             (int2_moe/int2_moe.cl:61-174)
  moe_prefill_int8  the int8 MoE prefill layer            (int2_moe/int2_moe_prefill_int8.cl)
"""
from __future__ import annotations

from typing import Optional

import torch

import ternocl_amd as T

__all__ = ["int2_gemm", "quant_a", "int2_int8_gemm", "bitcos_gemm", "fwht", "moe_prefill", "moe_decode", "moe_prefill_int8"]


def _out_dtype(A: torch.Tensor, out_f32: bool) -> torch.dtype:
    return torch.float32 if out_f32 else A.dtype


# One workspace per (device, stream), zeroed once when it is allocated and
# shared by every operator on that stream: the C ABI keeps the K splits'
# counters in the workspace header and every call leaves them at zero, and
# calls on one stream never overlap.  A larger request allocates a larger one
# (at least twice the size); the smaller ones are kept alive, since a captured
# graph may still address them.
_WS: dict = {}
_WS_OLD: list = []


def _workspace(device: torch.device, nbytes: int) -> Optional[torch.Tensor]:
    if nbytes == 0:
        return None
    key = (device.index, torch.cuda.current_stream(device).cuda_stream)
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if ws is not None:
            _WS_OLD.append(ws)
        ws = torch.zeros(max(nbytes, 0 if ws is None else 2 * ws.numel()), dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


# ---- input checks ------------------------------------------------------------
# The C ABI takes raw pointers and reads every tensor as a dense row-major array
# of the stated type, so the operators check dtype, shape, contiguity and device
# before any launch (an int64 ids tensor, say, would otherwise be read as int32
# pairs).  torch._check raises RuntimeError; on meta tensors (the fake
# implementations) the same checks run at trace time.

def _chk(t: Optional[torch.Tensor], name: str, dtype, shape, device) -> None:
    if t is None:
        return
    dts = dtype if isinstance(dtype, tuple) else (dtype,)
    torch._check(t.dtype in dts, lambda: f"{name}: dtype {t.dtype}, expected {' or '.join(map(str, dts))}")
    torch._check(tuple(t.shape) == tuple(shape), lambda: f"{name}: shape {tuple(t.shape)}, expected {tuple(shape)}")
    torch._check(t.is_contiguous(), lambda: f"{name} must be contiguous")
    torch._check(t.device == device, lambda: f"{name} is on {t.device}, expected {device}")


_DT = (torch.float16, torch.bfloat16)


def _chk_act(A: torch.Tensor, name: str = "A") -> None:
    torch._check(A.dim() == 2, lambda: f"{name} must be 2-D")
    _chk(A, name, _DT, A.shape, A.device)


def _chk_int2(A, B, S, other, bias, out_f32) -> None:
    _chk_act(A)
    M, K = A.shape
    torch._check(B.dim() == 2, lambda: "B must be int32 [K/16, N]")
    N = B.shape[1]
    _chk(B, "B", torch.int32, (K // 16, N), A.device)
    _chk(S, "S", A.dtype, (K // 128, N), A.device)
    _chk(other, "other", A.dtype, (M, N), A.device)
    _chk(bias, "bias", _out_dtype(A, out_f32), (N,), A.device)


def _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd) -> None:
    _chk_act(X, "X")
    Tk, H = X.shape
    torch._check(ids.dim() == 2 and Bg.dim() == 3, lambda: "ids must be [T, topk], Bg [E, H/16, I]")
    topk, I = ids.shape[1], Bg.shape[2]
    d = X.device
    _chk(ids, "ids", torch.int32, (Tk, topk), d)
    _chk(RW, "RW", X.dtype, (Tk, topk), d)
    for nm, b, s in (("Bg", Bg, Sg), ("Bu", Bu, Su)):
        _chk(b, nm, torch.int32, (E, H // 16, I), d)
        _chk(s, "S" + nm[1], X.dtype, (E, H // 128, I), d)
    _chk(Bd, "Bd", torch.int32, (E, I // 16, H), d)
    _chk(Sd, "Sd", X.dtype, (E, I // 128, H), d)


@torch.library.custom_op("ternocl::int2_gemm", mutates_args=())
def int2_gemm(A: torch.Tensor, B: torch.Tensor, S: torch.Tensor, other: Optional[torch.Tensor],
              bias: Optional[torch.Tensor], postop: int, out_f32: bool) -> torch.Tensor:
    """C [M, N] = ct(epi(A x dequant(B, S))); B int32 [K/16, N], S [K/128, N] in A's dtype."""
    _chk_int2(A, B, S, other, bias, out_f32)
    M, K = A.shape
    N = B.shape[1]
    C = torch.empty((M, N), dtype=_out_dtype(A, out_f32), device=A.device)
    ws = _workspace(A.device, T.int2_gemm_ws_bytes(M, N, K))  # K-split sums and counters, where it splits
    T.int2_fp16_upcvt_gemm(A, B, S, C, other, bias, M, N, K, postop, out_f32, ws=ws)
    return C


@int2_gemm.register_fake
def _(A, B, S, other, bias, postop, out_f32):
    _chk_int2(A, B, S, other, bias, out_f32)
    return A.new_empty((A.shape[0], B.shape[1]), dtype=_out_dtype(A, out_f32))


@torch.library.custom_op("ternocl::quant_a", mutates_args=())
def quant_a(A: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(SA [K/128, ldsa(M)] in A's dtype, Aq int8 [M, K]) of A [M, K]."""
    _chk_act(A)
    M, K = A.shape
    SA = torch.empty((K // 128, T.ldsa(M)), dtype=A.dtype, device=A.device)
    Aq = torch.empty((M, K), dtype=torch.int8, device=A.device)
    T.quant_a(A, SA, Aq, M, K)
    return SA, Aq


@quant_a.register_fake
def _(A):
    _chk_act(A)
    M, K = A.shape
    # ldsa(M) = (M + 31) & ~31 (LDSA of int2_int8_dpas.cl:58), computed here without the library
    return A.new_empty((K // 128, (M + 31) // 32 * 32)), A.new_empty((M, K), dtype=torch.int8)


@torch.library.custom_op("ternocl::int2_int8_gemm", mutates_args=())
def int2_int8_gemm(Aq: torch.Tensor, SA: torch.Tensor, B: torch.Tensor, SB: torch.Tensor,
                   other: Optional[torch.Tensor], bias: Optional[torch.Tensor], postop: int,
                   out_f32: bool) -> torch.Tensor:
    """C [M, N] of the s8 x s2 prefill on quant_a's (SA, Aq); SB [K/128, N] sets the dtype."""
    _chk_int8(Aq, SA, B, SB, other, bias, out_f32)
    M, K = Aq.shape
    N = B.shape[1]
    C = torch.empty((M, N), dtype=_out_dtype(SB, out_f32), device=Aq.device)
    ws = _workspace(Aq.device, T.int2_int8_gemm_ws_bytes(M, N, K))  # the K split's counters and partials
    T.int2_int8_gemm(None, Aq, SA, B, SB, C, other, bias, M, N, K, postop, out_f32, ws=ws)
    return C


def _chk_int8(Aq, SA, B, SB, other, bias, out_f32) -> None:
    torch._check(Aq.dim() == 2 and B.dim() == 2, lambda: "Aq must be int8 [M, K], B int32 [K/16, N]")
    M, K = Aq.shape
    N = B.shape[1]
    d = Aq.device
    _chk(Aq, "Aq", torch.int8, (M, K), d)
    _chk(SB, "SB", _DT, (K // 128, N), d)
    _chk(SA, "SA", SB.dtype, (K // 128, (M + 31) // 32 * 32), d)
    _chk(B, "B", torch.int32, (K // 16, N), d)
    _chk(other, "other", SB.dtype, (M, N), d)
    _chk(bias, "bias", _out_dtype(SB, out_f32), (N,), d)


@int2_int8_gemm.register_fake
def _(Aq, SA, B, SB, other, bias, postop, out_f32):
    _chk_int8(Aq, SA, B, SB, other, bias, out_f32)
    return SB.new_empty((Aq.shape[0], B.shape[1]), dtype=_out_dtype(SB, out_f32))


@torch.library.custom_op("ternocl::bitcos_gemm", mutates_args=())
def bitcos_gemm(A: torch.Tensor, B: torch.Tensor, S: torch.Tensor, SR: Optional[torch.Tensor], ls: int,
                N: int, other: Optional[torch.Tensor], bias: Optional[torch.Tensor], postop: int,
                out_f32: bool) -> torch.Tensor:
    """C [M, N] of the BITCOS weights B (the common/bitcos.hpp buffer, int32) with slice ranks SR
    for ls slices.  M >= 16 takes the M-tiled path (a workspace of the re-packed weights is
    allocated per call), smaller M the GEMV (with the split launch's workspace where it has one)."""
    _chk_bitcos(A, B, S, SR, ls, N, other, bias, out_f32)
    M, K = A.shape
    C = torch.empty((M, N), dtype=_out_dtype(A, out_f32), device=A.device)
    if M >= 16:
        ws = _workspace(A.device, T.bitcos_gemm_mt_ws_bytes(K, N))
        T.bitcos_fp16_upcvt_gemm_mt(A, B, S, SR, C, other, bias, M, N, K, ls, ws, postop, out_f32)
    else:
        ws = _workspace(A.device, T.bitcos_gemv_ws_bytes(N, ls))  # the split launch's sums and counters
        T.bitcos_fp16_upcvt_gemm(A, B, S, SR, C, other, bias, M, N, K, ls, postop, out_f32, ws=ws)
    return C


def _chk_bitcos(A, B, S, SR, ls, N, other, bias, out_f32) -> None:
    _chk_act(A)
    M, K = A.shape
    torch._check(B.dim() == 1, lambda: "B must be the 1-D int32 BITCOS buffer")
    _chk(B, "B", torch.int32, B.shape, A.device)
    _chk(S, "S", A.dtype, (K // 128, N), A.device)
    if ls > 1:
        torch._check(SR is not None, lambda: "SR is needed for ls > 1")
    if SR is not None and ls > 1:
        _chk(SR, "SR", torch.int32, ((ls - 1) * N,), A.device)
    _chk(other, "other", A.dtype, (M, N), A.device)
    _chk(bias, "bias", _out_dtype(A, out_f32), (N,), A.device)


@bitcos_gemm.register_fake
def _(A, B, S, SR, ls, N, other, bias, postop, out_f32):
    _chk_bitcos(A, B, S, SR, ls, N, other, bias, out_f32)
    return A.new_empty((A.shape[0], N), dtype=_out_dtype(A, out_f32))


@torch.library.custom_op("ternocl::fwht", mutates_args=())
def fwht(x: torch.Tensor, signs: Optional[torch.Tensor], HB: int) -> torch.Tensor:
    """y [rows, K] = DT(SCALE * H_HB(signs * x)) blockwise; signs int8 [K] or None."""
    _chk_act(x, "x")
    _chk(signs, "signs", torch.int8, (x.shape[1],), x.device)
    rows, K = x.shape
    y = torch.empty_like(x)
    T.hadamard_fwht(x, signs, y, rows, K, HB, signs is not None)
    return y


@fwht.register_fake
def _(x, signs, HB):
    _chk_act(x, "x")
    _chk(signs, "signs", torch.int8, (x.shape[1],), x.device)
    return torch.empty_like(x)


@torch.library.custom_op("ternocl::moe_prefill", mutates_args=())
def moe_prefill(X: torch.Tensor, ids: torch.Tensor, RW: torch.Tensor, E: int, Bg: torch.Tensor,
                Sg: torch.Tensor, Bu: torch.Tensor, Su: torch.Tensor, Bd: torch.Tensor,
                Sd: torch.Tensor) -> torch.Tensor:
    """O [T, H] of one int2 MoE layer: X [T, H], ids int32 [T, topk], RW [T, topk] in X's dtype,
    experts stacked: Bg / Bu int32 [E, H/16, I], Bd int32 [E, I/16, H], scales alike."""
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    Tk, H = X.shape
    topk = ids.shape[1]
    I = Bg.shape[2]
    O = torch.empty((Tk, H), dtype=X.dtype, device=X.device)
    ws = _workspace(X.device, T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I))
    T.int2_moe_prefill(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    return O


@moe_prefill.register_fake
def _(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd):
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    return torch.empty_like(X)


@torch.library.custom_op("ternocl::moe_decode", mutates_args=())
def moe_decode(X: torch.Tensor, ids: torch.Tensor, RW: torch.Tensor, E: int, Bg: torch.Tensor,
               Sg: torch.Tensor, Bu: torch.Tensor, Su: torch.Tensor, Bd: torch.Tensor,
               Sd: torch.Tensor) -> torch.Tensor:
    """O [T, H] of one int2 MoE decode layer (few tokens, T * topk <= 32767); arguments as
    moe_prefill."""
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    Tk, H = X.shape
    topk = ids.shape[1]
    I = Bg.shape[2]
    O = torch.empty((Tk, H), dtype=X.dtype, device=X.device)
    ws = _workspace(X.device, T.int2_moe_decode_ws_bytes(Tk, topk, H, I))
    T.int2_moe_decode(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    return O


@moe_decode.register_fake
def _(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd):
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    return torch.empty_like(X)


@torch.library.custom_op("ternocl::moe_prefill_int8", mutates_args=())
def moe_prefill_int8(X: torch.Tensor, ids: torch.Tensor, RW: torch.Tensor, E: int, Bg: torch.Tensor,
                     Sg: torch.Tensor, Bu: torch.Tensor, Su: torch.Tensor, Bd: torch.Tensor,
                     Sd: torch.Tensor) -> torch.Tensor:
    """O [T, H] of one MoE prefill layer on the s8 x s2 GEMM; arguments as moe_prefill."""
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    Tk, H = X.shape
    topk = ids.shape[1]
    I = Bg.shape[2]
    O = torch.empty((Tk, H), dtype=X.dtype, device=X.device)
    ws = _workspace(X.device, T.int2_moe_prefill_int8_ws_bytes(Tk, E, topk, H, I))
    T.int2_moe_prefill_int8(X, ids, RW, Tk, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws)
    return O


@moe_prefill_int8.register_fake
def _(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd):
    _chk_moe(X, ids, RW, E, Bg, Sg, Bu, Su, Bd, Sd)
    return torch.empty_like(X)
