"""Helpers for the GPU tests: numpy <-> device tensors and the tolerance rules."""
from __future__ import annotations

import numpy as np


def dev_dt(a: np.ndarray, bf16: bool, device="cuda:0"):
    """DT raw bits (uint16) -> a float16 / bfloat16 device tensor."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, np.uint16).view(np.int16)).to(device)
    return t.view(torch.bfloat16 if bf16 else torch.float16)


def dev_raw(a: np.ndarray, device="cuda:0"):
    """Any numpy array -> a device tensor with the same bytes (int view)."""
    import torch
    a = np.ascontiguousarray(a)
    view = {1: np.int8, 2: np.int16, 4: np.int32, 8: np.int64}[a.dtype.itemsize]
    if a.dtype == np.float32:
        return torch.from_numpy(a).to(device)
    return torch.from_numpy(a.view(view)).to(device)


def host_u16(t) -> np.ndarray:
    import torch
    return t.detach().view(torch.int16).cpu().numpy().view(np.uint16)


def host_u32(t) -> np.ndarray:
    import torch
    return t.detach().view(torch.int32).cpu().numpy().view(np.uint32)


def host_f32(t) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def allclose_report(got: np.ndarray, ref: np.ndarray, rtol=1e-2, atol=1e-3):
    """The floating-point parity rule: |got - ref| <= atol + rtol * |ref| element-wise."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    d = np.abs(got - ref)
    bad = ~(d <= atol + rtol * np.abs(ref))
    return int(bad.sum()), float(d.max() if d.size else 0.0)


def xetla_cmp(got_bits: np.ndarray, ref_bits: np.ndarray, bf16: bool, abs_tol=None, ulp_tol=None):
    """The reference's pass rule (int2_fp16_upcvt/main.cpp:100-121, common/dt16.hpp:44-48):
    per element |d| <= abs_tol or ulp <= ulp_tol or rel <= 1e-3.  Returns #failures."""
    from ternocl_amd.formats import dt_to_f32
    abs_tol = abs_tol if abs_tol is not None else (16.0 if bf16 else 8.0)
    ulp_tol = ulp_tol if ulp_tol is not None else (32 if bf16 else 64)
    a = np.asarray(got_bits, np.int64)
    g = np.asarray(ref_bits, np.int64)
    ulp = np.abs(a - g)
    act = dt_to_f32(got_bits, bf16).astype(np.float64)
    des = dt_to_f32(ref_bits, bf16).astype(np.float64)
    d = np.abs(act - des)
    with np.errstate(divide="ignore", invalid="ignore"):
        rel = np.abs((des - act) / des)
    ok = (d <= abs_tol) | (ulp <= ulp_tol) | (rel <= 1e-3)
    return int((~ok).sum())


# ---- int2 upcvt GEMM inputs / launch / gold, shared by the GEMV and GEMM tests ----

def int2_inputs(seed, M, K, N, bf16, ref_dist=False):
    from ternocl_amd import formats, synth
    g = synth.rng(seed)
    if ref_dist:  # the reference driver's distributions (int2_fp16_upcvt/main.cpp:236, :243)
        A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
        S = synth.scales(g, K, N, bf16, 0.75, 15.75)
    else:  # the workload's: A ~ N(0,1), S ~ U[0.005, 0.02]
        A = synth.activations(g, (M, K), bf16)
        S = synth.scales(g, K, N, bf16)
    B = synth.int2_weights(g, K, N)
    other = synth.activations(g, (M, N), bf16)
    bias_f = (g.standard_normal(N).astype(np.float32) * 0.1)
    return A, B, S, other, bias_f


def int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32, ws=True, tile=None):
    from ternocl_amd import formats
    dA, dB, dS = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16)
    dO = dev_dt(other, bf16)
    if out_f32:
        dBias = torch.from_numpy(bias_f).cuda()
        dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    else:
        dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
        dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
    wsb = T.int2_gemm_ws_bytes(M, N, K)
    dW = None
    if ws and wsb:
        dW = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        T.workspace_zero(dW)
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, postop, out_f32, ws=dW, tile=tile)
    torch.cuda.synchronize()
    return dC, dW


def int2_gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32):
    from ternocl_amd import formats
    acc = orc.int2_gold(A, B, S, M, K, N, bf16)
    bias = bias_f if out_f32 else formats.f32_to_dt(bias_f, bf16)
    return orc.epilogue(acc, other, bias, postop, out_f32, bf16), acc
