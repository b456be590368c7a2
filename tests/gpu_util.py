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
    """The north-star float rule: |got - ref| <= atol + rtol * |ref| element-wise."""
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
