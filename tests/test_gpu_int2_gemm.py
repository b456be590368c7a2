"""GPU parity of the int2 prefill GEMM (M > 16; engine 3 at any M) through the C ABI.

Reference test design followed: int2_fp16_upcvt/validate.sh:8-10 (shape list
with ragged M, fp16 + bf16), validate_epilogues.sh:19-36 (POSTOP 0..4 x DT /
fp32 output), int2_fp16_upcvt/main.cpp:351-353 (repeated launches reproduce
the first bit for bit).  Gold: the oracle's restatement of compute_gold +
epilogue_ref (int2_fp16_upcvt/main.cpp:79-98, common/epilogue.hpp:98-115).
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_raw, host_f32, host_u16, host_u32, xetla_cmp
from tests.gpu_util import int2_gold, int2_inputs, int2_run

pytestmark = pytest.mark.gpu

# ragged M (not a multiple of the 128-row tile), N down to one 16-column block,
# N not a multiple of the 128-column tile, long K
SHAPES = [(17, 256, 48), (33, 1024, 272), (64, 4096, 4096), (100, 2048, 1040), (128, 512, 128),
          (129, 640, 2064), (256, 4096, 4096), (300, 1408, 2048), (1024, 4096, 1024),
          (77, 14336, 512), (2048, 2048, 16)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_parity(dev, orc, M, K, N, bf16):
    import torch
    import ternocl_amd as T
    print(f"gemm parity M={M} K={K} N={N} bf16={bf16}", flush=True)
    A, B, S, other, bias_f = int2_inputs(2000 + M + K + N, M, K, N, bf16)
    dC, _ = int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    want, _ = int2_gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("M", [1, 5, 16])
def test_gemm_engine_small_m(dev, orc, M):
    """The GEMM engine forced at decode sizes (rows beyond M are masked)."""
    import torch
    import ternocl_amd as T
    K, N, bf16 = 2048, 528, True
    print(f"gemm engine M={M}", flush=True)
    A, B, S, other, bias_f = int2_inputs(31 + M, M, K, N, bf16)
    dC, _ = int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 3, False, tile=T.gemv_tile(T.GEMM))
    want, _ = int2_gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 3, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_gemm_epilogues(dev, orc, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N = 200, 1024, 528
    print(f"gemm epilogue bf16={bf16} postop={postop} f32={out_f32}", flush=True)
    A, B, S, other, bias_f = int2_inputs(70 + postop, M, K, N, bf16)
    dC, _ = int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    want, _ = int2_gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    if out_f32:
        got, ref = host_f32(dC), want
    else:
        got, ref = formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16)
    bad, dmax = allclose_report(got, ref)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_reference_distribution_rule(dev, orc, bf16):
    """The reference driver's own inputs (A ~ U[-5,5], S ~ U[0.75,15.75]) and
    pass rule (xetla_buff_cmp), at a prefill shape."""
    import torch
    import ternocl_amd as T
    M, K, N = 96, 5120, 1024
    A, B, S, other, bias_f = int2_inputs(98, M, K, N, bf16, ref_dist=True)
    dC, _ = int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    want, _ = int2_gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    assert xetla_cmp(host_u16(dC), want, bf16) == 0


def test_gemm_deterministic(dev, orc):
    import torch
    import ternocl_amd as T
    M, K, N, bf16 = 333, 2048, 1040, False
    A, B, S, other, bias_f = int2_inputs(6, M, K, N, bf16)
    outs = [host_u16(int2_run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False)[0])
            for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"


def test_gemm_explicit_gemv_engine_rejected_above_16(dev):
    import torch
    import ternocl_amd as T
    M, K, N = 17, 128, 16
    A = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    B = torch.zeros((K // 16, N), dtype=torch.int32, device="cuda")
    S = torch.zeros((K // 128, N), dtype=torch.float16, device="cuda")
    C = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    for eng in (T.VALU, T.MFMA):
        with pytest.raises(T.TernoclError) as e:
            T.int2_fp16_upcvt_gemm(A, B, S, C, None, None, M, N, K, tile=T.gemv_tile(eng))
        assert e.value.status == 2


@pytest.mark.parametrize("bf16", [False, True])
def test_gemm_decode_bit_exact(dev, bf16):
    """The GEMM's in-register B fragment at unit scale: dword 4h+i of a word
    holds rows (4h+i, 4h+i+8).  fp16: code << 14 in each half times 1.0, i.e.
    exactly 2x the signed weight (+-2.0 / +-0); bf16: the byte-table decode,
    +1.0 / -1.0 / +0 (code 2 reads as 0, as the reference's select decode)."""
    import torch
    import ternocl_amd as T
    K, N = 256, 64
    g = synth.rng(8)
    B = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)  # all four codes
    D = torch.empty(((K // 16) * N * 8,), dtype=torch.int32, device="cuda")
    T.int2_gemv_decode(dev_raw(B), D, K, N, bf16, engine=T.GEMM)
    torch.cuda.synchronize()
    got = host_u32(D).reshape(K // 16, N, 8)
    codes = ((B[..., None] >> (2 * np.arange(16, dtype=np.uint32))) & 3).astype(np.uint32)
    if bf16:
        lut = np.array([0x0000, 0x3F80, 0x0000, 0xBF80], np.uint32)
    else:
        lut = np.array([0x0000, 0x4000, 0x8000, 0xC000], np.uint32)
    for d in range(8):
        j = d  # dword 4h+i covers row j = 4h+i (low half) and j + 8 (high half)
        want = lut[codes[..., j]] | (lut[codes[..., j + 8]] << 16)
        assert np.array_equal(got[..., d], want.astype(np.uint32)), f"dword {d}"
