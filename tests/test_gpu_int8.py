"""GPU parity of the int2 x int8 prefill path (quant_a + s8 x s2 GEMM) through the C ABI.

Reference test design followed: int2_via_int2_x_int8_dpas/validate.sh (shape
list with ragged M, fp16 + bf16, the M-tiled kernel for M >= 64), its host gold
compute_scale_a / compute_gold (int2_via_int2_x_int8_dpas/main.cpp:82-121) and
the epilogue sweep of validate_epilogues.sh.  Bars: SA and Aq bit-exact with the
oracle's quantization; the B decode bit-exact with its closed form; C within
1e-3 + 1e-2 |ref| of the oracle's fp32 gold (the int32 dots are exact, only the
fp32 rescale may round differently).
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_dt, dev_raw, host_u16, host_u32

pytestmark = pytest.mark.gpu


def _quant(T, torch, A, M, K, bf16):
    dA = dev_dt(A, bf16)
    dSA = torch.zeros((K // 128, T.ldsa(M)), dtype=dA.dtype, device="cuda")
    dAq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    T.quant_a(dA, dSA, dAq, M, K)
    torch.cuda.synchronize()
    return dA, dSA, dAq


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K", [(1, 128), (3, 4096), (31, 256), (64, 1024), (100, 2048), (1024, 4096)])
def test_quant_a_bit_exact(dev, orc, M, K, bf16):
    import torch
    import ternocl_amd as T
    print(f"quant_a M={M} K={K} bf16={bf16}", flush=True)
    g = synth.rng(11 + M + K)
    A = synth.activations(g, (M, K), bf16, sigma=3.0)
    A[0, :5] = formats.f32_to_dt(np.array([0.0, -0.0, 1e-30, -2.5, 65504.0 if not bf16 else 3e38], np.float32), bf16)
    _, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    SA = orc.scale_a(A, M, K, bf16)
    Aq = orc.quant_a(A, SA, M, K, bf16)
    got_sa = host_u16(dSA)
    assert np.array_equal(got_sa[:, :M], SA[:, :M]), "SA differs from the oracle"
    assert np.array_equal(dAq.cpu().numpy(), Aq), "Aq differs from the oracle"


@pytest.mark.parametrize("bf16", [False, True])
def test_quant_a_scale_every_absmax(dev, orc, bf16):
    """SA = DT(127 / max(x, FLT_EPSILON)) for every positive finite DT value x
    as a group's absmax (one group per value; the rest of the group is
    smaller): checks the correctly rounded divide and the epsilon floor."""
    import torch
    import ternocl_amd as T
    top = 0x7BFF if not bf16 else 0x7F7F
    xs = np.arange(0, top + 1, dtype=np.uint16)
    K = 128 * 64
    M = (xs.size + 63) // 64
    A = np.zeros((M, K), np.uint16)
    flat = np.zeros(M * 64, np.uint16)
    flat[: xs.size] = xs
    A.reshape(M, 64, 128)[:, :, 0] = flat.reshape(M, 64)
    # a smaller negative element in each group: |.| <= x, so absmax stays x
    A.reshape(M, 64, 128)[:, :, 1] = flat.reshape(M, 64) | 0x8000
    print(f"quant_a every absmax bf16={bf16} M={M}", flush=True)
    _, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    SA = orc.scale_a(A, M, K, bf16)
    assert np.array_equal(host_u16(dSA)[:, :M], SA[:, :M])
    assert np.array_equal(dAq.cpu().numpy(), orc.quant_a(A, SA, M, K, bf16))


def _int8_case(seed, M, K, N, bf16, ref_dist=False, all_codes=False):
    g = synth.rng(seed)
    if ref_dist:  # the reference driver's A ~ U[-5, 5] (int2_via_int2_x_int8_dpas/main.cpp:232-245)
        A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
    else:
        A = synth.activations(g, (M, K), bf16)
    if all_codes:  # code 2 (-2) included: the s8 x s2 contract reads it as two's complement
        B = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    else:
        B = synth.int2_weights(g, K, N)
    SB = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = g.standard_normal(N).astype(np.float32) * np.float32(0.1)
    return A, B, SB, other, bias_f


def _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32):
    _, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    dB, dSB, dO = dev_raw(B), dev_dt(SB, bf16), dev_dt(other, bf16)
    if out_f32:
        dBias = torch.from_numpy(bias_f).cuda()
        dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    else:
        dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
        dC = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC, dO, dBias, M, N, K, postop, out_f32)
    torch.cuda.synchronize()
    return dC


def _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32):
    SA = orc.scale_a(A, M, K, bf16)
    acc = orc.int8_gold(A, B, SA, SB, M, K, N, bf16)
    bias = bias_f if out_f32 else formats.f32_to_dt(bias_f, bf16)
    return orc.epilogue(acc, other, bias, postop, out_f32, bf16)


def _as_f32(out, out_f32, bf16):
    return out if out_f32 else formats.dt_to_f32(out, bf16)


SHAPES = [(1, 256, 16), (7, 1024, 272), (64, 4096, 4096), (100, 2048, 1040), (128, 512, 128),
          (129, 640, 2064), (256, 4096, 4096), (1024, 4096, 1024), (77, 14336, 512), (2048, 2048, 16)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", SHAPES)
def test_int8_gemm_parity(dev, orc, M, K, N, bf16):
    import torch
    import ternocl_amd as T
    print(f"int8 gemm M={M} K={K} N={N} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(3000 + M + K + N, M, K, N, bf16)
    dC = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


def _wide_tile(M, N):
    """The library's planner rule: the 128 x 512 tile when it yields >= 192 tiles."""
    return -(-M // 128) * -(-N // 512) >= 192


# shapes the planner sends to the 128 x 512 engine: a ragged last row tile
# (1500 = 11 * 128 + 92), a ragged last column tile (8208 = 16 * 512 + 16:
# one 16-column block of one wave), and an exact tiling
WIDE_SHAPES = [(1500, 256, 8208), (1024, 512, 14336), (1536, 384, 12304)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", WIDE_SHAPES)
def test_int8_gemm_wide_tile_parity(dev, orc, M, K, N, bf16):
    """Every output of the 128 x 512 engine, all 2-bit codes, against the oracle."""
    import torch
    import ternocl_amd as T
    assert _wide_tile(M, N)
    print(f"int8 wide-tile gemm M={M} K={K} N={N} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(4100 + M + N, M, K, N, bf16, all_codes=True)
    dC = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_int8_gemm_wide_tile_epilogues(dev, orc, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N = 1500, 128, 8208
    assert _wide_tile(M, N)
    print(f"int8 wide-tile epilogue postop={postop} out_f32={out_f32} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(191 + postop, M, K, N, bf16)
    dC = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    got = dC.cpu().numpy() if out_f32 else host_u16(dC)
    bad, dmax = allclose_report(_as_f32(got, out_f32, bf16), _as_f32(want, out_f32, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
def test_int8_gemm_all_codes_and_reference_distribution(dev, orc, bf16):
    """Every 2-bit code (code 2 = -2) and the reference driver's A ~ U[-5, 5]."""
    import torch
    import ternocl_amd as T
    M, K, N = 200, 2048, 784
    A, B, SB, other, bias_f = _int8_case(77, M, K, N, bf16, ref_dist=True, all_codes=True)
    dC = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, 0, True)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 0, True)
    bad, dmax = allclose_report(dC.cpu().numpy(), want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_int8_gemm_epilogues(dev, orc, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N = 160, 1024, 528
    print(f"int8 epilogue postop={postop} out_f32={out_f32} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(91 + postop, M, K, N, bf16)
    dC = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    got = dC.cpu().numpy() if out_f32 else host_u16(dC)
    bad, dmax = allclose_report(_as_f32(got, out_f32, bf16), _as_f32(want, out_f32, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_int8_gemm_deterministic(dev, orc):
    """Repeated launches reproduce the first bit for bit (int2_via_int2_x_int8_dpas/main.cpp:379-383)."""
    import torch
    import ternocl_amd as T
    M, K, N, bf16 = 300, 2048, 1024, True
    A, B, SB, other, bias_f = _int8_case(5, M, K, N, bf16)
    first = host_u16(_int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, 5, False))
    for _ in range(3):
        again = host_u16(_int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, 5, False))
        assert np.array_equal(first, again)


def test_s8_decode_bit_exact(dev):
    """The B fragment bytes equal the 2-bit two's-complement values of rows 4b + i."""
    import torch
    import ternocl_amd as T
    K, N = 256, 48
    g = synth.rng(3)
    B = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    dD = torch.zeros((K // 16, N, 4), dtype=torch.int32, device="cuda")
    T.int2_s8_decode(dev_raw(B), dD, K, N)
    torch.cuda.synchronize()
    got = host_u32(dD).view(np.int8).reshape(K // 16, N, 4, 4)  # [kp][n][i][b]
    codes = (B[:, :, None] >> (2 * np.arange(16, dtype=np.uint32))[None, None, :]) & 3  # [kp][n][row]
    vals = np.where(codes >= 2, codes.astype(np.int16) - 4, codes.astype(np.int16)).astype(np.int8)
    want = vals.reshape(K // 16, N, 4, 4).transpose(0, 1, 3, 2)  # row 4b + i -> [i][b]
    assert np.array_equal(got, want)


def test_int8_gemm_requires_a_or_aq(dev):
    import torch
    import ternocl_amd as T
    with pytest.raises(T.TernoclError):
        T.int2_int8_gemm(None, None, torch.zeros(32, device="cuda"), torch.zeros(16, dtype=torch.int32, device="cuda"),
                         torch.zeros(16, dtype=torch.float16, device="cuda"),
                         torch.zeros(16, dtype=torch.float16, device="cuda"), None, None, 1, 16, 128)


@pytest.mark.parametrize("bf16", [False, True])
def test_quant_a_scales_only(dev, orc, bf16):
    """Aq = None writes SA alone (the reference's quant_a without WRITE_Q), bit-exact."""
    import torch
    import ternocl_amd as T
    M, K = 45, 1024
    A = synth.activations(synth.rng(8), (M, K), bf16)
    dA = dev_dt(A, bf16)
    dSA = torch.zeros((K // 128, T.ldsa(M)), dtype=dA.dtype, device="cuda")
    T.quant_a(dA, dSA, None, M, K)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(dSA)[:, :M], orc.scale_a(A, M, K, bf16)[:, :M])


IN_GEMM_SHAPES = [(1, 256, 16), (100, 2048, 1040), (129, 640, 2064), (1024, 4096, 1024)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", IN_GEMM_SHAPES)
def test_int8_gemm_in_gemm_quantization(dev, orc, M, K, N, bf16):
    """QMODE 1 (A quantized while staged) gives the upfront mode's C bit for bit, and so
    the oracle's within tolerance; the reference driver's A ~ U[-5, 5] and every code."""
    import torch
    import ternocl_amd as T
    print(f"int8 in-GEMM quantization M={M} K={K} N={N} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(4000 + M + N, M, K, N, bf16, ref_dist=True, all_codes=True)
    dA, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    dB, dSB, dO = dev_raw(B), dev_dt(SB, bf16), dev_dt(other, bf16)
    dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
    up = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    ig = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    T.int2_int8_gemm(None, dAq, dSA, dB, dSB, up, dO, dBias, M, N, K, 5, False)
    T.int2_int8_gemm(dA, None, dSA, dB, dSB, ig, dO, dBias, M, N, K, 5, False)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(up), host_u16(ig))
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 5, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(ig), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# ---- A off the int8 grid (validate.sh with OFFGRID=F) ---------------------------------

def _offgrid_a(orc, g, M, K, bf16, F):
    """The reference driver's A with --offgrid F (int2_via_int2_x_int8_dpas/main.cpp:250-272):
    A ~ U[-5, 5] fake-quantized per (row, 128-group) as v = sat_int8(rint(A SA)), then moved
    F LSB away from zero, A = DT((v +- F) / SA), so the rounding of A * SA is exercised near
    the int8 grid's midpoints (F = .5: ties before the DT rounding of A)."""
    A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
    SA = orc.scale_a(A, M, K, bf16)
    sa = formats.dt_to_f32(SA[:, :M], bf16).T.repeat(128, axis=1)  # [M, K]
    v = np.clip(np.rint(formats.dt_to_f32(A, bf16) * sa), -128, 127).astype(np.float32)
    off = np.where(v >= 0, np.float32(F), np.float32(-F))
    return formats.f32_to_dt(((v + off) * (np.float32(1.0) / sa)).astype(np.float32), bf16)


OFFGRID_SHAPES = [(77, 128, 48), (129, 256, 272), (4, 6144, 5120), (1, 17408, 5120), (100, 5120, 1024),
                  (1024, 1024, 512)]


@pytest.mark.parametrize("F", [0.5, 0.6])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", OFFGRID_SHAPES)
def test_int8_offgrid_activations(dev, orc, M, K, N, bf16, F):
    """validate.sh's OFFGRID runs: SA and Aq bit-exact with the oracle's quantization on A
    placed F LSB off the int8 grid; C of QMODE 1 (A quantized in the GEMM / GEMV) equal to
    QMODE 0's bit for bit, and within the rule of the oracle's gold."""
    import torch
    import ternocl_amd as T
    print(f"int8 offgrid F={F} M={M} K={K} N={N} bf16={bf16}", flush=True)
    g = synth.rng(int(7000 + 10 * F + M + K + N))
    A = _offgrid_a(orc, g, M, K, bf16, F)
    B = synth.int2_weights(g, K, N)
    SB = synth.scales(g, K, N, bf16)
    dA, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    SA = orc.scale_a(A, M, K, bf16)
    assert np.array_equal(host_u16(dSA)[:, :M], SA[:, :M]), "SA differs from the oracle"
    assert np.array_equal(dAq.cpu().numpy(), orc.quant_a(A, SA, M, K, bf16)), "Aq differs from the oracle"
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    up = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    ig = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    T.int2_int8_gemm(None, dAq, dSA, dB, dSB, up, None, None, M, N, K, 0, False)
    T.int2_int8_gemm(dA, None, dSA, dB, dSB, ig, None, None, M, N, K, 0, False)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(up), host_u16(ig)), "QMODE 1 differs from QMODE 0"
    want = orc.epilogue(orc.int8_gold(A, B, SA, SB, M, K, N, bf16), None, None, 0, False, bf16)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(up), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# ---- M <= 4: the s8 x s2 decode GEMV (int2_int8_dpas.cl:213-215) ------------------

DECODE_SHAPES = [(1, 128, 16), (1, 4096, 14336), (2, 14336, 4096), (3, 2048, 1040), (4, 4096, 4096),
                 (4, 256, 48), (1, 5376, 21504)]


@pytest.mark.parametrize("M,K,N", [(1, 128, 16), (1, 14336, 1024), (2, 4096, 4096), (3, 1024, 48), (4, 2048, 12288)])
def test_int8_gemv_group_dots_exact(dev, M, K, N):
    """With SA = SB = 1 and fp32 output the GEMV returns sum_k Aq * v exactly (integers below
    2^24): the int8 pieces, the two's-complement decode of every code (2 = -2) and the k
    order, checked bit for bit over the whole int8 range."""
    import torch
    import ternocl_amd as T
    print(f"int8 gemv exact dots M={M} K={K} N={N}", flush=True)
    g = synth.rng(600 + M * K + N)
    Aq = g.integers(-128, 128, size=(M, K), dtype=np.int8)
    B = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    one = formats.f32_to_dt(np.ones(1, np.float32), False)[0]
    SA = np.full((K // 128, T.ldsa(M)), one, np.uint16)
    SB = np.full((K // 128, N), one, np.uint16)
    dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    T.int2_int8_gemm(None, torch.from_numpy(Aq).cuda(), dev_dt(SA, False), dev_raw(B), dev_dt(SB, False), dC,
                     None, None, M, N, K, 0, True)
    torch.cuda.synchronize()
    shifts = np.arange(16, dtype=np.uint32) * 2
    codes = ((B[:, None, :] >> shifts[None, :, None]) & 3).astype(np.int64).reshape(K, N)
    v = np.where(codes >= 2, codes - 4, codes)
    want = Aq.astype(np.int64) @ v
    assert np.array_equal(dC.cpu().numpy(), want.astype(np.float32))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", DECODE_SHAPES)
def test_int8_gemv_parity(dev, orc, M, K, N, bf16):
    """M <= 4 against the oracle's s8 x s2 gold within 1e-3 + 1e-2 |ref|, the reference
    driver's A ~ U[-5, 5] and every code; the in-GEMV quantization (QMODE 1) gives the upfront
    mode's C bit for bit."""
    import torch
    import ternocl_amd as T
    print(f"int8 gemv M={M} K={K} N={N} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(5000 + M + N, M, K, N, bf16, ref_dist=True, all_codes=True)
    dA, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    up = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    ig = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
    T.int2_int8_gemm(None, dAq, dSA, dB, dSB, up, None, None, M, N, K, 0, False)
    T.int2_int8_gemm(dA, None, dSA, dB, dSB, ig, None, None, M, N, K, 0, False)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(up), host_u16(ig))
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(up), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# Long K over few strips: the GEMV's K split (a workspace of int2_int8_gemm_ws_bytes),
# 16- and 32-column strips, a last slice shorter than the others (K = 8320: 65 groups).
GEMV_SPLIT_SHAPES = [(1, 14336, 4096), (2, 14336, 4096), (3, 8320, 1040), (4, 16384, 2048), (1, 14336, 528)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", GEMV_SPLIT_SHAPES)
def test_int8_gemv_k_slices(dev, orc, M, K, N, bf16):
    """With the workspace: the oracle's gold within 1e-3 + 1e-2 |ref|; both quantization
    modes bit for bit; the same bits on a second call (the counters back at zero); the call
    without the workspace within the same rule."""
    import torch
    import ternocl_amd as T
    need = T.int2_int8_gemm_ws_bytes(M, N, K)
    print(f"int8 gemv split M={M} K={K} N={N} bf16={bf16} ws={need}", flush=True)
    assert need > 0, "this shape should split"
    A, B, SB, other, bias_f = _int8_case(5200 + M + N, M, K, N, bf16, ref_dist=True, all_codes=True)
    dA, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = []
    for a, aq in ((None, dAq), (dA, None), (None, dAq), (None, None)):
        C = torch.zeros((M, N), dtype=dSB.dtype, device="cuda")
        if a is None and aq is None:  # no workspace: the unsplit launch
            T.int2_int8_gemm(None, dAq, dSA, dB, dSB, C, None, None, M, N, K, 0, False)
        else:
            T.int2_int8_gemm(a, aq, dSA, dB, dSB, C, None, None, M, N, K, 0, False, ws=ws)
        torch.cuda.synchronize()
        outs.append(host_u16(C))
    assert np.array_equal(outs[0], outs[1]), "the two quantization modes differ"
    assert np.array_equal(outs[0], outs[2]), "split results differ between runs"
    assert not ws[: (N // 16) * 4].any().item(), "the strip counters did not return to zero"
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, 0, False)
    for got in (outs[0], outs[3]):
        bad, dmax = allclose_report(formats.dt_to_f32(got, bf16), formats.dt_to_f32(want, bf16))
        assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_int8_gemv_split_epilogues(dev, orc, bf16, postop, out_f32):
    """Every epilogue after the in-order slice sum (M = 3, K = 8320, N = 1040)."""
    import torch
    import ternocl_amd as T
    M, K, N = 3, 8320, 1040
    print(f"int8 gemv split epilogue postop={postop} f32={out_f32} bf16={bf16}", flush=True)
    A, B, SB, other, bias_f = _int8_case(80 + postop, M, K, N, bf16)
    dA, dSA, dAq = _quant(T, torch, A, M, K, bf16)
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    dO = dev_dt(other, bf16)
    dBias = torch.from_numpy(bias_f).cuda() if out_f32 else dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
    ws = torch.zeros(T.int2_int8_gemm_ws_bytes(M, N, K), dtype=torch.uint8, device="cuda")
    C = torch.zeros((M, N), dtype=torch.float32 if out_f32 else dSB.dtype, device="cuda")
    T.int2_int8_gemm(None, dAq, dSA, dB, dSB, C, dO, dBias, M, N, K, postop, out_f32, ws=ws)
    torch.cuda.synchronize()
    got = C.cpu().numpy() if out_f32 else host_u16(C)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    bad, dmax = allclose_report(_as_f32(got, out_f32, bf16), _as_f32(want, out_f32, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_int8_gemv_epilogues(dev, orc, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N = 2, 1024, 528
    A, B, SB, other, bias_f = _int8_case(70 + postop, M, K, N, bf16)
    got = _int8_run(T, torch, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    got = got.cpu().numpy() if out_f32 else host_u16(got)
    want = _int8_gold(orc, A, B, SB, other, bias_f, M, K, N, bf16, postop, out_f32)
    bad, dmax = allclose_report(_as_f32(got, out_f32, bf16), _as_f32(want, out_f32, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
