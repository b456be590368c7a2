"""GPU parity of the BITCOS GEMV, its slice ranks and decode, and the Hadamard
transform, through the C ABI.

Reference test design followed: bitcos_fp16_upcvt/validate.sh (shape list,
fp16 + bf16, zero densities, LS choices) and zsweep.sh (z sweep); the host
gold compute_gold (bitcos_fp16_upcvt/main.cpp:64-86) restated by the oracle;
the slice ranks of common/bitcos.hpp:81-94.  The reference has no Hadamard
test: the transform is checked bit for bit against the oracle's restatement of
hadamard_fwht.cl, which the CPU suite pins to the Sylvester matrix.
Bars: decode, slice ranks and FWHT bit-exact; C within 1e-3 + 1e-2 |ref|.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_dt, dev_raw, host_u16, host_u32

pytestmark = pytest.mark.gpu


# ---- Hadamard ------------------------------------------------------------------

@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("HB", [256, 512, 1024, 2048, 4096])
@pytest.mark.parametrize("rows,K,use_signs", [(1, 4096, True), (3, 8192, False), (2, 5376, True)])
def test_fwht_bit_exact(dev, orc, HB, bf16, rows, K, use_signs):
    import torch
    import ternocl_amd as T
    tail = K % HB
    if tail & (tail - 1):
        pytest.skip("K % HB is not a power of two for this pair")
    print(f"fwht HB={HB} rows={rows} K={K} signs={use_signs} bf16={bf16}", flush=True)
    g = synth.rng(HB + K + rows)
    x = synth.activations(g, (rows, K), bf16)
    s = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
    dy = torch.zeros((rows, K), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    T.hadamard_fwht(dev_dt(x, bf16), dev_raw(s), dy, rows, K, HB, use_signs)
    torch.cuda.synchronize()
    want = orc.fwht(x, s, rows, K, HB, use_signs, bf16)
    assert np.array_equal(host_u16(dy), want)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("case", ["tail4", "tail8", "offset", "tail256_hb4096"])
def test_fwht_both_kernels_bit_exact(dev, orc, bf16, case):
    """The register kernel (aligned rows, K % 8 == 0, a tail of 0 or >= 8) and the LDS
    kernel (everything else: a 4-element tail, rows that are not 16-byte aligned) give
    the oracle's bits; the 8-element tail is the register kernel's smallest block."""
    import torch
    import ternocl_amd as T
    rows, K, HB, off = {"tail4": (2, 1028, 1024, 0), "tail8": (2, 520, 512, 0), "offset": (3, 4096, 512, 1),
                        "tail256_hb4096": (1, 4352, 4096, 0)}[case]
    print(f"fwht kernels case={case} rows={rows} K={K} HB={HB} bf16={bf16}", flush=True)
    g = synth.rng(K + HB + off)
    x = synth.activations(g, (rows, K), bf16)
    s = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
    dt = torch.bfloat16 if bf16 else torch.float16
    xb = torch.zeros(rows * K + off, dtype=dt, device="cuda")  # off: x and y start one element in
    yb = torch.zeros(rows * K + off, dtype=dt, device="cuda")
    xb[off:].copy_(dev_dt(x, bf16).reshape(-1))
    T.hadamard_fwht(xb[off:], dev_raw(s), yb[off:], rows, K, HB, True)
    torch.cuda.synchronize()
    want = orc.fwht(x, s, rows, K, HB, True, bf16)
    assert np.array_equal(host_u16(yb[off:]).reshape(rows, K), want)


def test_fwht_rejects_bad_shapes(dev):
    import torch
    import ternocl_amd as T
    x = torch.zeros(1000, dtype=torch.float16, device="cuda")
    with pytest.raises(T.TernoclError):
        T.hadamard_fwht(x, None, x, 1, 1000, 512, False)  # tail 488 is not a power of two
    with pytest.raises(T.TernoclError):
        T.hadamard_fwht(x, None, x, 1, 1024, 100, False)  # HB not a power of two
    with pytest.raises(T.TernoclError):
        T.hadamard_fwht(x, None, x, 1, 1024, 512, True)  # signs missing


# ---- BITCOS ----------------------------------------------------------------------

def _bitcos_case(seed, M, K, N, z, bf16):
    g = synth.rng(seed)
    A = synth.activations(g, (M, K), bf16)
    codes = synth.ternary_codes(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = g.standard_normal(N).astype(np.float32) * np.float32(0.1)
    return A, codes, S, other, bias_f


def _bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, postop, out_f32, ws=None):
    dA, dB, dS, dO = dev_dt(A, bf16), dev_raw(buf), dev_dt(S, bf16), dev_dt(other, bf16)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    if out_f32:
        dBias = torch.from_numpy(bias_f).cuda()
        dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    else:
        dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
        dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
    T.bitcos_fp16_upcvt_gemm(dA, dB, dS, dSR if ls > 1 else None, dC, dO, dBias, M, N, K, ls, postop, out_f32,
                             ws=ws)
    torch.cuda.synchronize()
    return dC


def _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, postop, out_f32):
    acc = orc.bitcos_gold(A, buf, S, M, K, N, bf16)
    bias = bias_f if out_f32 else formats.f32_to_dt(bias_f, bf16)
    return orc.epilogue(acc, other, bias, postop, out_f32, bf16)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("z", [0.0, 0.3, 0.5, 0.7, 1.0])
def test_bitcos_dequant_bit_exact(dev, orc, z, bf16):
    import torch
    import ternocl_amd as T
    K, N = 1024, 96
    A, codes, S, _, _ = _bitcos_case(int(z * 10) + 1, 1, K, N, z, bf16)
    buf = formats.bitcos_pack(codes)
    dW = torch.zeros((K, N), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    T.bitcos_dequant(dev_raw(buf), dev_dt(S, bf16), dW, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(dW), orc.bitcos_dequant(buf, S, K, N))


@pytest.mark.parametrize("ls", [2, 3, 4, 7, 16])
def test_bitcos_slice_ranks(dev, orc, ls):
    import torch
    import ternocl_amd as T
    K, N = 21504, 80  # divisible by 64 * ls for every ls tested
    _, codes, _, _, _ = _bitcos_case(ls, 1, K, N, 0.4, False)
    buf = formats.bitcos_pack(codes)
    dSR = torch.zeros((ls - 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dev_raw(buf), dSR, K, N, ls)
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(dSR), orc.bitcos_slice_ranks(buf, K, N, ls))


SHAPES = [(1, 256, 16, 1), (1, 1024, 272, 4), (2, 4096, 1040, 8), (3, 2048, 528, 2),
          (4, 5376, 2048, 7), (5, 1536, 336, 6), (8, 640, 64, 5), (1, 5376, 21504, 14)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ls", SHAPES)
@pytest.mark.parametrize("z", [0.3, 0.7])
def test_bitcos_gemv_parity(dev, orc, M, K, N, ls, z, bf16):
    import torch
    import ternocl_amd as T
    print(f"bitcos gemv M={M} K={K} N={N} ls={ls} z={z} bf16={bf16}", flush=True)
    A, codes, S, other, bias_f = _bitcos_case(4000 + M + K + N + ls, M, K, N, z, bf16)
    buf = formats.bitcos_pack(codes)
    dC = _bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 0, False)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ls", SHAPES)
def test_bitcos_gemv_split_launch(dev, orc, M, K, N, ls, bf16):
    """With the workspace a strip's slices may run on several workgroups (here
    every shape but N = 256 strips' worth: too few strips, or 336 on 256 CUs);
    the last adds their sums in order.  The gold within 1e-3 + 1e-2 |ref| with
    the bias + residual epilogue, the same bits on repeated calls, the counters
    back at zero."""
    import torch
    import ternocl_amd as T
    wsb = T.bitcos_gemv_ws_bytes(N, ls)
    print(f"bitcos split M={M} K={K} N={N} ls={ls} bf16={bf16} ws={wsb}", flush=True)
    if ls > 1:
        assert wsb > 0
    A, codes, S, other, bias_f = _bitcos_case(6000 + M + K + N + ls, M, K, N, 0.5, bf16)
    buf = formats.bitcos_pack(codes)
    ws = torch.zeros(max(wsb, 16), dtype=torch.uint8, device="cuda")
    outs = [host_u16(_bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False, ws=ws))
            for _ in range(3)]
    assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"
    cnt_bytes = ((N + 63) // 64 * 4 + 255) // 256 * 256
    assert not ws[:cnt_bytes].any().item(), "strip counters not left at zero"
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 5, False)
    bad, dmax = allclose_report(formats.dt_to_f32(outs[0], bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("z", [0.0, 1.0])
def test_bitcos_gemv_extreme_density(dev, orc, z):
    """All weights non-zero (every sign bit consumed) and all zero (empty sign streams)."""
    import torch
    import ternocl_amd as T
    M, K, N, ls, bf16 = 1, 2048, 144, 4, False
    A, codes, S, other, bias_f = _bitcos_case(9, M, K, N, z, bf16)
    buf = formats.bitcos_pack(codes)
    dC = _bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 0, True)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 0, True)
    bad, dmax = allclose_report(dC.cpu().numpy(), want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_bitcos_gemv_epilogues(dev, orc, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N, ls = 2, 1024, 528, 4
    A, codes, S, other, bias_f = _bitcos_case(60 + postop, M, K, N, 0.5, bf16)
    buf = formats.bitcos_pack(codes)
    dC = _bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, postop, out_f32)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    got = dC.cpu().numpy() if out_f32 else formats.dt_to_f32(host_u16(dC), bf16)
    ref = want if out_f32 else formats.dt_to_f32(want, bf16)
    bad, dmax = allclose_report(got, ref)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_bitcos_ls_invariance_and_determinism(dev, orc):
    """Every slice count gives the reference result; repeated calls are bit-identical."""
    import torch
    import ternocl_amd as T
    M, K, N, bf16 = 1, 5376, 512, False
    A, codes, S, other, bias_f = _bitcos_case(21, M, K, N, 0.5, bf16)
    buf = formats.bitcos_pack(codes)
    want = formats.dt_to_f32(_bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 0, False), bf16)
    for ls in (1, 2, 3, 4, 6, 7, 12, 14):
        out = host_u16(_bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 0, False))
        bad, dmax = allclose_report(formats.dt_to_f32(out, bf16), want)
        assert bad == 0, f"ls={ls}: {bad} bad (max |d| {dmax})"
        again = host_u16(_bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 0, False))
        assert np.array_equal(out, again)


def test_bitcos_hadamard_pipeline(dev, orc):
    """The decode-step workload: sign flip + FWHT (HB 512) on the activation, then the
    BITCOS GEMV on the transformed activation (K = 5376: a 256-element tail block)."""
    import torch
    import ternocl_amd as T
    M, K, N, ls, bf16, HB = 1, 5376, 1024, 7, False, 512
    g = synth.rng(99)
    x = synth.activations(g, (M, K), bf16)
    sgn = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
    codes = synth.ternary_codes(g, K, N, 0.5)
    S = synth.scales(g, K, N, bf16)
    buf = formats.bitcos_pack(codes)
    dx, dy = dev_dt(x, bf16), torch.zeros((M, K), dtype=torch.float16, device="cuda")
    T.hadamard_fwht(dx, dev_raw(sgn), dy, M, K, HB, True)
    dB, dS = dev_raw(buf), dev_dt(S, bf16)
    dSR = torch.zeros((ls - 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    dC = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    T.bitcos_fp16_upcvt_gemm(dy, dB, dS, dSR, dC, None, None, M, N, K, ls)
    torch.cuda.synchronize()
    y = orc.fwht(x, sgn, M, K, HB, True, bf16)
    assert np.array_equal(host_u16(dy), y)
    want = formats.dt_to_f32(orc.epilogue(orc.bitcos_gold(y, buf, S, M, K, N, bf16), None, None, 0, False, bf16), bf16)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("z", [0.3, 0.5, 0.7])
def test_bitcos_c4_default_plan(dev, orc, z):
    """The decode-step workload as bench.py dispatches it: M=1 K=5376 N=21504 fp16, sign flip
    + FWHT (HB 512), then the BITCOS GEMV at the library's slice count
    (ternocl_bitcos_pick_ls: 12) through the split launch (ternocl_bitcos_fp16_upcvt_gemm_ws:
    three workgroups per strip) and unsplit; every output within 1e-3 + 1e-2 |ref| of the
    host gold on the transformed activation, the split launch bit-identical on repeated
    calls with its counters back at zero."""
    import torch
    import ternocl_amd as T
    M, K, N, bf16, HB = 1, 5376, 21504, False, 512
    ls = T.bitcos_pick_ls(M, N, K)
    wsb = T.bitcos_gemv_ws_bytes(N, ls)
    assert ls == 12 and wsb > 0
    print(f"bitcos C4 default plan z={z} ls={ls} ws={wsb}", flush=True)
    g = synth.rng(44 + int(10 * z))
    x = synth.activations(g, (M, K), bf16)
    sgn = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
    buf, _ = synth.bitcos_weights(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    dy = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    T.hadamard_fwht(dev_dt(x, bf16), dev_raw(sgn), dy, M, K, HB, True)
    dB, dS = dev_raw(buf), dev_dt(S, bf16)
    dSR = torch.zeros((ls - 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
    outs = []
    for w in (ws, ws, None):
        dC = torch.zeros((M, N), dtype=torch.float16, device="cuda")
        T.bitcos_fp16_upcvt_gemm(dy, dB, dS, dSR, dC, None, None, M, N, K, ls, ws=w)
        torch.cuda.synchronize()
        outs.append(host_u16(dC))
    assert np.array_equal(outs[0], outs[1]), "split launch not deterministic"
    assert not ws[:T.WS_HEADER_BYTES].any().item(), "split launch left a counter set"
    y = orc.fwht(x, sgn, M, K, HB, True, bf16)
    assert np.array_equal(host_u16(dy), y)
    want = formats.dt_to_f32(orc.epilogue(orc.bitcos_gold(y, buf, S, M, K, N, bf16), None, None, 0, False, bf16), bf16)
    for name, out in (("split", outs[0]), ("unsplit", outs[2])):
        bad, dmax = allclose_report(formats.dt_to_f32(out, bf16), want)
        assert bad == 0, f"{name}: {bad} bad (max |d| {dmax})"


def test_bitcos_rejects_bad_ls(dev):
    import torch
    import ternocl_amd as T
    A = torch.zeros((1, 1024), dtype=torch.float16, device="cuda")
    B = torch.zeros(4096, dtype=torch.int32, device="cuda")
    S = torch.zeros((8, 16), dtype=torch.float16, device="cuda")
    C = torch.zeros((1, 16), dtype=torch.float16, device="cuda")
    with pytest.raises(T.TernoclError):
        T.bitcos_fp16_upcvt_gemm(A, B, S, None, C, None, None, 1, 16, 1024, ls=3)  # 1024 % 192
    with pytest.raises(T.TernoclError):
        T.bitcos_fp16_upcvt_gemm(A, B, S, None, C, None, None, 1, 16, 1024, ls=2)  # SR missing


# ---- BITCOS M-tiled prefill (re-pack to int2 + the int2 prefill GEMM) -------------------

@pytest.mark.parametrize("K,N,ls", [(256, 16, 1), (1024, 272, 4), (5376, 1040, 14), (2048, 96, 16)])
@pytest.mark.parametrize("z", [0.0, 0.5, 1.0])
def test_bitcos_to_int2_bit_exact(dev, orc, K, N, ls, z):
    """The re-pack reproduces the int2 packing of the same codes bit for bit, through every
    slice count (each slice enters its columns' sign streams at the slice ranks)."""
    import torch
    import ternocl_amd as T
    print(f"bitcos to int2 K={K} N={N} ls={ls} z={z}", flush=True)
    _, codes, _, _, _ = _bitcos_case(700 + K + N + ls, 1, K, N, z, False)
    buf = formats.bitcos_pack(codes)
    dB = dev_raw(buf)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    dW = torch.full((K // 16, N), -1, dtype=torch.int32, device="cuda")
    T.bitcos_to_int2(dB, dSR if ls > 1 else None, ls, dW, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_u32(dW), formats.pack_int2(codes))


def _bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, postop, out_f32, in_tile=False):
    """The M-tiled entry: in_tile = the reference's call (no workspace, the tiles decode BITCOS),
    else the re-pack into a workspace."""
    dA, dB, dS, dO = dev_dt(A, bf16), dev_raw(buf), dev_dt(S, bf16), dev_dt(other, bf16)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    if out_f32:
        dBias = torch.from_numpy(bias_f).cuda()
        dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    else:
        dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
        dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
    ws = None if in_tile else torch.empty(T.bitcos_gemm_mt_ws_bytes(K, N), dtype=torch.uint8, device="cuda")
    T.bitcos_fp16_upcvt_gemm_mt(dA, dB, dS, dSR if ls > 1 else None, dC, dO, dBias, M, N, K, ls, ws,
                                postop, out_f32)
    torch.cuda.synchronize()
    return dC


MT_SHAPES = [(1, 256, 16, 1), (16, 1024, 272, 4), (64, 5376, 1024, 7), (130, 2048, 528, 8),
             (257, 1536, 96, 6), (1024, 5376, 256, 14),
             (2048, 256, 6144, 4)]  # 16 x 12 = 192 tiles of 128 x 512: the wide tile


@pytest.mark.parametrize("in_tile", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ls", MT_SHAPES)
def test_bitcos_gemm_mt_parity(dev, orc, M, K, N, ls, bf16, in_tile):
    """Ragged M (1, 130, 257), the reference's M >= 64 prefill range, the C4 K and a shape on
    the 128 x 512 tile; both paths (the tiles decoding BITCOS, and the re-pack)."""
    import torch
    import ternocl_amd as T
    print(f"bitcos mt M={M} K={K} N={N} ls={ls} bf16={bf16} in_tile={in_tile}", flush=True)
    A, codes, S, other, bias_f = _bitcos_case(5000 + M + K + N, M, K, N, 0.5, bf16)
    buf = formats.bitcos_pack(codes)
    dC = _bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 0, False, in_tile)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("in_tile", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_bitcos_gemm_mt_epilogues(dev, orc, postop, out_f32, in_tile):
    import torch
    import ternocl_amd as T
    M, K, N, ls, bf16 = 96, 1024, 272, 4, True
    A, codes, S, other, bias_f = _bitcos_case(80 + postop, M, K, N, 0.3, bf16)
    buf = formats.bitcos_pack(codes)
    dC = _bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, postop, out_f32, in_tile)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    got = dC.cpu().numpy() if out_f32 else formats.dt_to_f32(host_u16(dC), bf16)
    ref = want if out_f32 else formats.dt_to_f32(want, bf16)
    bad, dmax = allclose_report(got, ref)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_bitcos_gemm_mt_matches_gemv_path(dev, orc):
    """The M-tiled path and the row-block GEMV path agree (both within tolerance of the gold),
    and the M-tiled path is deterministic."""
    import torch
    import ternocl_amd as T
    M, K, N, ls, bf16 = 24, 5376, 512, 14, False
    A, codes, S, other, bias_f = _bitcos_case(31, M, K, N, 0.7, bf16)
    buf = formats.bitcos_pack(codes)
    a = host_u16(_bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False))
    b = host_u16(_bitcos_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False))
    bad, dmax = allclose_report(formats.dt_to_f32(a, bf16), formats.dt_to_f32(b, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    again = host_u16(_bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False))
    assert np.array_equal(a, again)


@pytest.mark.parametrize("z", [0.0, 1.0])
def test_bitcos_gemm_mt_in_tile_extremes(dev, orc, z):
    """The tiles' decode with every weight non-zero (a sign bit per row, the rank crossing every
    sign word) and with none (empty sign streams), and the same bits as the re-pack path, which
    runs the same int2 engine on the re-packed words."""
    import torch
    import ternocl_amd as T
    M, K, N, ls, bf16 = 160, 2048, 336, 8, False
    A, codes, S, other, bias_f = _bitcos_case(90 + int(z), M, K, N, z, bf16)
    buf = formats.bitcos_pack(codes)
    a = host_u16(_bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False, True))
    b = host_u16(_bitcos_mt_run(T, torch, A, buf, S, other, bias_f, M, K, N, ls, bf16, 5, False, False))
    assert np.array_equal(a, b)
    want = _bitcos_gold(orc, A, buf, S, other, bias_f, M, K, N, bf16, 5, False)
    bad, dmax = allclose_report(formats.dt_to_f32(a, bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_bitcos_gemm_mt_rejects_small_workspace(dev):
    import torch
    import ternocl_amd as T
    M, K, N = 32, 1024, 64
    A = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    B = torch.zeros(K // 32 * N + N + 8, dtype=torch.int32, device="cuda")
    S = torch.zeros((K // 128, N), dtype=torch.float16, device="cuda")
    C = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    small = torch.empty(T.bitcos_gemm_mt_ws_bytes(K, N) - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(T.TernoclError):
        T.bitcos_fp16_upcvt_gemm_mt(A, B, S, None, C, None, None, M, N, K, 1, small)
    # no workspace: the tiles decode the (all-zero) weights themselves
    C.fill_(1.0)
    T.bitcos_fp16_upcvt_gemm_mt(A, B, S, None, C, None, None, M, N, K, 1, None)
    torch.cuda.synchronize()
    assert not C.any().item()


# ---- the transform fused into the GEMV (ternocl_bitcos_fwht_gemm_ws) ----------------
# (M, K, N, ls, HB, z): C4 at its default plan, a 256-element tail block, HB 256,
# several rows (one and two launches of 4 rows), slices that straddle blocks
FUSED = [(1, 5376, 21504, 0, 512, 0.5), (1, 5376, 21504, 0, 512, 0.3), (1, 5376, 21504, 0, 512, 0.7),
         (2, 4096, 1040, 8, 512, 0.5), (3, 2048, 528, 4, 256, 0.4), (4, 5376, 2048, 7, 512, 0.5),
         (5, 1536, 336, 6, 512, 0.6), (1, 2304, 4096, 6, 256, 0.5)]


@pytest.mark.parametrize("use_signs", [True, False])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ls,HB,z", FUSED)
def test_bitcos_fwht_fused_bit_exact(dev, orc, M, K, N, ls, HB, z, bf16, use_signs):
    """The fused launch gives, bit for bit, what the transform followed by the GEMV gives
    (split launch and one workgroup per strip), and the GEMV's result within the rule of
    the host gold on the oracle's transform."""
    import torch
    import ternocl_amd as T
    ls = ls or T.bitcos_pick_ls(M, N, K)
    wsb = T.bitcos_gemv_ws_bytes(N, ls)
    print(f"bitcos fused fwht M={M} K={K} N={N} ls={ls} HB={HB} z={z} bf16={bf16} signs={use_signs} ws={wsb}",
          flush=True)
    g = synth.rng(8000 + M + K + N + HB)
    x = synth.activations(g, (M, K), bf16)
    sgn = (g.integers(0, 2, K, dtype=np.int8) * 2 - 1).astype(np.int8)
    buf, _ = synth.bitcos_weights(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias = formats.f32_to_dt(g.standard_normal(N).astype(np.float32) * np.float32(0.1), bf16)
    dt = torch.bfloat16 if bf16 else torch.float16
    dx, ds = dev_dt(x, bf16), dev_raw(sgn)
    dB, dS, dO, dBias = dev_raw(buf), dev_dt(S, bf16), dev_dt(other, bf16), dev_dt(bias, bf16)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    SR = dSR if ls > 1 else None
    dy = torch.zeros((M, K), dtype=dt, device="cuda")
    T.hadamard_fwht(dx, ds, dy, M, K, HB, use_signs)
    for w in ([torch.zeros(wsb, dtype=torch.uint8, device="cuda")] if wsb else []) + [None]:
        ref = torch.zeros((M, N), dtype=dt, device="cuda")
        T.bitcos_fp16_upcvt_gemm(dy, dB, dS, SR, ref, dO, dBias, M, N, K, ls, 5, False, ws=w)
        got = torch.full((M, N), 7.0, dtype=dt, device="cuda")
        T.bitcos_fwht_gemm(dx, ds, HB, dB, dS, SR, got, dO, dBias, M, N, K, ls, 5, False, ws=w, use_signs=use_signs)
        torch.cuda.synchronize()
        assert np.array_equal(host_u16(got), host_u16(ref)), f"fused differs (ws={w is not None})"
    y = orc.fwht(x, sgn, M, K, HB, use_signs, bf16)
    assert np.array_equal(host_u16(dy), y)
    want = orc.epilogue(orc.bitcos_gold(y, buf, S, M, K, N, bf16), other, bias, 5, False, bf16)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(got), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_bitcos_fwht_fused_rejects(dev):
    """Host checks of the fused entry: HB past one wave (1024), a tail that is not a power
    of two, x not 16-byte aligned."""
    import torch
    import ternocl_amd as T
    K, N = 4096, 64
    x = torch.zeros((1, K + 8), dtype=torch.float16, device="cuda")
    s = torch.ones(K, dtype=torch.int8, device="cuda")
    B = torch.zeros(K // 32 * N + N + 4, dtype=torch.int32, device="cuda")
    S = torch.zeros((K // 128, N), dtype=torch.float16, device="cuda")
    C = torch.zeros((1, N), dtype=torch.float16, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.bitcos_fwht_gemm(x, s, 1024, B, S, None, C, None, None, 1, N, K, 1)
    assert e.value.status == 2
    with pytest.raises(T.TernoclError) as e:
        T.bitcos_fwht_gemm(x, s, 512, B, S, None, C, None, None, 1, N, 4096 + 384, 1)
    assert e.value.status == 2
    with pytest.raises(T.TernoclError) as e:
        T.bitcos_fwht_gemm(x[:, 1:], s, 512, B, S, None, C, None, None, 1, N, K, 1)
    assert e.value.status == 1
