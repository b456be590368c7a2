"""GPU parity at the reference's own validation shapes and the workload shapes,
through the C ABI with the library's automatic kernel choice (the path a
drop-in caller gets).

Shape lists:
* int2 upcvt: int2_fp16_upcvt/validate.sh:8-10 (M K N; fp16 and bf16);
* int2 x int8 (quant_a + s8 x s2): int2_via_int2_x_int8_dpas/validate.sh:9-10,
  in both quantization modes (QMODE 0 upfront, QMODE 1 in the GEMM), as
  that script runs every shape in both;
* BITCOS: bitcos_fp16_upcvt/validate.sh:8-15 -- its GEMV lines (M <= 8, the
  given slice count and zero density, z = 0.4 where none is given, its
  default, bitcos_fp16_upcvt/main.cpp:47) with and without the split-launch
  workspace, and its M-tiled lines through the M-tiled entry, both with the
  re-pack workspace and without (the tiles decoding BITCOS);
* the prefill workload M=1024 K=4096 N=14336 in both paths, and the decode
  workload's sweep M in {1, 2, 4, 8} x (K, N) in {(4096, 14336), (14336, 4096)}
  in bf16 with the bias + residual epilogue.

At M >= 128 the gold is computed on a row sample: every column, and rows 0, 1,
31, 32, 63, 64, 126, 127 of every 128-row tile plus the last row (both GEMM
tiles are 128 rows high, so every tile and both halves of every wave's rows
are checked).  Bar: |got - ref| <= 1e-3 + 1e-2 |ref| against the oracle's
restatement of the reference's host gold.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_dt, dev_raw, host_f32, host_u16

pytestmark = pytest.mark.gpu

UPCVT_VALIDATE = [(1024, 17408, 5120), (1024, 5120, 14336), (1024, 5120, 34816), (1000, 5120, 4096),
                  (77, 128, 48), (129, 256, 272), (200, 5120, 16384), (1, 5120, 34816), (1, 17408, 5120),
                  (1, 5120, 248320), (1, 6144, 5120), (4, 6144, 5120), (3, 256, 48)]
INT8_VALIDATE = [(1024, 17408, 5120), (1024, 5120, 14336), (1024, 5120, 34816), (1000, 5120, 4096),
                 (77, 128, 48), (129, 256, 272), (200, 5120, 16384), (1, 5120, 34816), (1, 17408, 5120),
                 (1, 5120, 248320), (4, 6144, 5120)]
PREFILL_WORKLOAD = (1024, 4096, 14336)
# 128 x 512 tiles with ragged M and a last column tile of 16 columns
WIDE_RAGGED = (1000, 1024, 12304)
# 128 x 256 tiles (more than 256 tiles of 128 x 128, at most 256 of 128 x 256),
# HALF_RAGGED with ragged M and a last column tile of 16 columns, then one
# row tile of 77 and of 17 rows (the smallest M of the prefill engine)
HALF_RAGGED = (1000, 2048, 6160)
HALF_SHAPES = [(1024, 4096, 6144), (512, 4096, 14336), HALF_RAGGED, (77, 256, 40960), (17, 256, 33040)]


def sample_rows(M: int) -> np.ndarray:
    if M < 128:
        return np.arange(M)
    rows = {M - 1}
    for t0 in range(0, M, 128):
        rows.update(t0 + r for r in (0, 1, 31, 32, 63, 64, 126, 127) if t0 + r < M)
    return np.array(sorted(rows))


def _inputs(seed, M, K, N, bf16):
    g = synth.rng(seed)
    A = synth.activations(g, (M, K), bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = g.standard_normal(N).astype(np.float32) * np.float32(0.1)
    return A, B, S, other, bias_f


def _device_io(torch, S, other, bias_f, M, N, bf16, out_f32):
    dO = dev_dt(other, bf16)
    if out_f32:
        dBias = torch.from_numpy(bias_f).cuda()
        dC = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    else:
        dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
        dC = torch.zeros((M, N), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    return dO, dBias, dC


def _compare(orc, dC, acc_rows, other, bias_f, rows, bf16, postop, out_f32):
    bias = bias_f if out_f32 else formats.f32_to_dt(bias_f, bf16)
    want = orc.epilogue(acc_rows, other[rows], bias, postop, out_f32, bf16)
    if out_f32:
        got, ref = host_f32(dC)[rows], want
    else:
        got, ref = formats.dt_to_f32(host_u16(dC)[rows], bf16), formats.dt_to_f32(want, bf16)
    return allclose_report(got, ref)


def _upcvt_case(dev, orc, M, K, N, bf16, postop=0, out_f32=False, seed=0):
    import torch
    import ternocl_amd as T
    print(f"upcvt M={M} K={K} N={N} bf16={bf16} postop={postop} f32={out_f32}", flush=True)
    A, B, S, other, bias_f = _inputs(seed + 40000 + M + K + N, M, K, N, bf16)
    dO, dBias, dC = _device_io(torch, S, other, bias_f, M, N, bf16, out_f32)
    T.int2_fp16_upcvt_gemm(dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16), dC, dO, dBias, M, N, K,
                           postop, out_f32)
    torch.cuda.synchronize()
    rows = sample_rows(M)
    acc = orc.int2_gold(np.ascontiguousarray(A[rows]), B, S, rows.size, K, N, bf16)
    return _compare(orc, dC, acc, other, bias_f, rows, bf16, postop, out_f32)


def _int8_case(dev, orc, M, K, N, bf16, postop=0, out_f32=False, seed=0, split=False, qmode=0):
    """split: with the K-split workspace -- the same bits on a second call, and within the rule
    of the call without it.  qmode 1: the DT activations are quantized inside the GEMM (SA
    from quant_a), the reference's QMODE 1."""
    import torch
    import ternocl_amd as T
    print(f"int8 M={M} K={K} N={N} bf16={bf16} postop={postop} f32={out_f32} split={split} qmode={qmode}",
          flush=True)
    A, B, SB, other, bias_f = _inputs(seed + 50000 + M + K + N, M, K, N, bf16)
    dA = dev_dt(A, bf16)
    dSA = torch.zeros((K // 128, T.ldsa(M)), dtype=dA.dtype, device="cuda")
    dAq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    dO, dBias, dC = _device_io(torch, SB, other, bias_f, M, N, bf16, out_f32)
    T.quant_a(dA, dSA, dAq, M, K)
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    ws = None
    if split:
        need = T.int2_int8_gemm_ws_bytes(M, N, K)
        assert need > 0, "this shape should split"
        ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    if qmode == 1:
        T.int2_int8_gemm(dA, None, dSA, dB, dSB, dC, dO, dBias, M, N, K, postop, out_f32, ws=ws)
    else:
        T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC, dO, dBias, M, N, K, postop, out_f32, ws=ws)
    torch.cuda.synchronize()
    if split:
        first = dC.clone()
        T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC, dO, dBias, M, N, K, postop, out_f32, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(first, dC), "split-K results differ between runs"
        _, _, dC2 = _device_io(torch, SB, other, bias_f, M, N, bf16, out_f32)
        T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC2, dO, dBias, M, N, K, postop, out_f32)
        torch.cuda.synchronize()
        if out_f32:
            a, b = host_f32(dC), host_f32(dC2)
        else:
            a, b = formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(host_u16(dC2), bf16)
        bad_nows, _ = allclose_report(a, b)
        assert bad_nows == 0, f"{bad_nows} elements differ from the unsplit GEMM beyond the rule"
    rows = sample_rows(M)
    Ar = np.ascontiguousarray(A[rows])
    SA = orc.scale_a(Ar, rows.size, K, bf16)
    # quant_a's output on the sampled rows is bit-exact with the oracle's
    got_q = dAq.cpu().numpy()[rows]
    assert np.array_equal(got_q, orc.quant_a(Ar, SA, rows.size, K, bf16)), "Aq differs from the oracle"
    acc = orc.int8_gold(Ar, B, SA, SB, rows.size, K, N, bf16)
    return _compare(orc, dC, acc, other, bias_f, rows, bf16, postop, out_f32)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", UPCVT_VALIDATE + [PREFILL_WORKLOAD, WIDE_RAGGED])
def test_upcvt_validate_shapes(dev, orc, M, K, N, bf16):
    bad, dmax = _upcvt_case(dev, orc, M, K, N, bf16)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("qmode", [0, 1])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", INT8_VALIDATE + [PREFILL_WORKLOAD, WIDE_RAGGED])
def test_int8_validate_shapes(dev, orc, M, K, N, bf16, qmode):
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16, qmode=qmode)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_wide_tile_epilogues(dev, orc, bf16, postop, out_f32):
    """Every epilogue on the 128 x 512 tile (ragged rows, a 16-column last tile)."""
    M, K, N = WIDE_RAGGED[0], 256, WIDE_RAGGED[2]
    bad, dmax = _upcvt_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop)
    assert bad == 0, f"upcvt: {bad} bad (max |d| {dmax})"
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop)
    assert bad == 0, f"int8: {bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", HALF_SHAPES)
def test_half_tile_shapes(dev, orc, M, K, N, bf16):
    """The 128 x 256 tile against the oracle; with the split-K workspace the call takes the same
    tile (the same bits): with at least 192 of these tiles it beats the split."""
    import torch
    import ternocl_amd as T
    bad, dmax = _upcvt_case(dev, orc, M, K, N, bf16)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"
    A, B, S, other, bias_f = _inputs(40000 + M + K + N, M, K, N, bf16)
    dA, dB, dS = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16)
    outs = []
    for use_ws in (False, True):
        dO, dBias, dC = _device_io(torch, S, other, bias_f, M, N, bf16, False)
        need = T.int2_gemm_ws_bytes(M, N, K)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda") if use_ws and need else None
        T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, 0, False, ws=ws)
        torch.cuda.synchronize()
        outs.append(dC)
    assert torch.equal(outs[0], outs[1]), "the call with a workspace took another path"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_half_tile_epilogues(dev, orc, bf16, postop, out_f32):
    """Every epilogue on the 128 x 256 tile (ragged rows, a 16-column last tile), fp16 upcvt and
    s8 x s2."""
    M, K, N = HALF_RAGGED[0], 256, HALF_RAGGED[2]
    bad, dmax = _upcvt_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop)
    assert bad == 0, f"upcvt: {bad} bad (max |d| {dmax})"
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop)
    assert bad == 0, f"int8: {bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", HALF_SHAPES + [(1024, 17408, 5120)])
def test_int8_half_tile_shapes(dev, orc, M, K, N, bf16):
    """The s8 x s2 GEMM's 128 x 256 tile against the oracle (row sample, every column); with the
    split-K workspace the call takes the same tile (the same bits), at any count of these tiles."""
    import torch
    import ternocl_amd as T
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"
    A, B, SB, other, bias_f = _inputs(50000 + M + K + N, M, K, N, bf16)
    dA = dev_dt(A, bf16)
    dSA = torch.zeros((K // 128, T.ldsa(M)), dtype=dA.dtype, device="cuda")
    dAq = torch.zeros((M, K), dtype=torch.int8, device="cuda")
    T.quant_a(dA, dSA, dAq, M, K)
    dB, dSB = dev_raw(B), dev_dt(SB, bf16)
    outs = []
    for use_ws in (False, True):
        dO, dBias, dC = _device_io(torch, SB, other, bias_f, M, N, bf16, False)
        need = T.int2_int8_gemm_ws_bytes(M, N, K)
        ws = torch.zeros(need, dtype=torch.uint8, device="cuda") if use_ws and need else None
        T.int2_int8_gemm(None, dAq, dSA, dB, dSB, dC, dO, dBias, M, N, K, 0, False, ws=ws)
        torch.cuda.synchronize()
        outs.append(dC)
    assert torch.equal(outs[0], outs[1]), "the call with a workspace took another path"


@pytest.mark.parametrize("M", [1, 2, 4, 8])
@pytest.mark.parametrize("K,N", [(4096, 14336), (14336, 4096)])
def test_decode_workload_sweep(dev, orc, M, K, N):
    """The decode workload: bf16, bias + residual (postop 5), automatic engine."""
    bad, dmax = _upcvt_case(dev, orc, M, K, N, True, postop=5)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# Split-K (a workspace of ternocl_int2_gemm_ws_bytes): shapes whose 128 x 512
# tiles would leave CUs idle, including a ragged one (last row tile 104 rows,
# last column tile 16 columns).
SPLITK_SHAPES = [(1024, 14336, 4096), (1024, 17408, 5120), (200, 5120, 16384), (1000, 8192, 4112)]
# (the fp16 GEMM without the workspace runs 128 x 256 tiles at the second and
# the last, fewer than 192 of them, so the split stays with the workspace; the
# s8 x s2 GEMM runs those tiles there with or without it, and splits at the
# others and at a ragged shape of 128 x 128 tiles: last row tile 104 rows,
# last 128 x 512 column tile 416 columns)
FP16_SPLITK_SHAPES = SPLITK_SHAPES
INT8_SPLITK_SHAPES = [(1024, 14336, 4096), (200, 5120, 16384), (1000, 8192, 4000)]


def _splitk_case(dev, orc, M, K, N, bf16, postop=0, out_f32=False, seed=0):
    import torch
    import ternocl_amd as T
    need = T.int2_gemm_ws_bytes(M, N, K)
    assert need > 0, "this shape should split"
    print(f"split-K M={M} K={K} N={N} bf16={bf16} postop={postop} f32={out_f32} ws={need}", flush=True)
    A, B, S, other, bias_f = _inputs(seed + 60000 + M + K + N, M, K, N, bf16)
    dA, dB, dS = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16)
    dO, dBias, dC = _device_io(torch, S, other, bias_f, M, N, bf16, out_f32)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, postop, out_f32, ws=ws)
    torch.cuda.synchronize()
    first = dC.clone()
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, postop, out_f32, ws=ws)
    torch.cuda.synchronize()
    assert torch.equal(first, dC), "split-K results differ between runs"
    # the same call without the workspace (no split) agrees within the rule
    _, _, dC2 = _device_io(torch, S, other, bias_f, M, N, bf16, out_f32)
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC2, dO, dBias, M, N, K, postop, out_f32)
    torch.cuda.synchronize()
    if out_f32:
        a, b = host_f32(dC), host_f32(dC2)
    else:
        a, b = formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(host_u16(dC2), bf16)
    bad_nows, _ = allclose_report(a, b)
    rows = sample_rows(M)
    acc = orc.int2_gold(np.ascontiguousarray(A[rows]), B, S, rows.size, K, N, bf16)
    bad, dmax = _compare(orc, dC, acc, other, bias_f, rows, bf16, postop, out_f32)
    return bad, dmax, bad_nows


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", FP16_SPLITK_SHAPES)
def test_splitk_parity(dev, orc, M, K, N, bf16):
    bad, dmax, bad_nows = _splitk_case(dev, orc, M, K, N, bf16)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"
    assert bad_nows == 0, f"{bad_nows} elements differ from the unsplit GEMM beyond the rule"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", INT8_SPLITK_SHAPES)
def test_int8_splitk_parity(dev, orc, M, K, N, bf16):
    """The s8 x s2 GEMM's K split (ternocl_int2_int8_gemm_ws) on the same shapes."""
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16, split=True)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_int8_splitk_epilogues(dev, orc, bf16, postop, out_f32):
    M, K, N = INT8_SPLITK_SHAPES[-1]
    bad, dmax = _int8_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop, split=True)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
def test_splitk_epilogues(dev, orc, bf16, postop, out_f32):
    M, K, N = FP16_SPLITK_SHAPES[-1]
    bad, dmax, bad_nows = _splitk_case(dev, orc, M, K, N, bf16, postop, out_f32, seed=postop)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    assert bad_nows == 0


# ---- BITCOS: bitcos_fp16_upcvt/validate.sh:8-15 ----------------------------------
# (M, K, N, ls, z, postop, out_f32); ls 0 = the library's choice (the lines that give none)
BITCOS_VALIDATE_GEMV = [(1, 4096, 4096, 4, 0.4, 0, False), (1, 4096, 4096, 1, 0.4, 0, False),
                        (1, 4096, 6144, 8, 0.4, 0, False), (1, 12288, 4096, 8, 0.6, 0, False),
                        (1, 17408, 5120, 4, 0.3, 0, False), (1, 16384, 32768, 1, 0.4, 0, False),
                        (3, 4096, 2048, 2, 0.4, 0, False), (8, 1024, 512, 4, 0.1, 0, False),
                        (1, 4096, 1024, 16, 0.95, 0, False), (1, 4096, 4096, 0, 0.4, 1, False),
                        (1, 4096, 4096, 0, 0.4, 3, True)]
# (M, K, N, z, postop, out_f32): the --mt-m lines
BITCOS_VALIDATE_MT = [(64, 4096, 4096, 0.4, 0, False), (77, 4096, 2064, 0.05, 0, False),
                      (129, 17408, 5120, 0.4, 0, False), (512, 5120, 14336, 0.4, 0, False),
                      (9, 6144, 1024, 0.95, 0, False), (77, 4096, 2048, 0.4, 1, False),
                      (77, 4096, 2048, 0.4, 3, True)]
# and two lines of 128 x 256 tiles (ragged rows and a 16-column last tile; one row tile of 77)
BITCOS_HALF_MT = [(1000, 512, 6160, 0.4, 5, False), (77, 512, 40960, 0.3, 3, True)]


def _bitcos_inputs(seed, M, K, N, z, bf16):
    g = synth.rng(seed)
    A = synth.activations(g, (M, K), bf16)
    buf, _ = synth.bitcos_weights(g, K, N, z)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = g.standard_normal(N).astype(np.float32) * np.float32(0.1)
    return A, buf, S, other, bias_f


def _bitcos_device(torch, T, A, buf, S, other, bias_f, M, K, N, ls, bf16, out_f32):
    dB = dev_raw(buf)
    dSR = torch.zeros(max(ls - 1, 1) * N, dtype=torch.int32, device="cuda")
    T.bitcos_slice_ranks(dB, dSR, K, N, ls)
    dO, dBias, dC = _device_io(torch, S, other, bias_f, M, N, bf16, out_f32)
    return dev_dt(A, bf16), dB, dev_dt(S, bf16), dSR if ls > 1 else None, dO, dBias, dC


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ls,z,postop,out_f32", BITCOS_VALIDATE_GEMV)
def test_bitcos_validate_gemv(dev, orc, M, K, N, ls, z, postop, out_f32, bf16):
    """Each GEMV line, unsplit and (where the shape splits) through the split-launch
    workspace; both within the rule of the host gold, the split one bit-identical on a
    second call with its counters back at zero."""
    import torch
    import ternocl_amd as T
    ls = ls or T.bitcos_pick_ls(M, N, K)
    wsb = T.bitcos_gemv_ws_bytes(N, ls)
    print(f"bitcos validate gemv M={M} K={K} N={N} ls={ls} z={z} postop={postop} f32={out_f32} bf16={bf16} "
          f"ws={wsb}", flush=True)
    A, buf, S, other, bias_f = _bitcos_inputs(70000 + M + K + N + ls, M, K, N, z, bf16)
    dA, dB, dS, dSR, dO, dBias, dC = _bitcos_device(torch, T, A, buf, S, other, bias_f, M, K, N, ls, bf16, out_f32)
    T.bitcos_fp16_upcvt_gemm(dA, dB, dS, dSR, dC, dO, dBias, M, N, K, ls, postop, out_f32)
    torch.cuda.synchronize()
    acc = orc.bitcos_gold(A, buf, S, M, K, N, bf16)
    rows = np.arange(M)
    bad, dmax = _compare(orc, dC, acc, other, bias_f, rows, bf16, postop, out_f32)
    assert bad == 0, f"unsplit: {bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"
    if wsb:
        ws = torch.zeros(wsb, dtype=torch.uint8, device="cuda")
        _, _, dC2 = _device_io(torch, S, other, bias_f, M, N, bf16, out_f32)
        T.bitcos_fp16_upcvt_gemm(dA, dB, dS, dSR, dC2, dO, dBias, M, N, K, ls, postop, out_f32, ws=ws)
        torch.cuda.synchronize()
        first = dC2.clone()
        T.bitcos_fp16_upcvt_gemm(dA, dB, dS, dSR, dC2, dO, dBias, M, N, K, ls, postop, out_f32, ws=ws)
        torch.cuda.synchronize()
        assert torch.equal(first, dC2), "split launch not deterministic"
        assert not ws[:T.WS_HEADER_BYTES].any().item(), "split launch left a counter set"
        bad, dmax = _compare(orc, dC2, acc, other, bias_f, rows, bf16, postop, out_f32)
        assert bad == 0, f"split: {bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("in_tile", [False, True])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,z,postop,out_f32", BITCOS_VALIDATE_MT + BITCOS_HALF_MT)
def test_bitcos_validate_mt(dev, orc, M, K, N, z, postop, out_f32, bf16, in_tile):
    """Each M-tiled line through ternocl_bitcos_fp16_upcvt_gemm_mt: with the re-pack workspace
    and without (the reference's call: the tiles decode BITCOS), row-sampled above 127 rows."""
    import torch
    import ternocl_amd as T
    ls = T.bitcos_pick_ls(1, N, K)
    print(f"bitcos validate mt M={M} K={K} N={N} ls={ls} z={z} postop={postop} f32={out_f32} bf16={bf16} "
          f"in_tile={in_tile}", flush=True)
    A, buf, S, other, bias_f = _bitcos_inputs(71000 + M + K + N, M, K, N, z, bf16)
    dA, dB, dS, dSR, dO, dBias, dC = _bitcos_device(torch, T, A, buf, S, other, bias_f, M, K, N, ls, bf16, out_f32)
    ws = None if in_tile else torch.empty(T.bitcos_gemm_mt_ws_bytes(K, N), dtype=torch.uint8, device="cuda")
    T.bitcos_fp16_upcvt_gemm_mt(dA, dB, dS, dSR, dC, dO, dBias, M, N, K, ls, ws, postop, out_f32)
    torch.cuda.synchronize()
    rows = sample_rows(M)
    acc = orc.bitcos_gold(np.ascontiguousarray(A[rows]), buf, S, rows.size, K, N, bf16)
    bad, dmax = _compare(orc, dC, acc, other, bias_f, rows, bf16, postop, out_f32)
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"
