"""GPU parity of the int2 upcvt path (decode GEMV, M <= 8) through the C ABI.

Reference test design followed: int2_fp16_upcvt/validate.sh:8-10 (shape list,
fp16 + bf16, distinct sets), validate_epilogues.sh:19-36 (POSTOP 0..4 x DT/fp32
output x shapes), int2_fp16_upcvt/main.cpp:351-353 (every rotating set must
reproduce set 0 bit for bit).  Golds: the oracle's restatement of
compute_gold + epilogue_ref (int2_fp16_upcvt/main.cpp:79-98,
common/epilogue.hpp:98-115).
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_dt, dev_raw, host_f32, host_u16, host_u32, xetla_cmp
from tests.gpu_util import int2_gold as _gold, int2_inputs as _inputs, int2_run as _run

pytestmark = pytest.mark.gpu


SHAPES = [(1, 4096, 4096), (1, 4096, 14336), (1, 14336, 4096), (2, 4096, 14336), (4, 14336, 4096),
          (8, 4096, 14336), (3, 256, 48), (1, 128, 16), (5, 1024, 272), (7, 384, 2064), (1, 17408, 5120),
          (16, 4096, 4096), (13, 1024, 272), (11, 640, 48)]


F4_MAX_M = {False: 8, True: 8}  # the fp8 x fp4 engine: two 16-row MFMA row sets of 4 rows each


@pytest.mark.parametrize("engine", [1, 2, 4])
@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemv_parity(dev, orc, M, K, N, bf16, engine):
    import torch
    import ternocl_amd as T
    if engine == 1 and M > 8:
        pytest.skip("the VALU GEMV takes M <= 8")
    if engine == 4 and M > F4_MAX_M[bf16]:
        pytest.skip("the fp8 x fp4 GEMV takes M <= 8")
    print(f"gemv parity M={M} K={K} N={N} bf16={bf16} engine={engine}", flush=True)
    A, B, S, other, bias_f = _inputs(1000 + M + K + N, M, K, N, bf16)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False, tile=T.gemv_tile(engine))
    want, acc = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    got = formats.dt_to_f32(host_u16(dC), bf16)
    bad, dmax = allclose_report(got, formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} elements outside 1e-3 + 1e-2*|ref| (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4, 5])
@pytest.mark.parametrize("out_f32", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 5120, 4096), (3, 4096, 2048)])
def test_gemv_epilogues(dev, orc, M, K, N, bf16, postop, out_f32):
    import torch
    import ternocl_amd as T
    print(f"gemv epilogue M={M} K={K} N={N} bf16={bf16} postop={postop} f32={out_f32}", flush=True)
    A, B, S, other, bias_f = _inputs(7 + postop, M, K, N, bf16)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    if out_f32:
        got, ref = host_f32(dC), want
    else:
        got, ref = formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16)
    bad, dmax = allclose_report(got, ref)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_reference_distribution_rule(dev, orc, bf16):
    """The reference driver's own inputs and pass rule (xetla_buff_cmp)."""
    import torch
    import ternocl_amd as T
    M, K, N = 1, 5120, 4096
    A, B, S, other, bias_f = _inputs(99, M, K, N, bf16, ref_dist=True)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    assert xetla_cmp(host_u16(dC), want, bf16) == 0


TILES = [(1, 1, 0, 0, 4), (1, 3, 0, 0, 4), (1, 4, 0, 0, 4), (1, 1, 0, 0, 8), (1, 5, 0, 0, 8),
         (1, 8, 0, 0, 8), (1, 2, 0, 0, 16), (1, 8, 0, 0, 16), (1, 0, 0, 0, 0),
         (2, 1, 1, 1, 0), (2, 8, 1, 1, 0), (2, 4, 2, 1, 0), (2, 8, 2, 2, 0), (2, 2, 1, 4, 0),
         (2, 8, 2, 4, 0), (2, 3, 2, 2, 0), (2, 0, 0, 0, 0), (0, 0, 0, 0, 0),
         (4, 0, 0, 0, 0), (4, 1, 1, 1, 0), (4, 8, 1, 1, 0), (4, 4, 2, 1, 0), (4, 8, 2, 2, 0),
         (4, 2, 1, 4, 0), (4, 8, 2, 4, 0), (4, 3, 2, 2, 0), (4, 8, 4, 2, 0), (4, 5, 1, 8, 0),
         (4, 14, 1, 2, 0), (4, 16, 1, 1, 0)]


@pytest.mark.parametrize("tile", TILES)
def test_gemv_tiles_deterministic(dev, orc, tile):
    """Every tile (engine, waves, cols/lane, groups/wave, col_lanes) gives the
    gold, and repeated calls are bit-identical (the K reduction has a fixed order)."""
    import torch
    import ternocl_amd as T
    M, K, N, bf16 = 2, 3840, 1024, False
    A, B, S, other, bias_f = _inputs(5, M, K, N, bf16)
    outs = []
    for _ in range(3):
        dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False, tile=T.gemv_tile(*tile))
        outs.append(host_u16(dC))
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    bad, dmax = allclose_report(formats.dt_to_f32(outs[0], bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"tile {tile}: {bad} bad (max |d| {dmax})"
    assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"


def test_gemv_plan_too_big_for_lds_is_rejected(dev):
    import torch
    import ternocl_amd as T
    M, K, N = 2, 3840, 1024
    A = torch.zeros((M, K), dtype=torch.float16, device="cuda")
    B = torch.zeros((K // 16, N), dtype=torch.int32, device="cuda")
    S = torch.zeros((K // 128, N), dtype=torch.float16, device="cuda")
    C = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A, B, S, C, None, None, M, N, K, tile=T.gemv_tile(1, 16, 0, 0, 4))
    assert e.value.status == 1
    with pytest.raises(T.TernoclError):  # M > 8 on the VALU engine
        T.int2_fp16_upcvt_gemm(A.repeat(5, 1), B, S, C.repeat(5, 1), None, None, 10, N, K,
                               tile=T.gemv_tile(1))


@pytest.mark.parametrize("M,tile", [(1, (1, 2, 0, 0, 16)), (8, (1, 2, 0, 0, 16)), (8, (2, 0, 0, 0, 0)),
                                    (16, (2, 0, 0, 0, 0)), (3, (2, 2, 1, 1, 0)), (1, (4, 2, 1, 16, 0)),
                                    (4, (4, 0, 0, 0, 0)), (3, (4, 2, 2, 1, 0)), (1, (4, 8, 2, 4, 0)),
                                    (1, (4, 14, 1, 4, 0)), (1, (4, 0, 0, 0, 0))])
def test_gemv_multi_window(dev, orc, M, tile):
    """K long enough for several LDS rounds / windows (double-buffered staging)."""
    import torch
    import ternocl_amd as T
    K, N, bf16 = 40960, 64, True
    A, B, S, other, bias_f = _inputs(11, M, K, N, bf16)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, False, tile=T.gemv_tile(*tile))
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, False)
    bad, _ = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0


@pytest.mark.parametrize("bf16", [False, True])
def test_int2_dequant_bit_exact(dev, orc, bf16):
    """The reference B-operand unpack (dq_word): +0 / +s / s^0x8000, bit for bit."""
    import torch
    import ternocl_amd as T
    K, N = 512, 272
    g = synth.rng(3)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    dW = torch.empty((K, N), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    T.int2_dequant(dev_raw(B), dev_dt(S, bf16), dW, K, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(dW), orc.int2_dequant(B, S, K, N))


@pytest.mark.parametrize("engine", [1, 2])
@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_decode_bit_exact(dev, bf16, engine):
    """Each GEMV's own in-register unpack, bit for bit against its closed form:
    dword = DT(BASE + (v+2) * 2^p) for two rows of the word (low / high half),
    and every half decodes back to the signed weight."""
    import torch
    import ternocl_amd as T
    K, N = 256, 64
    g = synth.rng(4)
    B = synth.int2_weights(g, K, N)
    B[0, :16] = np.arange(16, dtype=np.uint32) * 0x11111111  # every code in every field
    D = torch.empty(((K // 16) * N * 8,), dtype=torch.int32, device="cuda")
    T.int2_gemv_decode(dev_raw(B), D, K, N, bf16, engine=engine)
    torch.cuda.synchronize()
    got = host_u32(D).reshape(K // 16, N, 8)
    codes = (B[..., None] >> (2 * np.arange(16, dtype=np.uint32))) & 3  # [K/16, N, 16]
    x = (codes ^ 2).astype(np.uint32)
    if engine == 1:  # pair j = rows (j, j+8)
        rows = list(range(8))
        shifts = [0, 2, 4, 0, 2, 4, 0, 2] if bf16 else [0, 2, 4, 6, 8, 2, 4, 6]
    else:  # dword 4h+i = rows (4h+i, 4h+i+8)
        rows = list(range(8))
        shifts = ([0, 2, 4, 5] if bf16 else [0, 2, 4, 6]) * 2
    base = 0x4300 if bf16 else 0x6400
    for d, (j, p) in enumerate(zip(rows, shifts)):
        want = (base | (x[..., j] << p)) | ((base | (x[..., j + 8] << p)) << 16)
        assert np.array_equal(got[..., d], want.astype(np.uint32)), f"dword {d}"
    sv = formats.unpack_int2(B, K).reshape(K // 16, 16, N).transpose(0, 2, 1)
    for d, (j, p) in enumerate(zip(rows, shifts)):
        for half, row in ((0, j), (1, j + 8)):
            vals = formats.dt_to_f32(((got[..., d] >> (16 * half)) & 0xFFFF).astype(np.uint16), bf16)
            v = (vals - (128.0 if bf16 else 1024.0)) / 2.0 ** p - 2
            assert np.array_equal(v.astype(np.int8), sv[..., row])


@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_f4_decode_bit_exact(dev, bf16):
    """The fp8 x fp4 engine's weight decode: per word two fp4 dwords, nibble n
    of dword h = row 2n + h, nibble = (b1 << 3) | (b0 << 2) of the code (e2m1
    +0, +2, -2, -0 for codes 0, 1, 3, 2), i.e. exactly 2v."""
    import torch
    import ternocl_amd as T
    K, N = 256, 64
    g = synth.rng(14)
    B = synth.int2_weights(g, K, N)
    B[0, :16] = np.arange(16, dtype=np.uint32) * 0x11111111  # every code in every field
    D = torch.empty(((K // 16) * N * 2,), dtype=torch.int32, device="cuda")
    T.int2_gemv_decode(dev_raw(B), D, K, N, bf16, engine=T.F4)
    torch.cuda.synchronize()
    got = host_u32(D).reshape(K // 16, N, 2)
    codes = (B[..., None] >> (2 * np.arange(16, dtype=np.uint32))) & 3
    nib = ((codes >> 1) << 3) | ((codes & 1) << 2)
    e2m1 = np.array([0, 0.5, 1, 1.5, 2, 3, 4, 6, -0.0, -0.5, -1, -1.5, -2, -3, -4, -6])
    sv = formats.unpack_int2(B, K).reshape(K // 16, 16, N).transpose(0, 2, 1)
    for h in range(2):
        want = np.zeros(got.shape[:2], np.uint64)
        for n in range(8):
            want |= nib[..., 2 * n + h].astype(np.uint64) << np.uint64(4 * n)
            vals = e2m1[(got[..., h] >> (4 * n)) & 15]
            valid = codes[..., 2 * n + h] != 2
            assert np.array_equal((vals / 2)[valid], sv[..., 2 * n + h][valid].astype(np.float64))
        assert np.array_equal(got[..., h], want.astype(np.uint32)), f"dword {h}"


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 14336), (1, 14336, 4096), (3, 1024, 512)])
def test_gemv_stream_probe_checksum(dev, M, K, N, bf16):
    """The decode-removed measurement kernel streams every word and scale it
    should: row m < M of its output is half the sum over groups g of
    float(B[8g + 2m, n] ^ B[8g + 2m + 1, n]) * S[g, n] (the words lane q = m of
    the GEMV takes), to fp32 rounding."""
    import torch
    import ternocl_amd as T
    g = synth.rng(71 + M)
    B = g.integers(0, 2**32, size=(K // 16, N), dtype=np.uint32)
    S = synth.scales(g, K, N, bf16)
    C = torch.zeros((M, N), dtype=torch.float32, device="cuda")
    T.int2_gemv_stream_probe(dev_raw(B), dev_dt(S, bf16), C, M, N, K)
    torch.cuda.synchronize()
    s = formats.dt_to_f32(S, bf16).astype(np.float64)
    for m in range(M):
        x = (B[2 * m::8] ^ B[2 * m + 1::8]).astype(np.float32).astype(np.float64)
        want = 0.5 * (x * s).sum(axis=0)
        np.testing.assert_allclose(C[m].cpu().numpy(), want, rtol=1e-5)


KSPLIT = [(8, 14336, 4096, 8, 4), (5, 4096, 14336, 2, 4), (1, 14336, 4096, 4, 2), (3, 5120, 272, 3, 1),
          (7, 384, 2064, 4, 1), (2, 256, 48, 4, 1), (4, 40960, 64, 16, 4), (8, 1024, 1024, 5, 2)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ks,cpl", KSPLIT)
def test_gemv_f4_k_slices(dev, orc, M, K, N, ks, cpl, bf16):
    """K split over ks workgroups per strip (slices of at most one per group;
    K = 256 with ks = 4 runs 2): the gold within 1e-3 + 1e-2 |ref| with and
    without the epilogue operands, bit-identical over repeated calls (the last
    workgroup adds the slices in order), the strip counters back at zero."""
    import torch
    import ternocl_amd as T
    print(f"gemv f4 k-slices M={M} K={K} N={N} ks={ks} cpl={cpl} bf16={bf16}", flush=True)
    A, B, S, other, bias_f = _inputs(55 + M + ks, M, K, N, bf16)
    tile = T.gemv_tile(T.F4, 0, cpl, 0, 0, ks)
    dA, dB, dS, dO = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16), dev_dt(other, bf16)
    dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
    cnt_bytes = (N // 16) * 4  # the strip counters, at the front of the workspace header
    ws = torch.zeros(T.WS_HEADER_BYTES + ks * M * N * 4, dtype=torch.uint8, device="cuda")
    for postop in (0, 5):
        outs = []
        for _ in range(3):
            dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
            T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, postop, False, ws=ws, tile=tile)
            torch.cuda.synchronize()
            outs.append(host_u16(dC))
        assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"
        assert not ws[:cnt_bytes].any().item(), "strip counters not left at zero"
        want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, False)
        bad, dmax = allclose_report(formats.dt_to_f32(outs[0], bf16), formats.dt_to_f32(want, bf16))
        assert bad == 0, f"postop {postop}: {bad} bad (max |d| {dmax})"


# (M, K, N, slices of the automatic plan): K whose power-of-two split gives slices
# that do not divide into waves of whole groups (K = 17408: 136 groups, 4 slices
# of 34 = 2 x 17) take the slice count whose plan has the fewest windows
AUTO_UNEVEN = [(1, 17408, 5120, 5), (2, 13312, 1024, 9), (3, 23552, 256, 12), (1, 34816, 256, 10)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ks", AUTO_UNEVEN)
def test_gemv_f4_auto_split_uneven_slices(dev, orc, M, K, N, ks, bf16):
    """The automatic K split on slice counts chosen for whole waves of groups: the
    workspace the entry asks for holds that many slices, the result is within the
    rule of the gold, bit-identical over repeated calls, and the counters are left
    at zero."""
    import torch
    import ternocl_amd as T
    print(f"gemv f4 auto split M={M} K={K} N={N} ks={ks} bf16={bf16}", flush=True)
    need = T.int2_gemm_ws_bytes(M, N, K)
    assert need == T.WS_HEADER_BYTES + ks * M * N * 4
    A, B, S, other, bias_f = _inputs(77 + M + K // 1024, M, K, N, bf16)
    dA, dB, dS, dO = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16), dev_dt(other, bf16)
    dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
    ws = torch.zeros(need, dtype=torch.uint8, device="cuda")
    outs = []
    for _ in range(3):
        dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
        T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, 5, False, ws=ws)
        torch.cuda.synchronize()
        outs.append(host_u16(dC))
    assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"
    assert not ws[:(N // 16) * 4].any().item(), "strip counters not left at zero"
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 5, False)
    bad, dmax = allclose_report(formats.dt_to_f32(outs[0], bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_gemv_f4_k_slices_need_the_workspace(dev):
    """An explicit split without a large enough workspace is an error; the
    automatic plan without one runs unsplit."""
    import torch
    import ternocl_amd as T
    M, K, N = 8, 14336, 4096
    need = T.int2_gemm_ws_bytes(M, N, K)
    assert need == T.WS_HEADER_BYTES + 4 * M * N * 4  # 4 slices of fp32 [M, N] after the counters' header
    dA = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    dB = torch.zeros((K // 16, N), dtype=torch.int32, device="cuda")
    dS = torch.zeros((K // 128, N), dtype=torch.bfloat16, device="cuda")
    dC = torch.ones((M, N), dtype=torch.bfloat16, device="cuda")
    short = torch.zeros(need - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, None, None, M, N, K, ws=short, tile=T.gemv_tile(T.F4, 0, 4, 0, 0, 8))
    assert e.value.status == 3
    with pytest.raises(T.TernoclError):  # k_slices on another engine
        T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, None, None, M, N, K, tile=T.gemv_tile(T.MFMA, 0, 0, 0, 0, 2))
    T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, None, None, M, N, K, ws=short)
    torch.cuda.synchronize()
    assert not dC.any().item()


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 4096, 1024), (2, 1024, 272), (4, 2048, 512), (6, 1024, 272), (8, 2048, 512)])
def test_gemv_f4_pieces_exact(dev, orc, M, K, N, bf16):
    """The fp8 pieces sum to each activation exactly, so the fp32 result agrees
    with the fp32 host gold to accumulation-order rounding (far inside the
    1e-2 rule: a dropped piece would show as ~3% errors)."""
    import torch
    import ternocl_amd as T
    if M > F4_MAX_M[bf16]:
        pytest.skip("M too large for the engine")
    A, B, S, other, bias_f = _inputs(31 + M, M, K, N, bf16)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, True, tile=T.gemv_tile(T.F4))
    _, acc = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, True)
    got = host_f32(dC).astype(np.float64)
    # |error| against the sum of |terms| the accumulation rounds over
    l1 = np.abs(formats.dt_to_f32(A, bf16)).astype(np.float64) @ (
        np.abs(formats.unpack_int2(B, K)).astype(np.float64) *
        np.repeat(formats.dt_to_f32(S, bf16).astype(np.float64), 128, axis=0))
    err = np.abs(got - acc.astype(np.float64))
    assert (err <= 4e-6 * l1 + 1e-7).all(), f"max err/l1 {float((err / (l1 + 1e-30)).max()):.3g}"


@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_f4_outlier_channels(dev, orc, bf16):
    """LLM-like activations: N(0,1) with outlier channels 300x larger.  The
    flush rule keeps every piece row of a block inside the MFMA's exact adding
    window, so the result stays at fp32-accumulation accuracy (the oracle is
    itself within ~1e-5 of the exact sum here)."""
    import torch
    import ternocl_amd as T
    M, K, N = 1, 4096, 512
    g = synth.rng(77)
    a = g.standard_normal((M, K)).astype(np.float32)
    a[0, 5::61] *= 300.0
    A = formats.f32_to_dt(a, bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = np.zeros(N, np.float32)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, True, tile=T.gemv_tile(T.F4))
    _, acc = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, True)
    d = np.abs(host_f32(dC).astype(np.float64) - acc)
    assert d.max() < 1e-4, f"max |d| {d.max():.3g}"


@pytest.mark.parametrize("bf16", [False, True])
def test_gemv_f4_wide_dynamic_range(dev, orc, bf16):
    """Activations spanning many binades inside one 32-block (outliers, tiny
    values, zeros of both signs, fp16 subnormals): the per-piece block scales
    still give the gold within the parity rule (1e-3 + 1e-2 |ref|)."""
    import torch
    import ternocl_amd as T
    M, K, N = 1, 4096, 512
    g = synth.rng(77)
    a = g.standard_normal((M, K)).astype(np.float32)
    a *= np.exp2(g.integers(-14, 9 if bf16 else 5, (M, K))).astype(np.float32)  # 2^-14 .. 2^8 (fp16 2^4)
    a[0, ::97] = 0.0
    a[0, 1::97] = -0.0
    a[0, 5::61] *= 3000.0 if bf16 else 100.0                        # outliers
    if not bf16:
        a[0, 7::53] = 3e-6                                            # fp16 subnormals
    A = formats.f32_to_dt(a, bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    other = synth.activations(g, (M, N), bf16)
    bias_f = np.zeros(N, np.float32)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 0, True, tile=T.gemv_tile(T.F4))
    _, acc = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 0, True)
    bad, dmax = allclose_report(host_f32(dC), acc)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# ---- the multi-strip GEMV (engine 5, M <= 4) ---------------------------------------
# (K, N): one window of waves x groups per wave covering K (1, 2 and 4 groups per
# wave, up to 16 waves), fewer strips than workgroups, many strips per workgroup,
# the two reference LM heads (int2_fp16_upcvt/bench.sh:12) and a 129-strip N
MULTISTRIP = [(128, 16), (256, 48), (1024, 2064), (2048, 40960), (4096, 14336), (5120, 34816),
              (8192, 4096), (4096, 151680), (5120, 248320)]


def _ms_plan(K):
    groups = K // 128
    gpw = 4 if groups >= 32 else 2 if groups >= 16 else 1
    return gpw, (groups + gpw - 1) // gpw


MULTISTRIP_M = [(M, K, N) for K, N in MULTISTRIP for M in (1, 2, 3, 4, 5, 8)
                if M == 1 or (N <= 40960 and (M <= 4 or K <= 4096))]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", MULTISTRIP_M)
def test_gemv_multistrip_parity(dev, orc, M, K, N, bf16):
    """Engine 5 gives engine 4's bits when engine 4 runs the same waves and groups per
    wave on 16-column strips (the same per-column arithmetic in the same order; engine 4
    takes at most 8 waves above one row, and at most 2 groups per wave at 8 rows, so those
    shapes are checked against the gold only), with and without the bias + residual
    epilogue, and every output within 1e-3 + 1e-2 |ref| of the host gold; rows M = 1..8
    (3, 5: the 4- and 8-row kernels with their last rows not stored)."""
    import ternocl_amd as T
    gpw, waves = _ms_plan(K)
    print(f"gemv multi-strip M={M} K={K} N={N} bf16={bf16} (waves {waves} x {gpw} groups)", flush=True)
    A, B, S, other, bias_f = _inputs(77 + K + N + M, M, K, N, bf16)
    for postop, cpl in ((0, 0), (5, 1), (5, 2), (5, 4)):
        if N % (16 * max(cpl, 1)) or (cpl == 4 and M > 1):
            continue
        ms, _ = _run(T, __import__("torch"), A, B, S, other, bias_f, M, K, N, bf16, postop, False,
                     tile=T.gemv_tile(T.F4MS, 0, cpl))
        if M == 1 or (waves <= 8 and M <= 4):
            f4, _ = _run(T, __import__("torch"), A, B, S, other, bias_f, M, K, N, bf16, postop, False,
                         tile=T.gemv_tile(T.F4, waves, 1, gpw, 0, 1))
            assert np.array_equal(host_u16(ms), host_u16(f4)), f"postop {postop}: engine 5 differs from engine 4"
        want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, False)
        bad, dmax = allclose_report(formats.dt_to_f32(host_u16(ms), bf16), formats.dt_to_f32(want, bf16))
        assert bad == 0, f"postop {postop}: {bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("M,K,N", [(6, 1024, 65536), (8, 2048, 65536), (3, 4096, 5120), (5, 4096, 6144),
                                   (1, 8192, 4224), (4, 2048, 4128)])
def test_gemv_multistrip_automatic_rows(dev, orc, M, K, N):
    """The automatic plan at 1..8 rows where it takes the multi-strip kernel (past 128
    strips of 32 columns; K <= 4096 above 4 rows): the same bits as the explicit engine and
    the gold within the rule, with the bias + residual epilogue."""
    import torch
    import ternocl_amd as T
    bf16 = True
    print(f"gemv multi-strip automatic M={M} K={K} N={N}", flush=True)
    A, B, S, other, bias_f = _inputs(313 + M, M, K, N, bf16)
    auto, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 5, False)
    ms, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, 5, False, tile=T.gemv_tile(T.F4MS))
    assert np.array_equal(host_u16(auto), host_u16(ms))
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, 5, False)
    bad, dmax = allclose_report(formats.dt_to_f32(host_u16(auto), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("postop,out_f32", [(1, False), (2, True), (3, True), (4, False)])
def test_gemv_multistrip_epilogues(dev, orc, postop, out_f32):
    import torch
    import ternocl_amd as T
    M, K, N, bf16 = 1, 4096, 40960, True
    A, B, S, other, bias_f = _inputs(91 + postop, M, K, N, bf16)
    dC, _ = _run(T, torch, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32, tile=T.gemv_tile(T.F4MS))
    want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, out_f32)
    if out_f32:
        bad, dmax = allclose_report(host_f32(dC), want)
    else:
        bad, dmax = allclose_report(formats.dt_to_f32(host_u16(dC), bf16), formats.dt_to_f32(want, bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


# (M, K, N, k_slices, groups per wave): one window per slice (K = 17408: 5 slices,
# the last of 24 groups), one strip per workgroup and many (N = 40960: 1280
# strips of 32 columns over 128 walkers per slice), 8 rows (two row sets)
MS_KSPLIT = [(1, 14336, 4096, 4, 2), (1, 14336, 4096, 2, 4), (3, 17408, 5120, 5, 4), (4, 8192, 4096, 4, 2),
             (8, 4096, 8192, 2, 2), (1, 16384, 40960, 4, 4), (2, 32768, 1024, 8, 4)]


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N,ks,gpw", MS_KSPLIT)
def test_gemv_multistrip_k_slices(dev, orc, M, K, N, ks, gpw, bf16):
    """Engine 5 over K slices (the workspace's slice sums and strip counters): engine 4's
    bits on the same slices, waves and groups per wave (the same per-column sums, added
    in slice order), bit-identical over repeated calls, the counters back at zero, and
    the gold within 1e-3 + 1e-2 |ref|, with and without the bias + residual epilogue."""
    import torch
    import ternocl_amd as T
    groups = K // 128
    gps = -(-groups // ks)
    waves = -(-gps // gpw)
    print(f"gemv multi-strip k-slices M={M} K={K} N={N} ks={ks} gpw={gpw} waves={waves} bf16={bf16}", flush=True)
    A, B, S, other, bias_f = _inputs(171 + M + ks + gpw, M, K, N, bf16)
    dA, dB, dS, dO = dev_dt(A, bf16), dev_raw(B), dev_dt(S, bf16), dev_dt(other, bf16)
    dBias = dev_dt(formats.f32_to_dt(bias_f, bf16), bf16)
    ws = torch.zeros(T.WS_HEADER_BYTES + ks * M * N * 4, dtype=torch.uint8, device="cuda")
    cnt_bytes = (N // 16) * 4
    for postop in (0, 5):
        outs = []
        for _ in range(3):
            dC = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
            T.int2_fp16_upcvt_gemm(dA, dB, dS, dC, dO, dBias, M, N, K, postop, False, ws=ws,
                                   tile=T.gemv_tile(T.F4MS, 0, 0, gpw, 0, ks))
            torch.cuda.synchronize()
            outs.append(host_u16(dC))
        assert all(np.array_equal(outs[0], o) for o in outs[1:]), "non-deterministic"
        assert not ws[:cnt_bytes].any().item(), "strip counters not left at zero"
        dC4 = torch.zeros((M, N), dtype=dA.dtype, device="cuda")
        T.int2_fp16_upcvt_gemm(dA, dB, dS, dC4, dO, dBias, M, N, K, postop, False, ws=ws,
                               tile=T.gemv_tile(T.F4, waves, 1, gpw, 0, ks))
        torch.cuda.synchronize()
        assert np.array_equal(outs[0], host_u16(dC4)), f"postop {postop}: engine 5 differs from engine 4"
        want, _ = _gold(orc, A, B, S, other, bias_f, M, K, N, bf16, postop, False)
        bad, dmax = allclose_report(formats.dt_to_f32(outs[0], bf16), formats.dt_to_f32(want, bf16))
        assert bad == 0, f"postop {postop}: {bad} bad (max |d| {dmax})"


def test_gemv_multistrip_automatic_and_rejects(dev):
    """The automatic plan takes engine 5 at M = 1 past 128 strips of 32 columns (the same
    bits as the explicit engine); engine 5 rejects M > 8, K > 4096 above 4 rows,
    cols_per_lane 4 above one row, K past one window (64 groups), an explicit wave
    count, and K slices without the workspace, at one column per lane or at one group
    per wave."""
    import torch
    import ternocl_amd as T
    K, N = 4096, 5120
    A = torch.randn((1, K), device="cuda").to(torch.bfloat16)
    B = torch.randint(-2**31, 2**31 - 1, (K // 16, N), dtype=torch.int32, device="cuda")
    S = (torch.rand((K // 128, N), device="cuda") * 0.01).to(torch.bfloat16)
    c0 = torch.zeros((1, N), dtype=torch.bfloat16, device="cuda")
    c1 = torch.ones((1, N), dtype=torch.bfloat16, device="cuda")
    T.int2_fp16_upcvt_gemm(A, B, S, c0, None, None, 1, N, K)
    T.int2_fp16_upcvt_gemm(A, B, S, c1, None, None, 1, N, K, tile=T.gemv_tile(T.F4MS))
    torch.cuda.synchronize()
    assert torch.equal(c0, c1)
    A9 = torch.zeros((9, K), dtype=torch.bfloat16, device="cuda")
    C9 = torch.zeros((9, N), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A9, B, S, C9, None, None, 9, N, K, tile=T.gemv_tile(T.F4MS))
    assert e.value.status == 2
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A9, B, S, C9, None, None, 2, N, K, tile=T.gemv_tile(T.F4MS, 0, 4))
    assert e.value.status == 2
    K6 = 5120
    A6 = torch.zeros((5, K6), dtype=torch.bfloat16, device="cuda")
    B6 = torch.zeros((K6 // 16, N), dtype=torch.int32, device="cuda")
    S6 = torch.zeros((K6 // 128, N), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A6, B6, S6, C9, None, None, 5, N, K6, tile=T.gemv_tile(T.F4MS))
    assert e.value.status == 2
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A, B, S, c0, None, None, 1, N, K, tile=T.gemv_tile(T.F4MS, 8))
    assert e.value.status == 1
    with pytest.raises(T.TernoclError) as e:  # K slices need the workspace
        T.int2_fp16_upcvt_gemm(A, B, S, c0, None, None, 1, N, K, tile=T.gemv_tile(T.F4MS, 0, 2, 2, 0, 2))
    assert e.value.status == 3
    ws = torch.zeros(T.WS_HEADER_BYTES + 2 * N * 4, dtype=torch.uint8, device="cuda")
    for cpl, gpw in ((1, 2), (2, 1)):
        with pytest.raises(T.TernoclError) as e:
            T.int2_fp16_upcvt_gemm(A, B, S, c0, None, None, 1, N, K, ws=ws,
                                   tile=T.gemv_tile(T.F4MS, 0, cpl, gpw, 0, 2))
        assert e.value.status == 2
    K2 = 8320
    A3 = torch.zeros((1, K2), dtype=torch.bfloat16, device="cuda")
    B3 = torch.zeros((K2 // 16, 64), dtype=torch.int32, device="cuda")
    S3 = torch.zeros((K2 // 128, 64), dtype=torch.bfloat16, device="cuda")
    C3 = torch.zeros((1, 64), dtype=torch.bfloat16, device="cuda")
    with pytest.raises(T.TernoclError) as e:
        T.int2_fp16_upcvt_gemm(A3, B3, S3, C3, None, None, 1, 64, K2, tile=T.gemv_tile(T.F4MS))
    assert e.value.status == 2
