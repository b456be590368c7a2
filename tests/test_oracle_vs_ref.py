"""Pin the C oracle against the reference's own host code, compiled from the
reference sources where they lie (oracle/ref_shim.cpp -> oracle/_ref).

Skipped where oracle/_ref was not built (no reference tree).  Everything here
must match bit for bit: both are fp32 loops in the same order.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth

pytestmark = pytest.mark.skipif(
    not __import__("oracle.binding", fromlist=["x"]).ref_available(),
    reason="oracle/_ref not built (reference tree absent)")


@pytest.mark.parametrize("bf16", [False, True])
def test_tof_exhaustive(orc, bf16):
    r = orc.ref()
    r.ref_set_bf16(int(bf16))
    h = np.arange(65536, dtype=np.uint16)
    mine = orc.tof(h, bf16)
    theirs = np.array([r.ref_tof(int(x)) for x in h], np.float32)
    # NaNs pass through a ctypes float return as doubles (payload quieted): compare as NaN
    same = (mine.view(np.uint32) == theirs.view(np.uint32)) | (np.isnan(mine) & np.isnan(theirs))
    assert same.all()


@pytest.mark.parametrize("bf16", [False, True])
def test_fromf_matches_reference(orc, bf16):
    r = orc.ref()
    r.ref_set_bf16(int(bf16))
    g = np.random.default_rng(7)
    u = g.integers(0, 2**32, 60000, dtype=np.uint64).astype(np.uint32)
    # plus every fp16/bf16 rounding boundary neighbourhood
    edges = np.array([0x477FEFFF, 0x477FF000, 0x477FF001, 0x33000000, 0x33000001, 0x387FFFFF,
                      0x38800000, 0x7F7FFFFF, 0x7F800000, 0xFF800000, 0x00000001, 0x80000000],
                     np.uint32)
    f = np.concatenate([u, edges]).view(np.float32)
    mine = orc.fromf(f, bf16)
    theirs = np.array([r.ref_fromf(float(x)) for x in f], np.uint16)
    finite = np.isfinite(f)  # NaN payloads do not survive the ctypes float round trip
    assert np.array_equal(mine[finite], theirs[finite])


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("M,K,N", [(1, 256, 48), (3, 512, 32), (5, 1024, 64)])
def test_int2_gold_bitwise(orc, M, K, N, bf16):
    g = synth.rng(M * 131 + K)
    A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16, 0.75, 15.75)
    assert np.array_equal(orc.int2_gold(A, B, S, M, K, N, bf16).view(np.uint32),
                          orc.ref_int2_gold(A, B, S, M, K, N, bf16).view(np.uint32))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop", [0, 1, 2, 3, 4])
@pytest.mark.parametrize("out_f32", [False, True])
def test_epilogue_bitwise(orc, postop, out_f32, bf16):
    g = synth.rng(postop)
    M, N = 4, 96
    acc = (g.standard_normal((M, N)) * 6).astype(np.float32)
    acc[0, :8] = [-10.0, -10.5, -9.99, 0.0, 80.0, -80.0, 1e-8, 3.0]
    other = formats.f32_to_dt(g.uniform(-4, 4, (M, N)).astype(np.float32), bf16)
    bias = (g.uniform(-8, 8, N).astype(np.float32) if out_f32
            else formats.f32_to_dt(g.uniform(-8, 8, N).astype(np.float32), bf16))
    mine = orc.epilogue(acc, other, bias, postop, out_f32, bf16)
    theirs = orc.ref_epilogue(acc, other, bias, postop, out_f32, bf16)
    assert np.array_equal(mine.view(np.uint8), theirs.view(np.uint8))


@pytest.mark.parametrize("bf16", [False, True])
def test_scale_a_and_int8_gold_bitwise(orc, bf16):
    M, K, N = 37, 512, 48
    g = synth.rng(21)
    A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
    A[3, :128] = 0  # an all-zero group: absmax floors at FLT_EPSILON
    B = synth.int2_weights(g, K, N)
    SB = synth.scales(g, K, N, bf16, 0.75, 15.75)
    SA = orc.scale_a(A, M, K, bf16)
    SA_ref = orc.ref_scale_a(A, M, K, bf16)
    assert np.array_equal(SA[:, :M], SA_ref[:, :M])
    assert np.array_equal(orc.int8_gold(A, B, SA, SB, M, K, N, bf16).view(np.uint32),
                          orc.ref_int8_gold(A, B, SA, SB, M, K, N, bf16).view(np.uint32))


@pytest.mark.parametrize("z", [0.05, 0.4, 0.95])
def test_bitcos_decode_ranks_gold_bitwise(orc, z):
    """Reference-generated BITCOS buffers (bitcos_random) through both decoders."""
    K, N, M = 1024, 48, 3
    buf = orc.ref_bitcos_random(K, N, z, 1234)
    codes = orc.bitcos_decode(buf, K, N)
    assert np.array_equal(codes, orc.ref_bitcos_decode(buf, K, N))
    for ls in (1, 2, 3, 4, 8):
        assert np.array_equal(orc.bitcos_slice_ranks(buf, K, N, ls), orc.ref_bitcos_slice_ranks(buf, K, N, ls))
        assert np.array_equal(formats.bitcos_slice_ranks(buf, K, N, ls), orc.ref_bitcos_slice_ranks(buf, K, N, ls))
    # our packer re-packs the decoded codes into the identical buffer
    assert np.array_equal(orc.bitcos_pack(codes), buf)
    assert np.array_equal(formats.bitcos_pack(codes), buf)
    for bf16 in (False, True):
        g = synth.rng(5)
        A = formats.f32_to_dt(g.uniform(-5, 5, (M, K)).astype(np.float32), bf16)
        S = synth.scales(g, K, N, bf16, 0.75, 15.75)
        assert np.array_equal(orc.bitcos_gold(A, buf, S, M, K, N, bf16).view(np.uint32),
                              orc.ref_bitcos_gold(A, buf, S, M, K, N, bf16).view(np.uint32))


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("out_f32", [False, True])
def test_epilogue_postop5_is_bias_then_residual(orc, out_f32, bf16):
    """postop 5 (bias + residual, no single reference counterpart) equals the
    reference's epilogue_ref applied twice (common/epilogue.hpp:98-115):
    postop 3 into fp32, then postop 2 into the requested output type."""
    g = synth.rng(55 + out_f32)
    M, N = 6, 160
    acc = (g.standard_normal((M, N)) * 6).astype(np.float32)
    acc[0, :6] = [0.0, -0.0, 1e-8, -3.0, 65000.0, -1e30]
    other = formats.f32_to_dt(g.uniform(-4, 4, (M, N)).astype(np.float32), bf16)
    bias_f = g.uniform(-8, 8, N).astype(np.float32)
    bias = bias_f if out_f32 else formats.f32_to_dt(bias_f, bf16)
    mine = orc.epilogue(acc, other, bias, 5, out_f32, bf16)
    bias32 = bias_f if out_f32 else formats.dt_to_f32(bias, bf16)  # DT -> fp32 is exact
    step1 = orc.ref_epilogue(acc, None, bias32, 3, True, bf16)
    theirs = orc.ref_epilogue(step1, other, None, 2, out_f32, bf16)
    assert np.array_equal(mine.view(np.uint8), theirs.view(np.uint8))
