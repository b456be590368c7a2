"""Pin the C oracle by what the mathematics fixes, independently of the
reference build: IEEE closed forms, dense float64 products, brute-force
Hadamard matrices, round trips and permutation invariants.  Each check is
chosen so that a plausible slip (dropped scale, transposed operand, wrong
rounding, wrong stage order or sign) fails it.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth


# ---- DT conversions (common/dt16.hpp:18-42) -------------------------------

def test_tof_fp16_ieee_exhaustive(orc):
    h = np.arange(65536, dtype=np.uint16)
    want = h.view(np.float16).astype(np.float32)
    got = orc.tof(h, False)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_tof_bf16_is_shift(orc):
    h = np.arange(65536, dtype=np.uint16)
    assert np.array_equal(orc.tof(h, True).view(np.uint32), h.astype(np.uint32) << 16)


def test_fromf_fp16_rte(orc):
    g = np.random.default_rng(0)
    f = np.concatenate([
        g.standard_normal(100000).astype(np.float32) * np.float32(1000),
        g.standard_normal(20000).astype(np.float32) * np.float32(1e-5),  # subnormal range
        np.array([65504, 65519.99, 65520, 65536, 2.0**-25, 2.0**-24 * 1.5, 2.0**-24 * 2.5,
                  1 + 2.0**-11, 1 + 3 * 2.0**-11, -0.0, np.inf, -np.inf], np.float32)])
    got = orc.fromf(f, False)
    want = f.astype(np.float16).view(np.uint16)  # numpy converts with RTE
    assert np.array_equal(got, want)


def test_fromf_bf16_rte_closed_form(orc):
    g = np.random.default_rng(1)
    f = np.concatenate([g.standard_normal(100000).astype(np.float32),
                        np.array([1 + 2.0**-8, 1 + 3 * 2.0**-8, 3.3895314e38, np.inf], np.float32)])
    got = orc.fromf(f, True)
    # RTE computed independently in float64: nearest bf16 value, ties to even
    hi = (f.view(np.uint32) >> 16).astype(np.uint64)
    lo_val = (hi.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    up_val = ((hi + 1).astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    x = f.astype(np.float64)
    d_lo, d_up = np.abs(x - lo_val), np.abs(up_val - x)
    choose_up = (d_up < d_lo) | ((d_up == d_lo) & (hi % 2 == 1))
    want = np.where(choose_up, hi + 1, hi).astype(np.uint16)
    fin = np.isfinite(f) & np.isfinite(up_val)
    assert np.array_equal(got[fin], want[fin])


def test_fromf_bf16_nan_quieted(orc):
    f = np.array([0x7F800001, 0xFF812345], np.uint32).view(np.float32)
    got = orc.fromf(f, True)
    assert list(got) == [0x7F80 | 0x40, 0xFF81 | 0x40]


# ---- int2 gold: int2_fp16_upcvt/main.cpp:79-98 ---------------------------

@pytest.mark.parametrize("bf16", [False, True])
def test_int2_gold_vs_dense_float64(orc, bf16):
    M, K, N = 3, 512, 48
    g = synth.rng(2)
    A = synth.activations(g, (M, K), bf16)
    B = synth.int2_weights(g, K, N)
    S = synth.scales(g, K, N, bf16)
    got = orc.int2_gold(A, B, S, M, K, N, bf16).astype(np.float64)
    W = formats.unpack_int2(B, K).astype(np.float64) * np.repeat(formats.dt_to_f32(S, bf16), 128, axis=0)
    want = formats.dt_to_f32(A, bf16).astype(np.float64) @ W
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    # a transposed group scale, or a dropped one, is caught
    W_bad = formats.unpack_int2(B, K).astype(np.float64)
    assert not np.allclose(got, formats.dt_to_f32(A, bf16).astype(np.float64) @ W_bad, rtol=1e-3)


def test_code_two_reads_minus_two(orc):
    """code_to_value: 2-bit two's complement, so code 2 (never generated) is -2."""
    B = np.full((1, 16), 0, np.uint32)
    B[0, 0] = 0b10  # row 0 of column 0 has code 2
    A = formats.f32_to_dt(np.ones((1, 16)), False)
    A = np.pad(A, ((0, 0), (0, 112)))
    Bk = np.zeros((8, 16), np.uint32)
    Bk[0] = B[0]
    S = formats.f32_to_dt(np.ones((1, 16)), False)
    out = orc.int2_gold(A, Bk, S, 1, 128, 16, False)
    assert out[0, 0] == -2.0 and np.all(out[0, 1:] == 0.0)


def test_int2_dequant_closed_form(orc):
    K, N = 128, 16
    B = np.zeros((K // 16, N), np.uint32)
    for n in range(N):
        B[:, n] = 0x1F3 * (n + 1)  # mixed codes
    S = formats.f32_to_dt(np.linspace(0.5, 2.0, (K // 128) * N).reshape(1, N), False)
    W = orc.int2_dequant(B, S, K, N)
    codes = ((B[:, None, :] >> (2 * np.arange(16, dtype=np.uint32))[None, :, None]) & 3).reshape(K, N)
    s = np.repeat(S, 128, axis=0)
    want = np.where(codes & 1, np.where(codes & 2, s ^ 0x8000, s), 0).astype(np.uint16)
    assert np.array_equal(W, want)


# ---- epilogue: common/epilogue.hpp:82, :98-115 ----------------------------

@pytest.mark.parametrize("postop", [1, 2, 3, 4, 5])
def test_epilogue_formulas(orc, postop):
    g = synth.rng(9)
    M, N = 2, 64
    acc = (g.standard_normal((M, N)) * 5).astype(np.float32)
    acc[0, 0], acc[0, 1] = -10.0, -9.5
    other = formats.f32_to_dt(g.uniform(-4, 4, (M, N)).astype(np.float32), False)
    bias = g.uniform(-8, 8, N).astype(np.float32)
    got = orc.epilogue(acc, other, bias, postop, True, False).astype(np.float64)
    a = acc.astype(np.float64)
    o = formats.dt_to_f32(other, False).astype(np.float64)
    sig = np.where(a <= -10, 0.0, 1.0 / (1.0 + np.exp(-a)))
    want = {1: a * sig * o, 2: a + o, 3: a + bias, 4: sig, 5: a + bias + o}[postop]
    assert np.allclose(got, want, rtol=1e-5, atol=1e-6)
    if postop == 4:
        assert got[0, 0] == 0.0 and got[0, 1] > 0.0  # the x <= -10 clamp


# ---- int8 quantization: int2_via_int2_x_int8_dpas/main.cpp:82-103 ---------

def test_scale_a_closed_form(orc):
    M, K = 3, 256
    A = np.zeros((M, K), np.float32)
    A[0, :128] = np.linspace(-3, 2, 128)
    A[1, 128:] = 0.0  # all-zero group -> 127 / FLT_EPSILON
    A[2] = np.float32(0.5)
    Ah = formats.f32_to_dt(A, False)
    SA = orc.scale_a(Ah, M, K, False)
    assert SA.shape == (2, 32)
    assert SA[0, 0] == formats.f32_to_dt(np.float32(127.0) / np.float32(3.0), False)
    assert SA[1, 1] == formats.f32_to_dt(np.float32(127.0 / np.finfo(np.float32).eps), False)  # inf in fp16
    assert SA[0, 2] == formats.f32_to_dt(np.float32(254.0), False)


def test_quant_rte_and_saturation(orc):
    M, K = 1, 128
    # SA = 1.0 (absmax 127): products are the values themselves
    vals = np.array([127, 2.5, 3.5, -2.5, -0.5, 0.5, 1.5, -127, 126.5, -126.5], np.float32)
    A = np.zeros((M, K), np.float32)
    A[0, :vals.size] = vals
    Ah = formats.f32_to_dt(A, False)
    SA = orc.scale_a(Ah, M, K, False)
    assert formats.dt_to_f32(SA[0, :1], False)[0] == 1.0
    q = orc.quant_a(Ah, SA, M, K, False)
    assert list(q[0, :vals.size]) == [127, 2, 4, -2, 0, 0, 2, -127, 126, -126]
    # saturation: a scale that pushes beyond 127 clamps (bf16 SA rounding can)
    SA2 = formats.f32_to_dt(np.full((1, 32), 2.0, np.float32), False)
    q2 = orc.quant_a(Ah, SA2, M, K, False)
    assert q2[0, 0] == 127 and q2[0, 7] == -128


def test_quant_overflowing_fp16_scale_saturates(orc):
    """fp16 group with absmax < 127/65504: SA = inf, so a * SA is +-inf (saturate
    to 127 / -128) or NaN for a = 0 (-> 0), the device kernel's
    convert_char8_sat_rte semantics (int2_int8_dpas.cl:120)."""
    M, K = 1, 128
    A = np.zeros((M, K), np.float32)
    A[0, :3] = [1e-3, -1e-3, 0.0]
    Ah = formats.f32_to_dt(A, False)
    SA = orc.scale_a(Ah, M, K, False)
    assert SA[0, 0] == 0x7C00  # +inf
    q = orc.quant_a(Ah, SA, M, K, False)
    assert list(q[0, :3]) == [127, -128, 0]
    assert (q[0, 3:] == 0).all()


@pytest.mark.parametrize("bf16", [False, True])
def test_int8_gold_vs_float64(orc, bf16):
    M, K, N = 4, 384, 32
    g = synth.rng(12)
    A = synth.activations(g, (M, K), bf16)
    B = synth.int2_weights(g, K, N)
    SB = synth.scales(g, K, N, bf16)
    SA = orc.scale_a(A, M, K, bf16)
    got = orc.int8_gold(A, B, SA, SB, M, K, N, bf16).astype(np.float64)
    q = orc.quant_a(A, SA, M, K, bf16).astype(np.float64)
    v = formats.unpack_int2(B, K).astype(np.float64)
    sa = formats.dt_to_f32(SA[:, :M], bf16).astype(np.float64)  # [G, M]
    sb = formats.dt_to_f32(SB, bf16).astype(np.float64)        # [G, N]
    want = np.zeros((M, N))
    for gi in range(K // 128):
        dot = q[:, gi * 128:(gi + 1) * 128] @ v[gi * 128:(gi + 1) * 128]
        want += dot * sb[gi][None, :] / sa[gi][:, None]
    assert np.allclose(got, want, rtol=1e-5, atol=1e-5)
    # and the dequantised product is close to the float product (quantization error only)
    Wf = v * np.repeat(sb, 128, axis=0)
    approx = formats.dt_to_f32(A, bf16).astype(np.float64) @ Wf
    assert np.abs(got - approx).max() < 0.05 * np.abs(approx).max()


# ---- BITCOS: common/bitcos.hpp -------------------------------------------

@pytest.mark.parametrize("z", [0.0, 0.3, 0.7, 1.0])
def test_bitcos_round_trip(orc, z):
    K, N = 256, 32
    g = synth.rng(int(z * 10))
    codes = synth.ternary_codes(g, K, N, z)
    buf = orc.bitcos_pack(codes)
    assert np.array_equal(buf, formats.bitcos_pack(codes))
    assert np.array_equal(orc.bitcos_decode(buf, K, N), codes)
    nnz = (codes != 0).sum(axis=0)
    assert buf.size == K // 32 * N + N + int(((nnz + 31) // 32).sum()) + 4
    # slice ranks = non-zeros above each boundary
    for ls in (2, 4):
        sr = orc.bitcos_slice_ranks(buf, K, N, ls).reshape(ls - 1, N)
        for s in range(1, ls):
            assert np.array_equal(sr[s - 1], (codes[: s * K // ls] != 0).sum(axis=0))


def test_bitcos_gold_equals_int2_gold(orc):
    """The same ternary matrix through both formats gives the same fp32 result
    (both golds skip zeros and accumulate per group in k order)."""
    K, N, M = 512, 32, 2
    g = synth.rng(8)
    codes = synth.ternary_codes(g, K, N, 0.5)
    A = synth.activations(g, (M, K), False)
    S = synth.scales(g, K, N, False)
    a = orc.bitcos_gold(A, orc.bitcos_pack(codes), S, M, K, N, False)
    b = orc.int2_gold(A, formats.pack_int2(codes), S, M, K, N, False)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))


def test_bitcos_dequant_closed_form(orc):
    K, N = 128, 16
    g = synth.rng(13)
    codes = synth.ternary_codes(g, K, N, 0.4)
    S = synth.scales(g, K, N, True)
    W = orc.bitcos_dequant(orc.bitcos_pack(codes), S, K, N)
    s = np.repeat(S, 128, axis=0)
    want = np.where(codes == 0, 0, np.where(codes > 0, s, s ^ 0x8000)).astype(np.uint16)
    assert np.array_equal(W, want)


# ---- FWHT: hadamard/hadamard_fwht.cl --------------------------------------

def _sylvester(n):
    H = np.array([[1.0]])
    while H.shape[0] < n:
        H = np.block([[H, H], [H, -H]])
    return H


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("HB", [256, 512])
def test_fwht_vs_sylvester(orc, HB, bf16):
    rows, K = 2, 2 * HB
    g = synth.rng(HB)
    x = synth.activations(g, (rows, K), bf16)
    s = (g.integers(0, 2, K) * 2 - 1).astype(np.int8)
    y = formats.dt_to_f32(orc.fwht(x, s, rows, K, HB, True, bf16), bf16).astype(np.float64)
    H = _sylvester(HB) / np.sqrt(HB)
    xf = formats.dt_to_f32(x, bf16).astype(np.float64) * s
    want = np.concatenate([xf[:, b * HB:(b + 1) * HB] @ H.T for b in range(K // HB)], axis=1)
    tol = 2.0 ** (-8 if bf16 else -11)
    assert np.allclose(y, want, rtol=2 * tol, atol=2 * tol)
    # SCALE is 1/sqrt(HB)
    assert abs(orc.fwht_scale(HB) - 1 / np.sqrt(HB)) < 1e-7


def test_fwht_involution_and_tail(orc):
    """H_n / sqrt(n) is an involution; a K % HB tail is its own smaller block."""
    HB, K, rows = 512, 5376, 1
    g = synth.rng(77)
    xf = g.standard_normal((rows, K)).astype(np.float32)
    x = formats.f32_to_dt(xf, False)
    y = orc.fwht(x, None, rows, K, HB, False, False)
    z = orc.fwht(y, None, rows, K, HB, False, False)
    assert np.allclose(formats.dt_to_f32(z, False), formats.dt_to_f32(x, False), atol=5e-3, rtol=5e-3)
    # the 256-wide tail transformed on its own
    tail = formats.dt_to_f32(x[:, 5120:], False).astype(np.float64) @ (_sylvester(256) / 16).T
    assert np.allclose(formats.dt_to_f32(y[:, 5120:], False), tail, atol=4e-3, rtol=4e-3)


def test_fwht_rejects_bad_hb(orc):
    x = np.zeros((1, 1000), np.uint16)
    with pytest.raises(ValueError):
        orc.fwht(x, None, 1, 1000, 512, False, False)  # tail 488 is not a power of two
    with pytest.raises(ValueError):
        orc.fwht(x, None, 1, 1000, 100, False, False)


# ---- MoE: int2_moe/int2_moe_prefill.cl, int2_moe/prefill.cpp ---------------

def test_moe_route_invariants(orc):
    g = synth.rng(1)
    T, E, topk, rpt = 64, 16, 4, 32
    ids = np.stack([g.choice(E, topk, replace=False) for _ in range(T)]).ravel().astype(np.int32)
    meta, perm, inv = orc.moe_route(ids, E, rpt)
    G = ids.size
    assert np.array_equal(np.sort(perm), np.arange(G))
    assert np.array_equal(perm[inv], np.arange(G)) and np.array_equal(inv[perm], np.arange(G))
    cnt = np.bincount(ids, minlength=E)
    assert np.array_equal(meta[:E + 1], np.concatenate([[0], np.cumsum(cnt)]))
    tiles = (cnt + rpt - 1) // rpt
    assert np.array_equal(meta[E + 1:], np.concatenate([[0], np.cumsum(tiles)]))
    assert np.all(np.diff(ids[perm]) >= 0)            # segments sorted by expert
    for e in range(E):                                  # stable inside a segment
        seg = perm[meta[e]:meta[e + 1]]
        assert np.all(np.diff(seg) > 0)


def test_moe_combine_closed_form(orc):
    g = synth.rng(2)
    T, topk, N = 5, 3, 32
    G = T * topk
    Y = g.standard_normal((G, N)).astype(np.float32)
    inv = g.permutation(G).astype(np.int32)
    RW = formats.f32_to_dt(g.uniform(0, 1, G).astype(np.float32), True)
    O = formats.dt_to_f32(orc.moe_combine(Y, inv, RW, T, topk, N, True), True)
    rw = formats.dt_to_f32(RW, True).reshape(T, topk)
    want = np.einsum("tj,tjn->tn", rw.astype(np.float64), Y[inv].reshape(T, topk, N).astype(np.float64))
    assert np.allclose(O, want, rtol=1e-2, atol=1e-3)


def test_moe_ref_tokens_vs_dense(orc):
    g = synth.rng(3)
    T, E, topk, H, I = 2, 4, 2, 128, 128
    X = synth.activations(g, (T, H), False)
    ids = np.array([0, 3, 1, 3], np.int32)
    RW = formats.f32_to_dt(np.array([0.6, 0.4, 0.7, 0.3], np.float32), False)
    Bg = np.stack([synth.int2_weights(g, H, I) for _ in range(E)])
    Bu = np.stack([synth.int2_weights(g, H, I) for _ in range(E)])
    Bd = np.stack([synth.int2_weights(g, I, H) for _ in range(E)])
    Sg = np.stack([synth.scales(g, H, I, False) for _ in range(E)])
    Su = np.stack([synth.scales(g, H, I, False) for _ in range(E)])
    Sd = np.stack([synth.scales(g, I, H, False) for _ in range(E)])
    O = orc.moe_ref_tokens(X, ids, RW, 0, T, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, False)
    Od = orc.moe_ref_tokens(X, ids, RW, 0, T, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, False, round_up=False)

    def W(B, S, K):
        return formats.unpack_int2(B, K).astype(np.float64) * np.repeat(formats.dt_to_f32(S, False), 128, axis=0)

    x = formats.dt_to_f32(X, False).astype(np.float64)
    rw = formats.dt_to_f32(RW, False)
    for t in range(T):
        o = np.zeros(H)
        for j in range(topk):
            e = ids[t * topk + j]
            sg, su = x[t] @ W(Bg[e], Sg[e], H), x[t] @ W(Bu[e], Su[e], H)
            h = sg / (1 + np.exp(-sg)) * su
            o += (h @ W(Bd[e], Sd[e], I)) * rw[t * topk + j]
        assert np.allclose(O[t], o, rtol=2e-2, atol=2e-3 * np.abs(o).max())
        # the decode check (up not rounded): the same within its one DT rounding of h
        assert np.allclose(Od[t], o, rtol=2e-2, atol=2e-3 * np.abs(o).max())
    # and the two modes differ only through up's rounding: tiny, but not zero
    assert 0 < np.abs(Od - O).max() <= 2e-2 * np.abs(O).max()
