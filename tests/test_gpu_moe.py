"""GPU parity of the int2 MoE prefill (route, gather, grouped GEMM, combine, the
whole layer) through the C ABI.

Reference test design followed: int2_moe/prefill.cpp -- a layer over random
routing checked on its first tokens against a double-precision host reference
with the rule max|err| / max|ref| < 1e-2 (:288-319, restated by the oracle's
moe_ref_tokens) -- plus stage-by-stage checks the reference does not have:
route and gather exact against the oracle's stable counting sort, each
expert's GEMM rows within 1e-3 + 1e-2 |ref| of the int2 host gold, and the
combine bit-exact against the oracle's fp32 sum in slot order.
"""
from __future__ import annotations

import numpy as np
import pytest

from ternocl_amd import formats, synth
from tests.gpu_util import allclose_report, dev_dt, dev_raw, host_u16

pytestmark = pytest.mark.gpu


def _ints(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a, np.int32)).cuda()


def _route(T, ids, G, E):
    import torch
    meta = torch.zeros(2 * E + 2, dtype=torch.int32, device="cuda")
    perm = torch.full((G,), -7, dtype=torch.int32, device="cuda")
    inv = torch.full((G,), -7, dtype=torch.int32, device="cuda")
    T.int2_moe_route(_ints(ids), meta, perm, inv, G, E)
    torch.cuda.synchronize()
    return meta, perm, inv


# past 64 x 1024 ids a route workgroup ranks its chunk in several passes
@pytest.mark.parametrize("G,E,skew", [(1, 1, False), (100, 7, False), (16384, 64, False), (16384, 64, True),
                                      (20000, 128, True), (3000, 512, False), (5000, 33, True), (40000, 64, False),
                                      (65537, 64, False), (100000, 64, True), (262144, 128, True),
                                      (300001, 512, False)])
def test_moe_route_matches_stable_sort(dev, orc, G, E, skew):
    import ternocl_amd as T
    g = synth.rng(G + E)
    if skew:  # the reference driver's skewed popularity (int2_moe/prefill.cpp:185-200), some experts empty
        p = 1.0 / (1.0 + np.arange(E) / 8.0)
        p[E // 2: E // 2 + 3] = 0.0
        ids = g.choice(E, size=G, p=p / p.sum()).astype(np.int32)
    else:
        ids = g.integers(0, E, G, dtype=np.int32)
    meta, perm, inv = _route(T, ids, G, E)
    m, pm, iv = orc.moe_route(ids, E, T.moe_tile_rows())
    assert np.array_equal(meta.cpu().numpy(), m)
    assert np.array_equal(perm.cpu().numpy(), pm)
    assert np.array_equal(inv.cpu().numpy(), iv)


@pytest.mark.parametrize("G", [3000, 150000])
def test_moe_route_drops_out_of_range_ids(dev, orc, G):
    import ternocl_amd as T
    E = 16
    g = synth.rng(5)
    ids = g.integers(0, E, G, dtype=np.int32)
    bad = g.random(G) < 0.1
    ids[bad] = np.where(g.random(bad.sum()) < 0.5, -1, E + 3)
    meta, perm, inv = _route(T, ids, G, E)
    keep = np.flatnonzero(~bad)
    m, pm, _ = orc.moe_route(ids[keep], E, T.moe_tile_rows())
    assert np.array_equal(meta.cpu().numpy(), m)
    n = int(m[E])
    assert np.array_equal(perm.cpu().numpy()[:n], keep[pm])
    assert (perm.cpu().numpy()[n:] == -1).all(), "perm past the kept rows must be -1"
    iv = inv.cpu().numpy()
    assert (iv[bad] == -1).all()
    assert np.array_equal(iv[keep[pm]], np.arange(n))


@pytest.mark.parametrize("G", [3000, 40000])
def test_moe_gather_after_dropped_ids(dev, orc, G):
    """Route then gather with out-of-range ids: the kept rows are the token rows in
    expert order and the rows past them (perm = -1) come out as zeros; the gather
    reads nothing outside X (single- and multi-block route)."""
    import torch
    import ternocl_amd as T
    E, topk, K, bf16 = 16, 4, 256, False
    Tk = G // topk
    g = synth.rng(G)
    X = synth.activations(g, (Tk, K), bf16)
    ids = g.integers(0, E, G, dtype=np.int32)
    bad = g.random(G) < 0.2
    ids[bad] = np.where(g.random(bad.sum()) < 0.5, -3, E)
    meta, perm, _ = _route(T, ids, G, E)
    dXs = torch.full((G, K), 7.0, dtype=torch.float16, device="cuda")
    T.int2_moe_gather(dev_dt(X, bf16), perm, dXs, G, K, topk)
    torch.cuda.synchronize()
    n = int(meta.cpu().numpy()[E])
    assert n == int((~bad).sum())
    got = host_u16(dXs)
    pm = perm.cpu().numpy()
    assert np.array_equal(got[:n], X[pm[:n] // topk])
    assert (got[n:] == 0).all()


def test_moe_gather(dev, orc):
    import torch
    import ternocl_amd as T
    Tk, E, topk, K, bf16 = 50, 8, 3, 384, True
    g = synth.rng(1)
    X = synth.activations(g, (Tk, K), bf16)
    ids, _ = synth.moe_routing(g, Tk, E, topk, bf16)
    G = Tk * topk
    _, perm, _ = _route(T, ids, G, E)
    dXs = torch.zeros((G, K), dtype=torch.bfloat16, device="cuda")
    T.int2_moe_gather(dev_dt(X, bf16), perm, dXs, G, K, topk)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(dXs), orc.moe_gather(X, perm.cpu().numpy(), topk))


def _experts(g, E, K, N, bf16):
    B = np.stack([synth.int2_weights(g, K, N) for _ in range(E)])
    S = np.stack([synth.scales(g, K, N, bf16) for _ in range(E)])
    return B, S


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("postop,out_f32,via_perm", [(0, False, True), (1, False, True), (0, True, False),
                                                     (2, True, True), (4, False, False)])
def test_moe_gemm_rows_match_int2_gold(dev, orc, bf16, postop, out_f32, via_perm):
    import torch
    import ternocl_amd as T
    Tk, E, topk, K, N = 300, 6, 2, 512, 272
    print(f"moe gemm postop={postop} out_f32={out_f32} perm={via_perm} bf16={bf16}", flush=True)
    g = synth.rng(40 + postop)
    X = synth.activations(g, (Tk, K), bf16)
    ids, _ = synth.moe_routing(g, Tk, E, topk, bf16)
    G = Tk * topk
    B, S = _experts(g, E, K, N, bf16)
    other = synth.activations(g, (G, N), bf16)
    meta, perm, _ = _route(T, ids, G, E)
    pm, mt = perm.cpu().numpy(), meta.cpu().numpy()
    Xs = X[pm // topk]
    dA = dev_dt(X if via_perm else Xs, bf16)
    dC = torch.zeros((G, N), dtype=torch.float32 if out_f32 else dA.dtype, device="cuda")
    T.int2_moe_gemm(meta, dA, perm if via_perm else None, topk, dev_raw(B), dev_dt(S, bf16), dC,
                    dev_dt(other, bf16), E, G, N, K, postop, out_f32)
    torch.cuda.synchronize()
    got = dC.cpu().numpy() if out_f32 else formats.dt_to_f32(host_u16(dC), bf16)
    for e in range(E):
        r0, r1 = int(mt[e]), int(mt[e + 1])
        if r0 == r1:
            continue
        acc = orc.int2_gold(Xs[r0:r1], B[e], S[e], r1 - r0, K, N, bf16)
        want = orc.epilogue(acc, other[r0:r1], None, postop, out_f32, bf16)
        want = want if out_f32 else formats.dt_to_f32(want, bf16)
        bad, dmax = allclose_report(got[r0:r1], want)
        assert bad == 0, f"expert {e}: {bad} bad (max |d| {dmax})"


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_combine_bit_exact(dev, orc, bf16):
    import torch
    import ternocl_amd as T
    Tk, E, topk, N = 200, 16, 8, 2048
    g = synth.rng(8)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    G = Tk * topk
    _, _, inv = _route(T, ids, G, E)
    Y = g.standard_normal((G, N), dtype=np.float32)
    dO = torch.zeros((Tk, N), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    T.int2_moe_combine(torch.from_numpy(Y).cuda(), inv, dev_dt(RW, bf16), dO, Tk, topk, N)
    torch.cuda.synchronize()
    assert np.array_equal(host_u16(dO), orc.moe_combine(Y, inv.cpu().numpy(), RW, Tk, topk, N, bf16))


def _special_f32_bits(g, n):
    """fp32 bit patterns of every class the DT rounding meets: ties and near-ties at the bf16 and
    fp16 rounding points, fp32 and DT denormals, the largest finite values and those that round to
    the DT's infinity, signed zeros, infinities, NaNs, then random patterns to fill n."""
    hi = g.integers(0, 1 << 16, 512, dtype=np.uint64)
    pats = [(hi << 16) | lo for lo in (0x0000, 0x7FFF, 0x8000, 0x8001, 0xFFFF)]  # bf16 ties / near-ties
    e = g.integers(0x33, 0x48, 512, dtype=np.uint64) << 23  # exponents 2^-26 .. 2^16: fp16 denormals to overflow
    m = g.integers(0, 1 << 10, 512, dtype=np.uint64) << 13
    pats += [e | m | lo for lo in (0x0000, 0x0FFF, 0x1000, 0x1001)]  # fp16 ties / near-ties
    pats.append(np.array([0, 1, 0x7FFFFF, 0x8000, 0x18000, 0x17FFF, 0x7F7FFFFF, 0x7F7F8000, 0x7F7F7FFF,
                          0x477FE000, 0x477FEFFF, 0x477FF000, 0x477FF001, 0x387FE000, 0x33800000, 0x33000001,
                          0x7F800000, 0x7FC00000, 0x7F800001, 0x7FBFFFFF, 0x7FFFFFFF, 0x3F808000, 0x3F818000],
                         dtype=np.uint64))
    base = np.concatenate(pats)
    base = np.concatenate([base, base | (1 << 31)])  # both signs
    rnd = g.integers(0, 1 << 32, max(0, n - base.size), dtype=np.uint64)
    return np.concatenate([base, rnd])[:n].astype(np.uint32)


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_combine_rounding_special_values(dev, orc, bf16):
    """The output rounding to DT (one expert, top-1, weight 1.0: O = DT(0 + 1.0 * Y)) bit for bit
    against the oracle's restatement of the reference's fromf (common/dt16.hpp:30-36) on every class
    of fp32 value; a NaN stays a NaN of its sign (its payload through the fp32 arithmetic is the
    platform's)."""
    import torch
    import ternocl_amd as T
    Tk, N = 16, 2048
    Yb = _special_f32_bits(synth.rng(9), Tk * N)
    Y = Yb.view(np.float32).reshape(Tk, N)
    _, _, inv = _route(T, np.zeros(Tk, np.int32), Tk, 1)
    RW = formats.f32_to_dt(np.ones(Tk, np.float32), bf16)
    dO = torch.zeros((Tk, N), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    T.int2_moe_combine(torch.from_numpy(Y.copy()).cuda(), inv, dev_dt(RW, bf16), dO, Tk, 1, N)
    torch.cuda.synchronize()
    got = host_u16(dO)
    want = orc.moe_combine(Y, inv.cpu().numpy(), RW, Tk, 1, N, bf16)
    nan = np.isnan(Y)
    assert nan.any() and np.isinf(Y).any()
    assert np.array_equal(got[~nan], want[~nan])
    gf = formats.dt_to_f32(got, bf16)
    assert np.isnan(gf[nan]).all() and np.array_equal(np.signbit(gf[nan]), np.signbit(Y[nan]))


def _layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16):
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    dO = torch.zeros((Tk, H), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    ws = torch.empty(T.int2_moe_prefill_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
    T.int2_moe_prefill(dev_dt(X, bf16), _ints(ids), dev_dt(RW, bf16), Tk, E, topk, H, I,
                       dev_raw(Bg), dev_dt(Sg, bf16), dev_raw(Bu), dev_dt(Su, bf16), dev_raw(Bd),
                       dev_dt(Sd, bf16), dO, ws)
    torch.cuda.synchronize()
    return host_u16(dO)


def _oracle_layer(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, rpt):
    """The layer composed from the oracle's stages, same semantics stage by stage."""
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    G = Tk * topk
    meta, perm, inv = orc.moe_route(ids, E, rpt)
    Xs = X[perm // topk]
    Y = np.zeros((G, H), np.float32)
    for e in range(E):
        r0, r1 = int(meta[e]), int(meta[e + 1])
        if r0 == r1:
            continue
        Me = r1 - r0
        U = orc.epilogue(orc.int2_gold(Xs[r0:r1], Bu[e], Su[e], Me, H, I, bf16), None, None, 0, False, bf16)
        Hs = orc.epilogue(orc.int2_gold(Xs[r0:r1], Bg[e], Sg[e], Me, H, I, bf16), U, None, 1, False, bf16)
        Y[r0:r1] = orc.epilogue(orc.int2_gold(Hs, Bd[e], Sd[e], Me, I, H, bf16), None, None, 0, True, bf16)
    return orc.moe_combine(Y, inv, RW, Tk, topk, H, bf16)


def _weights(g, E, H, I, bf16):
    return _experts(g, E, H, I, bf16), _experts(g, E, H, I, bf16), _experts(g, E, I, H, bf16)


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_layer_small(dev, orc, bf16):
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I = 96, 8, 2, 256, 384
    g = synth.rng(17)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    got = formats.dt_to_f32(_layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    want = formats.dt_to_f32(_oracle_layer(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, T.moe_tile_rows()), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    ref = orc.moe_ref_tokens(X, ids, RW, 0, 8, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16)
    rel = np.abs(got[:8] - ref).max() / np.abs(ref).max()
    assert rel < 1e-2, rel


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_layer_multi_tile_experts(dev, orc, bf16):
    """Experts spanning two to three 128-row tiles with ragged last tiles (T=512, E=8, top-4:
    ~256 rows each) and I = 1408 = 5.5 x 256 (a half-live last column tile): every output of
    the layer within 1e-3 + 1e-2 |ref| of the oracle's stage composition, so the tiles past
    each expert's first (the tile search's later row offsets, their perm rows and the
    live-block tail loops) are all compared."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I = 512, 8, 4, 256, 1408
    g = synth.rng(4242)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    counts = np.bincount(ids, minlength=E)
    rpt = T.moe_tile_rows()
    assert (counts > rpt).all() and (counts > 2 * rpt).any() and (counts % rpt != 0).all(), counts
    print(f"moe multi-tile T={Tk} E={E} topk={topk} H={H} I={I} bf16={bf16} rows/expert {counts.tolist()}",
          flush=True)
    W = _weights(g, E, H, I, bf16)
    got = formats.dt_to_f32(_layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    want = formats.dt_to_f32(_oracle_layer(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, rpt), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} of {got.size} outputs outside the rule (max |d| {dmax})"


# rows per expert: empty experts, tails of 1..64 rows (an odd count of them: one
# is left alone), tails of 65 and 72 rows, whole tiles with and without a tail
PAIR_COUNTS = [0, 64, 65, 1, 128, 129, 30, 200, 0, 63, 5, 7]


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_layer_pair_tiles(dev, orc, bf16):
    """The layer's tile list (two experts' tails of at most 64 rows share a row tile, the
    others alone): every output within 1e-3 + 1e-2 |ref| of the oracle's stage composition,
    at a routing made for it (top-1, the rows per expert of PAIR_COUNTS, shuffled)."""
    import torch
    import ternocl_amd as T
    E, topk, H, I = len(PAIR_COUNTS), 1, 256, 384
    g = synth.rng(777)
    ids = np.repeat(np.arange(E, dtype=np.int32), PAIR_COUNTS)
    g.shuffle(ids)
    Tk = ids.size
    print(f"moe pair tiles T={Tk} E={E} rows/expert {PAIR_COUNTS} bf16={bf16}", flush=True)
    X = synth.activations(g, (Tk, H), bf16)
    RW = formats.f32_to_dt(np.ones(Tk, np.float32), bf16)
    W = _weights(g, E, H, I, bf16)
    got = formats.dt_to_f32(_layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    want = formats.dt_to_f32(_oracle_layer(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, T.moe_tile_rows()), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} of {got.size} outputs outside the rule (max |d| {dmax})"


def _c5_check_tokens(Tk, seed=2026, n_random=8):
    """Tokens of the C5 layer the double-precision check covers: the first four (the first
    rows of every expert's first tile), the last four (their rows land at the ends of the
    expert segments, in the last tiles) and a seeded random sample."""
    g = np.random.default_rng(seed)
    rand = sorted(int(t) for t in g.choice(np.arange(4, Tk - 4), n_random, replace=False))
    return [(0, 4), (Tk - 4, Tk)] + [(t, t + 1) for t in rand]


def test_moe_layer_workload_shape(dev, orc):
    """T=2048 tokens, 64 experts, top-8, H=2048, I=1408, bf16: the first and last four tokens
    and a random sample against the double-precision reference check
    (int2_moe/prefill.cpp:288-319, rule rel < 1e-2), every output finite; two runs
    bit-identical."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I, bf16 = 2048, 64, 8, 2048, 1408, True
    g = synth.rng(2025)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    out = _layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16)
    got = formats.dt_to_f32(out, bf16)
    assert np.isfinite(got).all()
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    for t0, t1 in _c5_check_tokens(Tk):
        ref = orc.moe_ref_tokens(X, ids, RW, t0, t1, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16)
        rel = np.abs(got[t0:t1] - ref).max() / np.abs(ref).max()
        assert rel < 1e-2, (t0, t1, rel)
    again = _layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16)
    assert np.array_equal(out, again)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("I", [384, 512])
def test_moe_layer_equals_stage_composition(dev, orc, bf16, I):
    """The layer (up and gate as one launch) gives, bit for bit, what the separate entry
    points give stage by stage: route, up (POSTOP 0), gate (POSTOP 1 on up), down (fp32),
    combine.  I = 384 takes 128-column tiles, I = 512 256-column tiles."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H = 160, 8, 4, 256
    g = synth.rng(31 + I)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    got = _layer(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16)
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    G = Tk * topk
    dt = torch.bfloat16 if bf16 else torch.float16
    meta, perm, inv = _route(T, ids, G, E)
    dX = dev_dt(X, bf16)
    U = torch.zeros((G, I), dtype=dt, device="cuda")
    Hs = torch.zeros((G, I), dtype=dt, device="cuda")
    Y = torch.zeros((G, H), dtype=torch.float32, device="cuda")
    O = torch.zeros((Tk, H), dtype=dt, device="cuda")
    T.int2_moe_gemm(meta, dX, perm, topk, dev_raw(Bu), dev_dt(Su, bf16), U, None, E, G, I, H, 0, False)
    T.int2_moe_gemm(meta, dX, perm, topk, dev_raw(Bg), dev_dt(Sg, bf16), Hs, U, E, G, I, H, 1, False)
    T.int2_moe_gemm(meta, Hs, None, 1, dev_raw(Bd), dev_dt(Sd, bf16), Y, None, E, G, H, I, 0, True)
    T.int2_moe_combine(Y, inv, dev_dt(RW, bf16), O, Tk, topk, H)
    torch.cuda.synchronize()
    assert np.array_equal(got, host_u16(O))


# ---- the decode layer (int2_moe/int2_moe.cl, int2_moe/main.cpp) ----------------------

def _decode(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16, ws_bytes=None):
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    dO = torch.full((Tk, H), 7.0, dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    n = T.int2_moe_decode_ws_bytes(Tk, topk, H, I) if ws_bytes is None else ws_bytes
    ws = torch.full((n,), 0x7f, dtype=torch.uint8, device="cuda")
    T.int2_moe_decode(dev_dt(X, bf16), _ints(ids), dev_dt(RW, bf16), Tk, E, topk, H, I,
                      dev_raw(Bg), dev_dt(Sg, bf16), dev_raw(Bu), dev_dt(Su, bf16), dev_raw(Bd),
                      dev_dt(Sd, bf16), dO, ws)
    torch.cuda.synchronize()
    return host_u16(dO)


def _oracle_decode(orc, X, ids, RW, Tk, topk, H, I, W, bf16):
    """The decode layer from the oracle's int2 gold, stage by stage: fp32 gate and up per
    assignment, h = DT(silu(gate) * up), fp32 down of h, then the weighted combine in slot order
    (assignment g = t * topk + j, int2_moe/main.cpp:263-289)."""
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    G = Tk * topk
    Y = np.zeros((G, H), np.float32)
    for g in range(G):
        e, x = int(ids[g]), X[g // topk: g // topk + 1]
        gate = orc.int2_gold(x, Bg[e], Sg[e], 1, H, I, bf16).astype(np.float64)
        up = orc.int2_gold(x, Bu[e], Su[e], 1, H, I, bf16).astype(np.float64)
        h = formats.f32_to_dt((gate / (1.0 + np.exp(-gate)) * up).astype(np.float32), bf16)
        Y[g] = orc.int2_gold(h, Bd[e], Sd[e], 1, I, H, bf16)[0]
    return orc.moe_combine(Y, np.arange(G, dtype=np.int32), RW, Tk, topk, H, bf16)


def _decode_case(seed, Tk, E, topk, H, I, bf16):
    g = synth.rng(seed)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    return X, ids, RW, _weights(g, E, H, I, bf16)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("Tk,E,topk,H,I", [(1, 8, 2, 256, 384), (2, 16, 4, 512, 256), (5, 6, 3, 384, 640),
                                          (3, 32, 8, 1024, 512), (2, 20, 16, 256, 128), (2, 24, 20, 256, 256)])
def test_moe_decode_matches_oracle(dev, orc, bf16, Tk, E, topk, H, I):
    """Every output within 1e-3 + 1e-2 |ref| of the oracle's stage composition, and the
    reference's own check (rel < 1e-2 of the double-precision layer, int2_moe/main.cpp:263-294).
    topk <= 16 takes the fused down-and-sum launch, topk = 20 the down GEMV and the sum kernel."""
    import torch
    import ternocl_amd as T
    print(f"moe decode T={Tk} E={E} topk={topk} H={H} I={I} bf16={bf16}", flush=True)
    X, ids, RW, W = _decode_case(100 + Tk * E + H, Tk, E, topk, H, I, bf16)
    got = formats.dt_to_f32(_decode(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    want = formats.dt_to_f32(_oracle_decode(orc, X, ids, RW, Tk, topk, H, I, W, bf16), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    ref = orc.moe_ref_tokens(X, ids, RW, 0, Tk, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16, round_up=False)
    rel = np.abs(got - ref).max() / np.abs(ref).max()
    assert rel < 1e-2, rel


@pytest.mark.parametrize("bf16", [False, True])
def test_moe_decode_reference_default_shape(dev, orc, bf16):
    """The reference driver's default problem (int2_moe/main.cpp:6): T=1, E=128, top-8,
    H=2048, I=768; two runs bit-identical."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I = 1, 128, 8, 2048, 768
    X, ids, RW, W = _decode_case(77, Tk, E, topk, H, I, bf16)
    out = _decode(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16)
    got = formats.dt_to_f32(out, bf16)
    bad, dmax = allclose_report(got, formats.dt_to_f32(_oracle_decode(orc, X, ids, RW, Tk, topk, H, I, W, bf16),
                                                       bf16))
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    ref = orc.moe_ref_tokens(X, ids, RW, 0, Tk, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16, round_up=False)
    assert np.abs(got - ref).max() / np.abs(ref).max() < 1e-2
    assert np.array_equal(out, _decode(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16))


def test_moe_decode_out_of_range_ids_add_nothing(dev, orc):
    """An id outside [0, E) contributes zero: the layer equals the oracle's with that slot's
    weight set to 0 (the prefill route drops such ids the same way)."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I, bf16 = 4, 12, 4, 256, 256, True
    X, ids, RW, W = _decode_case(9, Tk, E, topk, H, I, bf16)
    bad_ids = ids.copy()
    bad_ids[[1, 6, 7, 12]] = [-1, E, E + 100, -5]
    got = formats.dt_to_f32(_decode(T, torch, X, bad_ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    ok_ids, rw0 = ids.copy(), RW.copy()
    ok_ids[[1, 6, 7, 12]] = 0
    rw0[[1, 6, 7, 12]] = 0
    want = formats.dt_to_f32(_oracle_decode(orc, X, ok_ids, rw0, Tk, topk, H, I, W, bf16), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"


def test_moe_decode_rejects_bad_arguments(dev):
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I, bf16 = 2, 4, 2, 256, 256, False
    X, ids, RW, W = _decode_case(3, Tk, E, topk, H, I, bf16)
    need = T.int2_moe_decode_ws_bytes(Tk, topk, H, I)
    with pytest.raises(T.TernoclError):
        _decode(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16, ws_bytes=need - 256)
    with pytest.raises(T.TernoclError):
        _decode(T, torch, X[:, :192], ids, RW, Tk, E, topk, 192, I, W, bf16)


# ---- the int8 prefill layer (int2_moe/int2_moe_prefill_int8.cl, QMODE 1) ----------------

def _layer_int8(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16):
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    dO = torch.zeros((Tk, H), dtype=torch.bfloat16 if bf16 else torch.float16, device="cuda")
    ws = torch.empty(T.int2_moe_prefill_int8_ws_bytes(Tk, E, topk, H, I), dtype=torch.uint8, device="cuda")
    T.int2_moe_prefill_int8(dev_dt(X, bf16), _ints(ids), dev_dt(RW, bf16), Tk, E, topk, H, I,
                            dev_raw(Bg), dev_dt(Sg, bf16), dev_raw(Bu), dev_dt(Su, bf16), dev_raw(Bd),
                            dev_dt(Sd, bf16), dO, ws)
    torch.cuda.synchronize()
    return host_u16(dO)


def _oracle_layer_int8(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, rpt):
    """The int8 layer from the oracle's stages: expert-sorted rows, per-row quant_a scales,
    the s8 x s2 gold for up, gate (POSTOP 1 on up) and down (fp32), the combine."""
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    G = Tk * topk
    meta, perm, inv = orc.moe_route(ids, E, rpt)
    Xs = X[perm // topk]
    Y = np.zeros((G, H), np.float32)
    for e in range(E):
        r0, r1 = int(meta[e]), int(meta[e + 1])
        if r0 == r1:
            continue
        Me, Xe = r1 - r0, Xs[r0:r1]
        SAx = orc.scale_a(Xe, Me, H, bf16)
        U = orc.epilogue(orc.int8_gold(Xe, Bu[e], SAx, Su[e], Me, H, I, bf16), None, None, 0, False, bf16)
        Hs = orc.epilogue(orc.int8_gold(Xe, Bg[e], SAx, Sg[e], Me, H, I, bf16), U, None, 1, False, bf16)
        SAh = orc.scale_a(Hs, Me, I, bf16)
        Y[r0:r1] = orc.epilogue(orc.int8_gold(Hs, Bd[e], SAh, Sd[e], Me, I, H, bf16), None, None, 0, True, bf16)
    return orc.moe_combine(Y, inv, RW, Tk, topk, H, bf16)


@pytest.mark.parametrize("bf16", [False, True])
@pytest.mark.parametrize("Tk,E,topk,H,I", [(96, 8, 2, 256, 384), (300, 6, 3, 512, 256), (7, 16, 4, 384, 128)])
def test_moe_int8_layer_matches_oracle(dev, orc, bf16, Tk, E, topk, H, I):
    """Within 1e-3 + 1e-2 |ref| of the oracle's s8 x s2 stage composition, and the reference's
    own int8 check on the first tokens (rel < 5e-2 of the double-precision layer,
    int2_moe/prefill.cpp:288-319)."""
    import torch
    import ternocl_amd as T
    print(f"moe int8 layer T={Tk} E={E} topk={topk} H={H} I={I} bf16={bf16}", flush=True)
    g = synth.rng(300 + Tk + E)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    got = formats.dt_to_f32(_layer_int8(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    want = formats.dt_to_f32(_oracle_layer_int8(orc, X, ids, RW, Tk, E, topk, H, I, W, bf16, T.moe_tile_rows()),
                             bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    n = min(Tk, 8)
    ref = orc.moe_ref_tokens(X, ids, RW, 0, n, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16)
    assert np.abs(got[:n] - ref).max() / np.abs(ref).max() < 5e-2


def test_moe_int8_layer_workload_shape(dev, orc):
    """T=2048 tokens, 64 experts, top-8, H=2048, I=1408, bf16: the reference's int8 check on the
    first tokens (rel < 5e-2), every output finite, two runs bit-identical."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I, bf16 = 2048, 64, 8, 2048, 1408, True
    g = synth.rng(2026)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    out = _layer_int8(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16)
    got = formats.dt_to_f32(out, bf16)
    assert np.isfinite(got).all()
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    ref = orc.moe_ref_tokens(X, ids, RW, 0, 4, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, bf16)
    assert np.abs(got[:4] - ref).max() / np.abs(ref).max() < 5e-2
    assert np.array_equal(out, _layer_int8(T, torch, X, ids, RW, Tk, E, topk, H, I, W, bf16))


def test_moe_int8_layer_out_of_range_ids_add_nothing(dev, orc):
    """Ids outside [0, E) are dropped by the route: the int8 layer equals the oracle's
    composition with those slots' weights set to 0 (the kept rows route the same way)."""
    import torch
    import ternocl_amd as T
    Tk, E, topk, H, I, bf16 = 64, 8, 2, 256, 256, True
    g = synth.rng(44)
    X = synth.activations(g, (Tk, H), bf16)
    ids, RW = synth.moe_routing(g, Tk, E, topk, bf16)
    W = _weights(g, E, H, I, bf16)
    drop = np.array([1, 6, 7, 40, 101])
    bad_ids = ids.copy()
    bad_ids[drop] = [-1, E, E + 9, -3, E]
    got = formats.dt_to_f32(_layer_int8(T, torch, X, bad_ids, RW, Tk, E, topk, H, I, W, bf16), bf16)
    (Bg, Sg), (Bu, Su), (Bd, Sd) = W
    G = Tk * topk
    keep = np.setdiff1d(np.arange(G), drop)
    meta, pm, _ = orc.moe_route(bad_ids[keep], E, T.moe_tile_rows())
    Xs = X[keep[pm] // topk]
    Y = np.zeros((G, H), np.float32)
    for e in range(E):
        r0, r1 = int(meta[e]), int(meta[e + 1])
        if r0 == r1:
            continue
        Me, Xe = r1 - r0, Xs[r0:r1]
        SAx = orc.scale_a(Xe, Me, H, bf16)
        U = orc.epilogue(orc.int8_gold(Xe, Bu[e], SAx, Su[e], Me, H, I, bf16), None, None, 0, False, bf16)
        Hs = orc.epilogue(orc.int8_gold(Xe, Bg[e], SAx, Sg[e], Me, H, I, bf16), U, None, 1, False, bf16)
        SAh = orc.scale_a(Hs, Me, I, bf16)
        Y[keep[pm[r0:r1]]] = orc.epilogue(orc.int8_gold(Hs, Bd[e], SAh, Sd[e], Me, I, H, bf16), None, None, 0,
                                          True, bf16)
    rw0 = RW.copy()
    rw0[drop] = 0
    want = formats.dt_to_f32(orc.moe_combine(Y, np.arange(G, dtype=np.int32), rw0, Tk, topk, H, bf16), bf16)
    bad, dmax = allclose_report(got, want)
    assert bad == 0, f"{bad} bad (max |d| {dmax})"
