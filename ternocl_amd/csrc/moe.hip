// moe.hip -- int2 MoE prefill on gfx950: routing, gather and combine, and the
// layer driver that chains them with the grouped GEMMs of int2_gemm_mfma.hip.
// Replaces int2_moe_route / int2_moe_gather / int2_moe_combine
// (int2_moe/int2_moe_prefill.cl:29-70, :143-156) and the layer sequence of
// int2_moe/prefill.cpp:268-279:
//
//   route     meta[0..E] row offsets, meta[E+1..2E+1] row-tile offsets,
//             perm (sorted row -> assignment g = t * topk + j), inv = perm^-1
//   up        U = X[perm / topk] x B_up[e]                 (DT, POSTOP 0)
//   gate      Hs = silu(X[perm / topk] x B_gate[e]) * U    (DT, POSTOP 1)
//             (the layer runs the two as one launch, U kept in registers:
//             the same operations, bit for bit)
//   down      Y = Hs x B_down[e]                           (fp32)
//   combine   O[t, n] = DT(sum_j RW[g] * Y[inv[g], n]),  g = t * topk + j, j in order
//
// The route is a stable counting sort (rows of an expert in assignment order),
// so every run produces the same permutation: the reference's atomic-order
// permutation is not reproducible.  A workgroup per 1024 assignments, each
// counting all ids (the histogram) and those before its chunk, ranking lanes
// among equal expert ids with log2(E) ballots, and placing its chunk: no
// communication between workgroups.
// Assignments whose expert id is outside [0, E) are dropped: no row,
// inv = -1, no contribution to the combine.  The gather is not a separate pass
// in the layer: the grouped GEMM reads row perm[p] / topk of X directly.
#include "common.hpp"

#include <mutex>

namespace tcl {

int moe_tile_rows();  // int2_gemm_mfma.hip
ternocl_status moe_gemm_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                            const uint32_t *B_all, const void *S_all, void *C_all, const void *Other_all,
                            int E, int G, int N, int K, int postop, int out_f32, hipStream_t st,
                            const int4 *desc = nullptr);
ternocl_status moe_gate_up_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                               const uint32_t *Bu, const void *Su, const uint32_t *Bg, const void *Sg, void *Hs,
                               int E, int G, int N, int K, hipStream_t st, const int4 *desc = nullptr);

namespace {

constexpr int kRouteThreads = 1024, kRouteWaves = kRouteThreads / 64;
constexpr int kRoutePieces = 1;                                // 64-id pieces per wave of a chunk
constexpr int kRouteChunk = kRouteWaves * kRoutePieces * 64;   // ids ranked per pass of a workgroup (1024)
// Every workgroup counts all G ids, so the workgroups are capped: past
// 64 x 1024 ids a workgroup's chunk grows (whole passes of 1024) and the
// total work stays linear in G (at most 64 G counts and G ranks).
constexpr int kRouteMaxBlocks = 64;

// Sum over the 64 lanes of a wave (every lane gets it).
__device__ __forceinline__ int wave_sum(int v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// Lanes of a wave holding the same valid expert id as this lane (log2(E)
// ballots); invalid lanes get an empty set.
__device__ __forceinline__ unsigned long long route_group(bool valid, int e, int E) {
    unsigned long long same = __ballot(valid);
    for (int bit = 0; (1 << bit) < E; ++bit) {
        const bool on = (e >> bit) & 1;
        const unsigned long long bal = __ballot(valid && on);
        same &= on ? bal : ~bal;
    }
    return valid ? same : 0ull;
}

// Stable counting sort over ceil(G / chunk) workgroups, no communication
// between them: workgroup b places the ids of its chunk [b chunk, (b + 1)
// chunk), chunk a multiple of kRouteChunk.  It counts all ids (the histogram,
// hence each expert's first row) and those before its chunk (the expert's
// rows that precede the chunk) with LDS atomics (integer counts: order-free);
// then it ranks its chunk in passes of kRouteChunk ids, in order (passes in
// order, waves in order, pieces in order, lanes in order, lanes of one expert
// found with log2(E) ballots) and writes perm and inv.  Workgroup 0 writes
// meta.  Ids outside [0, E) are dropped (inv = -1), and perm past the kept
// rows is -1.  desc (the layer's tile list, or nullptr): workgroup 0 also
// lists the row tiles of rpt rows in expert order, each expert's last rows
// (its tail) sharing a tile with the next tail of at most rpt / 2 rows when
// its own has at most rpt / 2: desc[0].x = the tile count, desc[1 + t] =
// {row0 a, e_a << 8 | rows a, row0 b, e_b << 8 | rows b}, e_b = -1 alone.
__global__ void __launch_bounds__(kRouteThreads)
k_moe_route(const int *__restrict__ ids, int *__restrict__ meta, int *__restrict__ perm,
            int *__restrict__ inv, int G, int E, int rpt, int chunk, int4 *__restrict__ desc) {
    extern __shared__ int sh[];
    // counts of all ids tot [E] (first those from the chunk on) and of the
    // ids before the chunk bef [E], the
    // pass's per-wave counts / wave bases wc [W][E], each expert's first row
    // for this pass base [E]
    int *tot = sh, *bef = sh + E, *wc = sh + 2 * E, *base = sh + (2 + kRouteWaves) * E;
    __shared__ int s_rows;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const unsigned long long below = (1ull << lane) - 1ull;
    const int c0 = blockIdx.x * chunk, c1 = (int)min((long long)c0 + chunk, (long long)G);
    for (int i = tid; i < (2 + kRouteWaves) * E; i += kRouteThreads) sh[i] = 0;
    __syncthreads();

    // counts, sixteen ids' loads in flight per thread (G = 16384: one round)
    for (int i0 = tid; i0 < G; i0 += 16 * kRouteThreads) {
        int ev[16];
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int g = i0 + u * kRouteThreads;
            ev[u] = g < G ? ids[g] : -1;
        }
#pragma unroll
        for (int u = 0; u < 16; ++u) {
            const int g = i0 + u * kRouteThreads;
            if (ev[u] >= 0 && ev[u] < E) atomicAdd((g < c0 ? bef : tot) + ev[u], 1);  // before / from the chunk
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += kRouteThreads) tot[e] += bef[e];
    __syncthreads();
    if (wave == 0) {  // row and row-tile offsets: a 64-lane inclusive scan per 64 experts
        int r0 = 0, t0 = 0;
        for (int e0 = 0; e0 < E; e0 += 64) {
            const int e = e0 + lane;
            const int c = e < E ? tot[e] : 0, tl = (c + rpt - 1) / rpt;
            int r = c, t = tl;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const int ru = __shfl_up(r, o), tu = __shfl_up(t, o);
                if (lane >= o) { r += ru; t += tu; }
            }
            if (e < E) {
                base[e] = r0 + r - c + bef[e];
                if (blockIdx.x == 0) {
                    meta[e] = r0 + r - c;
                    meta[E + 1 + e] = t0 + t - tl;
                }
            }
            r0 += __shfl(r, 63);
            t0 += __shfl(t, 63);
        }
        if (lane == 0) {
            s_rows = r0;
            if (blockIdx.x == 0) {
                meta[E] = r0;
                meta[2 * E + 1] = t0;
            }
        }
        if (desc && blockIdx.x == 0) {
            // The tile list: first every expert's full tiles and its tail of
            // more than rpt / 2 rows, in expert order (a scan of the per-expert
            // counts), then the tails of at most rpt / 2 rows in pairs, in
            // expert order (the k-th such tail takes half k % 2 of pair k / 2;
            // an odd last one is alone).  Each half is one int2 store.
            const int hr = rpt / 2;
            int s_all = 0, m_all = 0;
            for (int e0 = 0; e0 < E; e0 += 64) {  // totals
                const int e = e0 + lane, c = e < E ? tot[e] : 0, tail = c % rpt;
                s_all += wave_sum(c / rpt + (tail > hr ? 1 : 0));
                m_all += wave_sum(tail > 0 && tail <= hr ? 1 : 0);
            }
            int2 *d2 = (int2 *)desc;
            int s_run = 0, m_run = 0, r_run = 0;
            for (int e0 = 0; e0 < E; e0 += 64) {
                const int e = e0 + lane, c = e < E ? tot[e] : 0, full = c / rpt, tail = c - full * rpt;
                const int f = full + (tail > hr ? 1 : 0), sm = tail > 0 && tail <= hr ? 1 : 0;
                int fi = f, si = sm, ri = c;  // inclusive scans over the 64 lanes
#pragma unroll
                for (int o = 1; o < 64; o <<= 1) {
                    const int fu = __shfl_up(fi, o), su = __shfl_up(si, o), ru = __shfl_up(ri, o);
                    if (lane >= o) { fi += fu; si += su; ri += ru; }
                }
                const int t0 = s_run + fi - f, rank = m_run + si - sm, row = r_run + ri - c;
                for (int i = 0; i < full; ++i) desc[1 + t0 + i] = make_int4(row + i * rpt, (e << 8) | rpt, 0, -1);
                if (tail > hr) desc[1 + t0 + full] = make_int4(row + full * rpt, (e << 8) | tail, 0, -1);
                if (sm) {
                    const int t = 1 + s_all + (rank >> 1);
                    d2[2 * t + (rank & 1)] = make_int2(row + full * rpt, (e << 8) | tail);
                    if ((rank & 1) == 0 && rank == m_all - 1) d2[2 * t + 1] = make_int2(0, -1);  // alone
                }
                s_run += __shfl(fi, 63);
                m_run += __shfl(si, 63);
                r_run += __shfl(ri, 63);
            }
            if (lane == 0) desc[0] = make_int4(s_all + (m_all + 1) / 2, 0, 0, 0);
        }
    }

    // rank the chunk, a pass of kRouteChunk ids at a time: wave w's ids
    // s0 + (w P + c) 64 + lane, pieces c in order
    int *mine = wc + wave * E;
    for (int s0 = c0; s0 < c1; s0 += kRouteChunk) {
        int eid[kRoutePieces], loc[kRoutePieces];
        const int seg = s0 + wave * kRoutePieces * 64;
#pragma unroll
        for (int c = 0; c < kRoutePieces; ++c) {
            const int g = seg + c * 64 + lane;
            eid[c] = g < c1 ? ids[g] : -1;
        }
#pragma unroll
        for (int c = 0; c < kRoutePieces; ++c) {
            const bool valid = eid[c] >= 0 && eid[c] < E;
            const int e = valid ? eid[c] : 0;
            const unsigned long long same = route_group(valid, e, E);
            const int before = valid ? mine[e] : 0;  // every lane reads before the leader writes
            loc[c] = before + __popcll(same & below);
            if (valid && (same & below) == 0ull) mine[e] = before + __popcll(same);
        }
        __syncthreads();
        for (int e = tid; e < E; e += kRouteThreads) {  // wave counts -> wave bases, in wave order
            int r = base[e];
            for (int w = 0; w < kRouteWaves; ++w) {
                const int n = wc[w * E + e];
                wc[w * E + e] = r;
                r += n;
            }
            base[e] = r;  // the next pass's first row of expert e
        }
        __syncthreads();
#pragma unroll
        for (int c = 0; c < kRoutePieces; ++c) {
            const int g = seg + c * 64 + lane;
            if (eid[c] >= 0 && eid[c] < E) {
                const int p = mine[eid[c]] + loc[c];
                perm[p] = g;
                inv[g] = p;
            } else if (g < c1) {
                inv[g] = -1;
            }
        }
        if (s0 + kRouteChunk < c1) {  // a next pass: its wave counts start from zero
            __syncthreads();
            for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) wc[i] = 0;
            __syncthreads();
        }
    }
    // perm past the kept rows: this workgroup's share of [rows, G)
    const int rows = s_rows;
    for (int i = c0 + tid; i < c1; i += kRouteThreads)
        if (i >= rows) perm[i] = -1;
}

// Xs[p] = X[perm[p] / topk] (rows of K DT), one workgroup per row; a row whose
// perm is negative (past the kept rows: the route writes -1 there) is zeroed
__global__ void __launch_bounds__(256)
k_moe_gather(const uint16_t *__restrict__ X, const int *__restrict__ perm, uint16_t *__restrict__ Xs,
             int K, int topk) {
    const int p = blockIdx.x;
    const int g = perm[p];
    uint16_t *dst = Xs + (size_t)p * K;
    if (g < 0) {
        for (int i = threadIdx.x; i < K; i += blockDim.x) dst[i] = 0;
        return;
    }
    const uint16_t *src = X + (size_t)(g / topk) * K;
    if ((K & 7) == 0) {
        for (int i = threadIdx.x; i < K / 8; i += blockDim.x) ((uint4 *)dst)[i] = ((const uint4 *)src)[i];
    } else {
        for (int i = threadIdx.x; i < K; i += blockDim.x) dst[i] = src[i];
    }
}

// O[t, n..n+3]: the topk weighted rows summed in j order, fp32 without
// contraction (each product rounded, then added), then one rounding to DT.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_moe_combine(const float *__restrict__ Y, const int *__restrict__ inv, const uint16_t *__restrict__ RW,
              uint16_t *__restrict__ O, int N, int topk) {
#pragma clang fp contract(off)
    const int t = blockIdx.y;
    const int n = 4 * (blockIdx.x * blockDim.x + threadIdx.x);
    if (n >= N) return;
    float s[4] = {0.f, 0.f, 0.f, 0.f};
    for (int j = 0; j < topk; ++j) {
        const int g = t * topk + j;
        const int row = inv ? inv[g] : g;  // no inv: Y in assignment order (the decode layer)
        if (row < 0) continue;  // a dropped assignment (expert id out of range)
        const float w = dt2f<BF16>(RW[g]);
        const float4 y = *(const float4 *)(Y + (size_t)row * N + n);
        s[0] += w * y.x;
        s[1] += w * y.y;
        s[2] += w * y.z;
        s[3] += w * y.w;
    }
    uint2 o;
    o.x = f2dt<BF16>(s[0]) | (f2dt<BF16>(s[1]) << 16);
    o.y = f2dt<BF16>(s[2]) | (f2dt<BF16>(s[3]) << 16);
    *(uint2 *)(O + (size_t)t * N + n) = o;
}

}  // namespace

// per-wave total, preceding and chunk counts, and each expert's base row
size_t moe_route_lds(int E) { return (size_t)(3 + kRouteWaves) * E * sizeof(int); }

ternocl_status moe_route_run(const int *ids, int *meta, int *perm, int *inv, int G, int E, hipStream_t st,
                             int4 *desc) {
    const int passes = (G + kRouteChunk - 1) / kRouteChunk;
    const int per = (passes + kRouteMaxBlocks - 1) / kRouteMaxBlocks;  // passes per workgroup
    const int chunk = per * kRouteChunk;
    const unsigned blocks = (unsigned)((G + chunk - 1) / chunk);
    hipLaunchKernelGGL(k_moe_route, dim3(blocks), dim3(kRouteThreads), moe_route_lds(E), st, ids, meta, perm, inv,
                       G, E, moe_tile_rows(), chunk, desc);
    return check_launch();
}

ternocl_status moe_gather_run(const void *X, const int *perm, void *Xs, int G, int K, int topk, hipStream_t st) {
    hipLaunchKernelGGL(k_moe_gather, dim3(G), dim3(256), 0, st, (const uint16_t *)X, perm, (uint16_t *)Xs, K, topk);
    return check_launch();
}

ternocl_status moe_combine_run(int dtype, const float *Y, const int *inv, const void *RW, void *O, int T,
                               int topk, int N, hipStream_t st) {
    const dim3 grid((unsigned)((N / 4 + 255) / 256), (unsigned)T), block(256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_moe_combine<true>, grid, block, 0, st, Y, inv, (const uint16_t *)RW, (uint16_t *)O, N, topk);
    else
        hipLaunchKernelGGL(k_moe_combine<false>, grid, block, 0, st, Y, inv, (const uint16_t *)RW, (uint16_t *)O, N, topk);
    return check_launch();
}

// Workspace of the layer: the header (counters of other entries sharing the
// workspace; untouched), then meta | perm | inv | Hs | Y, each 256-byte aligned.
MoeWs moe_ws_layout(int T, int E, int topk, int H, int I) {
    const size_t G = (size_t)T * topk;
    MoeWs w;
    size_t o = kWsHeader;
    w.meta = o; o = align_up(o + (size_t)(2 * E + 2) * 4, 256);
    w.desc = o; o = align_up(o + (size_t)(1 + (G + moe_tile_rows() - 1) / moe_tile_rows() + E) * 16, 256);
    w.perm = o; o = align_up(o + G * 4, 256);
    w.inv = o;  o = align_up(o + G * 4, 256);
    w.h = o;    o = align_up(o + G * I * 2, 256);
    w.y = o;    o = align_up(o + G * H * 4, 256);
    w.total = o;
    return w;
}

ternocl_status moe_prefill_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                               int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                               const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                               void *O, void *ws, hipStream_t st) {
    const MoeWs w = moe_ws_layout(T, E, topk, H, I);
    char *b = (char *)ws;
    int *meta = (int *)(b + w.meta), *perm = (int *)(b + w.perm), *inv = (int *)(b + w.inv);
    int4 *desc = (int4 *)(b + w.desc);
    void *Hs = b + w.h;
    float *Y = (float *)(b + w.y);
    const int G = T * topk;
    ternocl_status s;
    // the route lists the row tiles (two experts' short tails share one)
    if ((s = moe_route_run(ids, meta, perm, inv, G, E, st, desc)) != TERNOCL_OK) return s;
    // up and gate in one pass over the gathered rows (U never leaves the registers)
    if ((s = moe_gate_up_run(dtype, meta, X, perm, topk, Bu, Su, Bg, Sg, Hs, E, G, I, H, st, desc)) != TERNOCL_OK)
        return s;
    if ((s = moe_gemm_run(dtype, meta, Hs, nullptr, 1, Bd, Sd, Y, nullptr, E, G, H, I, 0, 1, st, desc)) != TERNOCL_OK)
        return s;
    return moe_combine_run(dtype, Y, inv, RW, O, T, topk, H, st);
}

// ---- int8 MoE prefill layer (int2_moe/int2_moe_prefill_int8.cl, QMODE 1; the sequence of
// int2_moe/prefill.cpp:243-279 with --int8 1) ----
// (int2_int8.hip)
ternocl_status quant_a_run(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K, hipStream_t st,
                           const int *perm = nullptr, int topk = 1, const int *nrows = nullptr);
ternocl_status int8_moe_gemm_run(int dtype, const int *meta, const int8_t *Aq, const void *SA, const uint32_t *B,
                                 const void *SB, void *C, const void *Other, int E, int G, int N, int K, int postop,
                                 int out_f32, hipStream_t st, const int *perm = nullptr, int topk = 1,
                                 int arows = 0);
ternocl_status int8_moe_dual_run(int dtype, const int *meta, const int8_t *Aq, const void *SA,
                                 const uint32_t *Bu, const void *Su, const uint32_t *Bg, const void *Sg, void *Hs,
                                 int E, int G, int N, int K, hipStream_t st, const int *perm, int topk, int arows);

// Workspace: meta | perm | inv | SA1 [H/128][ldsa(T)] | Hs DT [G][I] |
// SA2 [I/128][ldsa(G)] | Y fp32 [G][H] | Xq int8 [T][H] | Hq int8 [G][I], each
// 256-byte aligned.
MoeI8Ws moe_i8_ws_layout(int T, int E, int topk, int H, int I) {
    const size_t G = (size_t)T * topk, lda = ((size_t)G + 31) & ~(size_t)31, ldt = ((size_t)T + 31) & ~(size_t)31;
    MoeI8Ws w;
    size_t o = kWsHeader;
    w.meta = o; o = align_up(o + (size_t)(2 * E + 2) * 4, 256);
    w.perm = o; o = align_up(o + G * 4, 256);
    w.inv = o;  o = align_up(o + G * 4, 256);
    w.sa1 = o;  o = align_up(o + (size_t)(H / 128) * ldt * 2, 256);
    w.h = o;    o = align_up(o + G * I * 2, 256);
    w.sa2 = o;  o = align_up(o + (size_t)(I / 128) * lda * 2, 256);
    w.y = o;    o = align_up(o + G * H * 4, 256);
    w.xq = o;   o = align_up(o + (size_t)T * H, 256);
    w.hq = o;   o = align_up(o + G * I, 256);
    w.total = o;
    return w;
}

// route; quant_a of the T token rows (SA1, Xq: each token quantized once, the
// reference's quant_x); up = s8 x s2 (POSTOP 0) and h = silu(gate) * up (POSTOP 1,
// Other = up) in one launch, gathering the A rows from Xq through perm (the
// reference's gather_q, fused into the A loads); quant_a of h (SA2, Hq); Y =
// s8 x s2 down (fp32); combine.  The int8 values are quant_a's of each row,
// wherever it is quantized: the reference's QMODE 0 and QMODE 1 give the same.
ternocl_status moe_prefill_int8_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                                    int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                    const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                                    void *O, void *ws, hipStream_t st) {
    const MoeI8Ws w = moe_i8_ws_layout(T, E, topk, H, I);
    char *b = (char *)ws;
    int *meta = (int *)(b + w.meta), *perm = (int *)(b + w.perm), *inv = (int *)(b + w.inv);
    void *SA1 = b + w.sa1, *Hs = b + w.h, *SA2 = b + w.sa2;
    float *Y = (float *)(b + w.y);
    int8_t *Xq = (int8_t *)(b + w.xq), *Hq = (int8_t *)(b + w.hq);
    const int G = T * topk;
    ternocl_status s;
    if ((s = moe_route_run(ids, meta, perm, inv, G, E, st, nullptr)) != TERNOCL_OK) return s;
    if ((s = quant_a_run(dtype, X, SA1, Xq, T, H, st)) != TERNOCL_OK) return s;
    // up and gate in one pass over the gathered int8 rows (U never leaves the registers)
    if ((s = int8_moe_dual_run(dtype, meta, Xq, SA1, Bu, Su, Bg, Sg, Hs, E, G, I, H, st, perm, topk, T)) !=
        TERNOCL_OK)
        return s;
    if ((s = quant_a_run(dtype, Hs, SA2, Hq, G, I, st, nullptr, 1, meta + E)) != TERNOCL_OK) return s;
    if ((s = int8_moe_gemm_run(dtype, meta, Hq, SA2, Bd, Sd, Y, nullptr, E, G, H, I, 0, 1, st)) != TERNOCL_OK)
        return s;
    return moe_combine_run(dtype, Y, inv, RW, O, T, topk, H, st);
}

// ---- MoE decode layer (int2_moe/int2_moe.cl, the sequence of int2_moe/main.cpp:226-261) ----
// (int2_gemv_f4.hip)
ternocl_status int2_gemv_f4_group_run(int dtype, const void *A, const int *ids, int G, int E, int topk,
                                      const uint32_t *B, const void *S, const uint32_t *B2, const void *S2,
                                      float *C, int N, int K, const void *RW, void *O, int mode,
                                      hipStream_t st);

// Workspace: the header (untouched), then gate/up fp32 [2G][I] | Y fp32 [G][H]
// (used when topk > 16), each 256-byte aligned.
size_t moe_decode_ws_bytes(int T, int topk, int H, int I) {
    const size_t G = (size_t)T * topk;
    return kWsHeader + align_up(2 * G * I * 4, 256) + align_up(G * H * 4, 256);
}

// (1) One grouped GEMV over 2G rows: gate and up of every pair, fp32.
// (2) topk <= 16: one launch per (column strip, token), a wave per slot: down
//     of h = DT(silu(gate) * up) (formed while staging), then
//     O[t] = DT(sum_j RW[g] * y_g) in slot order (the reference's down_sum);
//     topk > 16: the down GEMV into Y (fp32) and the weighted-sum kernel.
ternocl_status moe_decode_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                              int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                              const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                              void *O, void *ws, hipStream_t st) {
    const int G = T * topk;
    uint8_t *b = (uint8_t *)ws + kWsHeader;
    float *GU = (float *)b;
    float *Y = (float *)(b + align_up((size_t)2 * G * I * 4, 256));
    ternocl_status s;
    if ((s = int2_gemv_f4_group_run(dtype, X, ids, G, E, topk, Bg, Sg, Bu, Su, GU, I, H, nullptr, nullptr, 0,
                                    st)) != TERNOCL_OK)
        return s;
    if (topk <= 16)
        return int2_gemv_f4_group_run(dtype, GU, ids, G, E, topk, Bd, Sd, nullptr, nullptr, nullptr, H, I, RW, O,
                                      2, st);
    if ((s = int2_gemv_f4_group_run(dtype, GU, ids, G, E, topk, Bd, Sd, nullptr, nullptr, Y, H, I, nullptr,
                                    nullptr, 1, st)) != TERNOCL_OK)
        return s;
    return moe_combine_run(dtype, Y, nullptr, RW, O, T, topk, H, st);
}

// ---- the MoE decode layer without a caller workspace ----
// For callers that cannot allocate (code under HIP graph capture, serving
// loops): the layer's scratch -- the fp32 gate/up rows and, for topk > 16, the
// fp32 down rows, the same layout as the workspace of moe_decode_run -- lives in
// one fixed array per device, held until the process ends.  Every call on a
// device shares that device's array: calls that overlap on one device race.
// Nothing in it has to start at zero (every row the layer reads back it has
// written in the same call), so it is never cleared.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxDevices];  // device address of scratch on each device (looked up once)
}  // namespace

ternocl_status moe_decode_noalloc_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                                      int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                      const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                                      void *O, hipStream_t st) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return launch_status(e);
    if (dev < 0 || dev >= kMaxDevices) {
        set_error("device ordinal beyond the 64 devices the scratch table holds");
        return TERNOCL_ERR_INVALID_ARG;
    }
    void *ptr;
    {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        if (!g_scratch_ptr[dev]) {
            // the host-side name of scratch is not a device address: kernels get
            // the address the runtime reports for this device
            void *p = nullptr;
            e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess) return launch_status(e);
            if (!p) {
                set_error("hipGetSymbolAddress returned no address for the scratch array");
                return TERNOCL_ERR_LAUNCH;
            }
            g_scratch_ptr[dev] = p;
        }
        ptr = g_scratch_ptr[dev];
    }
    return moe_decode_run(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ptr, st);
}

}  // namespace tcl
