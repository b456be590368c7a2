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
//   down      Y = Hs x B_down[e]                           (fp32)
//   combine   O[t, n] = DT(sum_j RW[g] * Y[inv[g], n]),  g = t * topk + j, j in order
//
// The route is a stable counting sort (rows of an expert in assignment order),
// so every run produces the same permutation: the reference's atomic-order
// permutation is not reproducible.  One workgroup: a histogram (LDS atomics,
// order-free), the offsets, then chunks of 1024 assignments in order where each
// wave ranks its lanes among equal expert ids with log2(E) ballots, the waves'
// per-expert counts are prefix-summed in wave order, and every assignment gets
// its slot.  Assignments whose expert id is outside [0, E) are dropped: no row,
// inv = -1, no contribution to the combine.  The gather is not a separate pass
// in the layer: the grouped GEMM reads row perm[p] / topk of X directly.
#include "common.hpp"

namespace tcl {

int moe_tile_rows();  // int2_gemm_mfma.hip
ternocl_status moe_gemm_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                            const uint32_t *B_all, const void *S_all, void *C_all, const void *Other_all,
                            int E, int G, int N, int K, int postop, int out_f32, hipStream_t st);

namespace {

constexpr int kRouteThreads = 1024, kRouteWaves = kRouteThreads / 64;

__global__ void __launch_bounds__(kRouteThreads)
k_moe_route(const int *__restrict__ ids, int *__restrict__ meta, int *__restrict__ perm,
            int *__restrict__ inv, int G, int E, int rpt) {
    extern __shared__ int sh[];
    int *cnt = sh, *base = sh + E, *wcnt = sh + 2 * E;  // wcnt [kRouteWaves][E]
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    for (int e = tid; e < E; e += kRouteThreads) cnt[e] = 0;
    __syncthreads();
    for (int g = tid; g < G; g += kRouteThreads) {
        const int e = ids[g];
        if (e >= 0 && e < E) atomicAdd(&cnt[e], 1);
    }
    __syncthreads();
    if (tid == 0) {
        int r = 0, t = 0;
        for (int e = 0; e < E; ++e) {
            meta[e] = r;
            meta[E + 1 + e] = t;
            base[e] = r;
            r += cnt[e];
            t += (cnt[e] + rpt - 1) / rpt;
        }
        meta[E] = r;
        meta[2 * E + 1] = t;
    }
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int c0 = 0; c0 < G; c0 += kRouteThreads) {
        for (int i = tid; i < kRouteWaves * E; i += kRouteThreads) wcnt[i] = 0;
        __syncthreads();  // also orders base[] after the offsets on the first chunk
        const int g = c0 + tid;
        const int eg = g < G ? ids[g] : -1;
        const bool valid = eg >= 0 && eg < E;  // out-of-range ids are dropped
        const int e = valid ? eg : 0;
        unsigned long long same = __ballot(valid);
        for (int b = 0; (1 << b) < E; ++b) {
            const bool bit = (e >> b) & 1;
            const unsigned long long bal = __ballot(valid && bit);
            same &= bit ? bal : ~bal;
        }
        const int rank = __popcll(same & below);
        if (valid && rank == 0) wcnt[wave * E + e] = __popcll(same);
        __syncthreads();
        for (int x = tid; x < E; x += kRouteThreads) {
            int run = base[x];
            for (int w = 0; w < kRouteWaves; ++w) {
                const int c = wcnt[w * E + x];
                wcnt[w * E + x] = run;
                run += c;
            }
            base[x] = run;
        }
        __syncthreads();
        if (valid) {
            const int p = wcnt[wave * E + e] + rank;
            perm[p] = g;
            inv[g] = p;
        } else if (g < G) {
            inv[g] = -1;
        }
        __syncthreads();  // wcnt is cleared for the next chunk
    }
}

// Xs[p] = X[perm[p] / topk] (rows of K DT), one workgroup per row
__global__ void __launch_bounds__(256)
k_moe_gather(const uint16_t *__restrict__ X, const int *__restrict__ perm, uint16_t *__restrict__ Xs,
             int K, int topk) {
    const int p = blockIdx.x;
    const uint16_t *src = X + (size_t)(perm[p] / topk) * K;
    uint16_t *dst = Xs + (size_t)p * K;
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
        if (inv[g] < 0) continue;  // a dropped assignment (expert id out of range)
        const float w = dt2f<BF16>(RW[g]);
        const float4 y = *(const float4 *)(Y + (size_t)inv[g] * N + n);
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

size_t moe_route_lds(int E) { return (size_t)(2 + kRouteWaves) * E * sizeof(int); }

ternocl_status moe_route_run(const int *ids, int *meta, int *perm, int *inv, int G, int E, hipStream_t st) {
    hipLaunchKernelGGL(k_moe_route, dim3(1), dim3(kRouteThreads), moe_route_lds(E), st, ids, meta, perm, inv,
                       G, E, moe_tile_rows());
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

// Workspace of the layer: meta | perm | inv | U | Hs | Y, each 256-byte aligned.
struct MoeWs {
    size_t meta, perm, inv, u, h, y, total;
};
MoeWs moe_ws_layout(int T, int E, int topk, int H, int I) {
    const size_t G = (size_t)T * topk;
    MoeWs w;
    size_t o = 0;
    w.meta = o; o = align_up(o + (size_t)(2 * E + 2) * 4, 256);
    w.perm = o; o = align_up(o + G * 4, 256);
    w.inv = o;  o = align_up(o + G * 4, 256);
    w.u = o;    o = align_up(o + G * I * 2, 256);
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
    void *U = b + w.u, *Hs = b + w.h;
    float *Y = (float *)(b + w.y);
    const int G = T * topk;
    ternocl_status s;
    if ((s = moe_route_run(ids, meta, perm, inv, G, E, st)) != TERNOCL_OK) return s;
    if ((s = moe_gemm_run(dtype, meta, X, perm, topk, Bu, Su, U, nullptr, E, G, I, H, 0, 0, st)) != TERNOCL_OK) return s;
    if ((s = moe_gemm_run(dtype, meta, X, perm, topk, Bg, Sg, Hs, U, E, G, I, H, 1, 0, st)) != TERNOCL_OK) return s;
    if ((s = moe_gemm_run(dtype, meta, Hs, nullptr, 1, Bd, Sd, Y, nullptr, E, G, H, I, 0, 1, st)) != TERNOCL_OK) return s;
    return moe_combine_run(dtype, Y, inv, RW, O, T, topk, H, st);
}

}  // namespace tcl
