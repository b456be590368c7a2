// int2_gemm_mfma.hip -- prefill GEMM (M > 16) for packed 2-bit ternary weights
// on gfx950: the MI355X replacement of int2_fp16_upcvt_gemm_mt
// (int2_fp16_upcvt/int2_fp16_upcvt.cl:292-395), and the tile engine of the MoE
// prefill (int2_moe/int2_moe_prefill.cl:72-141).
//
//   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(B[k,n])))
//
// Tiling: a workgroup of 4 waves computes a 128 x 128 tile of C; each wave a
// 64 x 64 quarter as 4 x 4 v_mfma_f32_16x16x32_{f16,bf16} tiles.  K advances
// one 128-row scale group at a time (4 MFMA k-steps of 32).
//   * A (DT, row-major) goes global -> registers -> LDS once per workgroup and
//     group, each 16-element chunk stored in the order 0,8,1,9,...,7,15, so the
//     MFMA A fragment of lane (row, q) -- pairs (4h+i, 4h+i+8) of one chunk --
//     is one 16-byte LDS read;
//   * B is never expanded in memory: each wave loads the packed words of its 64
//     columns (L2-resident across the M tiles) and decodes the MFMA B fragment
//     in registers: for the pair of rows (j, j+8) of a word,
//     (w << (14 - 2j)) & 0xC000C000 is exactly +-2.0 / 0 in fp16 and in bf16
//     (the code's low bit lands on the exponent LSB, its high bit on the sign),
//     two VALU ops per pair, no tables;
//   * each group accumulates in its own fp32 MFMA accumulators (the chain for
//     k-step 0 starts from zero), then one FMA per output element applies the
//     group scale: acc += acc_g * (S[g,n] / 2);
//   * workgroup -> tile mapping keeps the M tiles of one column strip on one
//     XCD, so a strip's packed weights are fetched into that XCD's L2 once.
#include "common.hpp"

namespace tcl {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int BM = 128, BN = 128, BK = 128;
constexpr int A_PITCH = BK + 8;  // DT elements per LDS row (16 bytes of padding)

template <bool BF16>
__device__ __forceinline__ f32x4_t mfma16(const uint32_t a[4], const uint32_t b[4], f32x4_t c) {
    if constexpr (BF16) {
        bf168_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c, 0, 0, 0);
    } else {
        half8_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c, 0, 0, 0);
    }
}

// B fragment of half h of word w: dword i = rows (4h+i, 4h+i+8) as +-2.0 / 0.
__device__ __forceinline__ void pm2_fragment(uint32_t w, int h, uint32_t b[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int j = 4 * h + i;
        b[i] = (w << (14 - 2 * j)) & 0xC000C000u;
    }
}

// Interleave a 16-element chunk (v[0..3] = elements 0..7, v[4..7] = 8..15) into
// 0,8,1,9,...,7,15.
__device__ __forceinline__ void chunk_interleave(const uint32_t v[8], uint32_t o[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = v[i >> 1], hi = v[4 + (i >> 1)];
        o[i] = __builtin_amdgcn_perm(hi, lo, (i & 1) ? 0x07060302u : 0x05040100u);
    }
}

// Row source of the A tile: a plain row-major [M, K] matrix, or rows gathered
// through an index (the MoE path reads token rows of X through perm).
struct ARows {
    const uint16_t *A;
    const int *idx;  // nullptr: row r is A + r * K; else A + (idx[r] / div) * K
    int div;
    __device__ __forceinline__ const uint16_t *row(int r, int K) const {
        return A + (size_t)(idx ? idx[r] / div : r) * K;
    }
};

// One 128 x 128 output tile of rows [m0, m0 + mrows) (mrows <= 128 valid) and
// columns [n0, n0 + 128) (N % 16 == 0; columns >= N masked).
template <bool BF16>
__device__ __forceinline__ void gemm_tile(const ARows &ar, int mrows, const uint32_t *__restrict__ B,
                                          const uint16_t *__restrict__ S, void *__restrict__ C,
                                          const uint16_t *__restrict__ Other, const void *__restrict__ Bias,
                                          int ldc_rows_base, int N, int K, int n0, int postop,
                                          int out_f32, uint16_t *lds) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, q = lane >> 4;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;  // this wave's quarter
    const int groups = K / kGS;

    // A staging: thread tid owns rows (tid >> 3) + 32 * u (u = 0..3) and the
    // 16-element chunk (tid & 7) of the group: 4 x 32 bytes per group.
    const int arow0 = tid >> 3, achunk = tid & 7;
    uint4 av[4][2];
    auto a_load = [&](int g) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = arow0 + 32 * u;
            const int rc = r < mrows ? r : mrows - 1;
            const uint4 *p = (const uint4 *)(ar.row(rc, K) + (size_t)g * kGS + 16 * achunk);
            av[u][0] = p[0];
            av[u][1] = p[1];
            if (r >= mrows) av[u][0] = av[u][1] = make_uint4(0, 0, 0, 0);
        }
    };
    auto a_store = [&](uint16_t *buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const uint32_t v[8] = {av[u][0].x, av[u][0].y, av[u][0].z, av[u][0].w,
                                   av[u][1].x, av[u][1].y, av[u][1].z, av[u][1].w};
            uint32_t o[8];
            chunk_interleave(v, o);
            uint4 *d = (uint4 *)(buf + (size_t)(arow0 + 32 * u) * A_PITCH + 16 * achunk);
            d[0] = make_uint4(o[0], o[1], o[2], o[3]);
            d[1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    };

    // B words of this wave for group g: column block cb, k-step ks -> word
    // (kp = 8g + 2ks + q/2, column n0 + wn + 16cb + c16); half q % 2.
    uint32_t bw[4][4];
    uint32_t sc[4];
    auto b_load = [&](int g) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            int n = n0 + wn + 16 * cb + c16;
            n = n < N ? n : N - 1;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) bw[cb][ks] = B[((size_t)g * 8 + 2 * ks + (q >> 1)) * N + n];
            sc[cb] = S[(size_t)g * N + n];
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    a_load(0);
    b_load(0);
    a_store(lds);
    for (int g = 0; g < groups; ++g) {
        __syncthreads();  // A tile g staged, tile g-1 consumed
        const uint16_t *abuf = lds + (size_t)(g & 1) * BM * A_PITCH;
        uint32_t bwc[4][4], scc[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            scc[cb] = sc[cb];
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) bwc[cb][ks] = bw[cb][ks];
        }
        const bool more = g + 1 < groups;
        if (more) {  // next group's loads in flight during this group's MFMAs
            a_load(g + 1);
            b_load(g + 1);
        }
        f32x4_t accg[4][4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            uint32_t af[4][4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const uint4 v = *(const uint4 *)(abuf + (size_t)(wm + 16 * mb + c16) * A_PITCH +
                                                 (2 * ks + (q >> 1)) * 16 + 8 * (q & 1));
                af[mb][0] = v.x; af[mb][1] = v.y; af[mb][2] = v.z; af[mb][3] = v.w;
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                uint32_t bf[4];
                pm2_fragment(bwc[cb][ks], q & 1, bf);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    accg[mb][cb] = mfma16<BF16>(af[mb], bf, ks == 0 ? f32x4_t{0.f, 0.f, 0.f, 0.f} : accg[mb][cb]);
            }
        }
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            const float s = 0.5f * dt2f<BF16>(scc[cb]);
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) acc[mb][cb] = accg[mb][cb] * s + acc[mb][cb];
        }
        if (more) a_store(lds + (size_t)((g + 1) & 1) * BM * A_PITCH);
    }

    // lane holds rows wm + 16mb + 4q + i of column wn + 16cb + c16
#pragma unroll
    for (int cb = 0; cb < 4; ++cb) {
        const int n = n0 + wn + 16 * cb + c16;
        if (n >= N) continue;
#pragma unroll
        for (int mb = 0; mb < 4; ++mb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = wm + 16 * mb + 4 * q + i;
                if (r < mrows)
                    epi_store1<BF16>(C, Other, Bias, postop, out_f32, N, ldc_rows_base + r, n, acc[mb][cb][i]);
            }
    }
}

template <bool BF16>
__global__ void __launch_bounds__(256)
k_int2_gemm(const uint16_t *__restrict__ A, const uint32_t *__restrict__ B,
            const uint16_t *__restrict__ S, void *__restrict__ C, const uint16_t *__restrict__ Other,
            const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * BM * A_PITCH];  // 68 KiB
    const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    int tm, tn;
    xcd_tile_of(blockIdx.x, mt, nt, tm, tn);
    const ARows ar{A + (size_t)tm * BM * K, nullptr, 1};
    const int mrows = min(BM, M - tm * BM);
    gemm_tile<BF16>(ar, mrows, B, S, C, Other, Bias, tm * BM, N, K, tn * BN, postop, out_f32, lds);
}

// Grouped GEMM of the MoE prefill (int2_moe/int2_moe_prefill.cl:72-141): the
// rows of each expert e are meta[e] .. meta[e+1]-1 of the expert-sorted order,
// cut into 128-row tiles numbered from meta[E+1+e]; workgroup (tile, column
// block) finds its expert by binary search over the tile offsets.  A rows come
// from A_all[perm[p] / topk] when perm is given (the gather fused into the
// A-tile load), else from A_all[p].  Expert e's weights: B_all + e*(K/16)*N,
// S_all + e*(K/128)*N; C and Other are indexed by the sorted row p.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_int2_moe_gemm(const int *__restrict__ meta, const uint16_t *__restrict__ A_all,
                const int *__restrict__ perm, int topk, const uint32_t *__restrict__ B_all,
                const uint16_t *__restrict__ S_all, void *__restrict__ C_all,
                const uint16_t *__restrict__ Other_all, int E, int N, int K, int postop, int out_f32,
                int ntn) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * BM * A_PITCH];
    const int tile = blockIdx.x / ntn, tn = blockIdx.x - tile * ntn;
    if (tile >= meta[2 * E + 1]) return;  // whole workgroup: past the last row tile
    int lo = 0, hi = E - 1;
    while (lo < hi) {  // the last expert whose first tile is <= tile
        const int mid = (lo + hi + 1) >> 1;
        if (meta[E + 1 + mid] <= tile) lo = mid;
        else hi = mid - 1;
    }
    const int e = lo, row0 = meta[e];
    const int m0 = (tile - meta[E + 1 + e]) * BM;
    const int mrows = min(BM, meta[e + 1] - row0 - m0);
    const ARows ar = perm ? ARows{A_all, perm + row0 + m0, topk}
                          : ARows{A_all + (size_t)(row0 + m0) * K, nullptr, 1};
    gemm_tile<BF16>(ar, mrows, B_all + (size_t)e * (K / 16) * N, S_all + (size_t)e * (K / kGS) * N, C_all,
                    Other_all, nullptr, row0 + m0, N, K, tn * BN, postop, out_f32, lds);
}

// Test hook: the B fragments the GEMM builds, D[word][0..3] = half 0,
// D[word][4..7] = half 1 (the same bits for fp16 and bf16).
__global__ void k_int2_gemm_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D, int words) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    uint32_t b[8];
    pm2_fragment(B[i], 0, b);
    pm2_fragment(B[i], 1, b + 4);
    uint4 *d = (uint4 *)(D + (size_t)i * 8);
    d[0] = make_uint4(b[0], b[1], b[2], b[3]);
    d[1] = make_uint4(b[4], b[5], b[6], b[7]);
}

}  // namespace

int moe_tile_rows() { return BM; }

ternocl_status moe_gemm_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                            const uint32_t *B_all, const void *S_all, void *C_all, const void *Other_all,
                            int E, int G, int N, int K, int postop, int out_f32, hipStream_t st) {
    const int ntn = (N + BN - 1) / BN;
    const int max_tiles = (G + BM - 1) / BM + E;  // each expert's ragged tail adds at most one tile
    const dim3 grid((unsigned)(max_tiles * ntn)), block(256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_moe_gemm<true>, grid, block, 0, st, meta, (const uint16_t *)A_all, perm, topk,
                           B_all, (const uint16_t *)S_all, C_all, (const uint16_t *)Other_all, E, N, K, postop,
                           out_f32, ntn);
    else
        hipLaunchKernelGGL(k_int2_moe_gemm<false>, grid, block, 0, st, meta, (const uint16_t *)A_all, perm, topk,
                           B_all, (const uint16_t *)S_all, C_all, (const uint16_t *)Other_all, E, N, K, postop,
                           out_f32, ntn);
    return check_launch();
}

ternocl_status int2_gemm_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st) {
    const int words = K / 16 * N;
    hipLaunchKernelGGL(k_int2_gemm_decode, dim3((words + 255) / 256), dim3(256), 0, st, B, D, words);
    return check_launch();
}

ternocl_status int2_gemm_mfma_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K,
                                  int postop, int out_f32, hipStream_t st) {
    const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    const dim3 grid(mt * nt), block(256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_gemm<true>, grid, block, 0, st, (const uint16_t *)A, B,
                           (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    else
        hipLaunchKernelGGL(k_int2_gemm<false>, grid, block, 0, st, (const uint16_t *)A, B,
                           (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    return check_launch();
}

}  // namespace tcl
