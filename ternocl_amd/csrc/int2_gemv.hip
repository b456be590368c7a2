// int2_gemv.hip -- decode GEMV (M <= 8) for packed 2-bit ternary weights on
// gfx950: the MI355X replacement of int2_fp16_upcvt_gemm
// (int2_fp16_upcvt/int2_fp16_upcvt.cl:193-290).
//
//   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(B[k,n])))
//
// Bandwidth design (the packed weights are >93% of the bytes, read once):
//   * a workgroup owns 4*LC adjacent columns over the whole of K, so workgroups
//     never communicate (no split-K partials, fences or atomics: a device-scope
//     release fence writes back the XCD's L2 and serialises across workgroups);
//   * lane l of a wave owns the 4 columns of quad (l % LC) and "k-slot" l / LC;
//     the W waves x 64/LC k-slots of the workgroup take 128-row groups
//     round-robin, so each lane streams the 8 B-row words of its groups with
//     16-byte loads (a wave reads 64/LC row segments of 16*LC contiguous bytes)
//     and issues the next round's loads before decoding the current one;
//   * weights are unpacked in registers by the mantissa-field decode of
//     int2_decode.hpp (9-11 VALU ops per 16 weights) and multiplied with
//     v_dot2_f32_{f16,bf16} (2 MACs per op, fp32 accumulate), no MFMA;
//   * activations are pre-scaled, pair-interleaved and staged in LDS once per
//     round of groups; one ds_read_b128 gives 4 pairs and serves the lane's 4
//     words (reading them per word would make LDS, not HBM, the bound), with one
//     correction term per (row, group) computed in the same prologue;
//   * reduction: k-slots of a wave by cross-lane adds, then waves through LDS in
//     wave order -- a fixed order, so results are deterministic bit for bit.
#include "common.hpp"
#include "int2_decode.hpp"

namespace tcl {
namespace {

// LDS layout of one round buffer: for each row m and round-local group q,
// 64 packed activation pairs plus 4 dwords of padding (keeps the k-slots of a
// wave, which read different groups, on different banks); then beta[m][q].
constexpr int kGroupStride = 68;  // dwords per (m, group) of pairs

__host__ __device__ inline size_t gemv_round_dwords(int MR, int ksl) {
    // rounded up to 4 dwords: the second buffer stays 16-byte aligned
    return ((size_t)MR * ksl * kGroupStride + (size_t)MR * ksl + 3) & ~(size_t)3;
}

// Stage the activation pairs (row j, row j+8) of groups [g0, g0+ksl) scaled by
// 2^-p_j, and beta = BASE * sum a' + 2 * sum a per (row, group).  The 64 pairs
// of one (row, group) are one wavefront iteration: beta is a cross-lane sum.
template <int MR, bool BF16>
__device__ __forceinline__ void stage_round(uint32_t *buf, const uint16_t *__restrict__ A, int M,
                                            int K, int groups, int g0, int ksl) {
    constexpr float BASE = gemv_base(BF16);
    uint32_t *pairs = buf;
    float *beta = (float *)(buf + (size_t)MR * ksl * kGroupStride);
    const int total = MR * ksl * 64;
    const int lane = threadIdx.x & 63;
    for (int idx0 = 0; idx0 < total; idx0 += blockDim.x) {
        const int idx = idx0 + threadIdx.x;
        const int mq = idx >> 6, q = idx & 63;  // (m, round-local group), pair index
        const int m = mq / ksl, gl = mq - m * ksl;
        const int g = g0 + gl;
        const int r = q >> 3, j = q & 7;
        uint32_t v = 0;
        float contrib = 0.0f;
        if (idx < total && m < M && g < groups) {
            const size_t k = (size_t)m * K + (size_t)g * kGS + r * 16 + j;
            const float sc = 1.0f / (float)(1 << gemv_pair_shift(BF16, j));
            const float alo = dt2f<BF16>(A[k]), ahi = dt2f<BF16>(A[k + 8]);
            const uint32_t plo = f2dt<BF16>(alo * sc), phi = f2dt<BF16>(ahi * sc);
            v = plo | (phi << 16);
            contrib = BASE * (dt2f<BF16>(plo) + dt2f<BF16>(phi)) + 2.0f * (alo + ahi);
        }
        if (idx < total) pairs[(size_t)mq * kGroupStride + q] = v;
#pragma unroll
        for (int o = 32; o >= 1; o >>= 1) contrib += __shfl_xor(contrib, o);
        if (lane == 0 && idx < total) beta[mq] = contrib;
    }
}

// One workgroup: 4*LC columns over all of K.  W = blockDim.x / 64 waves.  Lane
// (kl, cl) of a wave owns the 4 adjacent columns n0 = 4 * (strip * LC + cl) and
// k-slot kl; one LDS activation read serves the 4 words of a row.
// Up to 16 waves for one row (<= 128 VGPRs); up to 8 for MR >= 2, whose
// accumulators and activation pairs need more registers.
__host__ __device__ constexpr int gemv_max_waves(int MR) { return MR == 1 ? 16 : 8; }

template <int MR, int LC, bool BF16>
__global__ void __launch_bounds__(64 * gemv_max_waves(MR))
k_int2_gemv(const uint16_t *__restrict__ A, const uint4 *__restrict__ B4,
            const uint2 *__restrict__ S4, void *__restrict__ C, const uint16_t *__restrict__ Other,
            const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32, int swz) {
    extern __shared__ uint32_t lds[];
    constexpr int LK = 64 / LC;               // k-slots per wave
    const int W = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int kl = lane / LC, cl = lane % LC;
    const int slot = wave * LK + kl;           // this lane's k-slot
    const int ksl = W * LK;                    // groups per round
    const int groups = K / kGS;
    const int rounds = (groups + ksl - 1) / ksl;
    const int NQ = N >> 2;                     // 4-column quads per row

    // Workgroup -> strip.  With swz, strips 2j and 2j+1 (which share 128-byte
    // lines when a strip is 64 bytes wide) go to workgroups 8 apart, i.e. to the
    // same XCD and its L2.
    int strip = blockIdx.x;
    if (swz) {
        const int q = blockIdx.x >> 3, x = blockIdx.x & 7;
        strip = (((q >> 1) << 3) + x) * 2 + (q & 1);
    }
    const int q4 = strip * LC + cl;            // this lane's quad (< NQ: N % (4 LC) == 0)
    const size_t rd = gemv_round_dwords(MR, ksl);

    // round 0 loads first: HBM latency overlaps the activation prologue
    uint4 w[8];
    uint2 sc = make_uint2(0, 0);
    {
        const int g = slot;
        if (g < groups) {
            const uint4 *bp = B4 + (size_t)g * 8 * NQ + q4;
#pragma unroll
            for (int r = 0; r < 8; ++r) w[r] = bp[(size_t)r * NQ];
            sc = S4[(size_t)g * NQ + q4];
        } else {
#pragma unroll
            for (int r = 0; r < 8; ++r) w[r] = make_uint4(0, 0, 0, 0);
        }
    }
    stage_round<MR, BF16>(lds, A, M, K, groups, 0, ksl);

    uint32_t B2 = gemv_base2(BF16);
    asm volatile("" : "+v"(B2));  // the decode base lives in one VGPR
    float acc[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[m][c] = 0.0f;

    for (int rr = 0; rr < rounds; ++rr) {
        __syncthreads();  // round rr staged; round rr-1 fully consumed
        uint32_t *buf = lds + (size_t)(rr & 1) * rd;
        const int g = rr * ksl + slot;
        // next round: loads in flight and its activations staged while this one computes
        uint4 wn[8];
        uint2 scn = make_uint2(0, 0);
        const int gn = g + ksl;
        if (rr + 1 < rounds) {
            if (gn < groups) {
                const uint4 *bp = B4 + (size_t)gn * 8 * NQ + q4;
#pragma unroll
                for (int r = 0; r < 8; ++r) wn[r] = bp[(size_t)r * NQ];
                scn = S4[(size_t)gn * NQ + q4];
            } else {
#pragma unroll
                for (int r = 0; r < 8; ++r) wn[r] = make_uint4(0, 0, 0, 0);
            }
            stage_round<MR, BF16>(lds + (size_t)((rr + 1) & 1) * rd, A, M, K, groups, (rr + 1) * ksl, ksl);
        }
        if (g < groups) {
            const uint32_t *pairs = buf + (size_t)slot * kGroupStride;
            const float *beta = (const float *)(buf + (size_t)MR * ksl * kGroupStride);
            float accg[MR][4];
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int c = 0; c < 4; ++c) accg[m][c] = 0.0f;
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                uint4 ap[MR][2];
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    const uint4 *pp = (const uint4 *)(pairs + (size_t)m * ksl * kGroupStride + r * 8);
                    ap[m][0] = pp[0];
                    ap[m][1] = pp[1];
                }
                const uint32_t wv[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    uint32_t d[8];
                    gemv_decode_word<BF16>(wv[c], d, B2);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float a = accg[m][c];
                        a = dot2<BF16>(d[0], ap[m][0].x, a);
                        a = dot2<BF16>(d[1], ap[m][0].y, a);
                        a = dot2<BF16>(d[2], ap[m][0].z, a);
                        a = dot2<BF16>(d[3], ap[m][0].w, a);
                        a = dot2<BF16>(d[4], ap[m][1].x, a);
                        a = dot2<BF16>(d[5], ap[m][1].y, a);
                        a = dot2<BF16>(d[6], ap[m][1].z, a);
                        a = dot2<BF16>(d[7], ap[m][1].w, a);
                        accg[m][c] = a;
                    }
                }
            }
            const float s[4] = {dt2f<BF16>(sc.x & 0xffffu), dt2f<BF16>(sc.x >> 16),
                                dt2f<BF16>(sc.y & 0xffffu), dt2f<BF16>(sc.y >> 16)};
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                const float bt = beta[m * ksl + slot];
#pragma unroll
                for (int c = 0; c < 4; ++c) acc[m][c] += (accg[m][c] - bt) * s[c];
            }
        }
        if (rr + 1 < rounds) {
#pragma unroll
            for (int r = 0; r < 8; ++r) w[r] = wn[r];
            sc = scn;
        }
    }

    // ---- reduction: k-slots of the wave, then waves in order ----------------
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int o = LC; o < 64; o <<= 1) acc[m][c] += __shfl_xor(acc[m][c], o);
    if (W > 1) {
        __syncthreads();  // every wave is done with the round buffers
        float4 *red = (float4 *)lds;  // [W][MR][LC]
        if (kl == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
                red[(wave * MR + m) * LC + cl] = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
        }
        __syncthreads();
        if (wave != 0) return;
        if (kl == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
                for (int w2 = 1; w2 < W; ++w2) {
                    const float4 t = red[(w2 * MR + m) * LC + cl];
                    acc[m][0] += t.x; acc[m][1] += t.y; acc[m][2] += t.z; acc[m][3] += t.w;
                }
        }
    }
    if (kl != 0) return;
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
#pragma unroll
        for (int m = 0; m < MR; ++m)
            if (m < M)
                epi_store4_c<BF16, decltype(P_)::value, decltype(F_)::value>(C, Other, Bias, N, m, q4 * 4, acc[m]);
    });
}

// Test hooks: the reference-semantics unpack and the GEMV's own decode.
template <bool BF16>
__global__ void k_int2_dequant(const uint32_t *__restrict__ B, const uint16_t *__restrict__ S,
                               uint16_t *__restrict__ W, int K, int N) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (size_t)K * N) return;
    const int k = (int)(i / N), n = (int)(i % N);
    W[i] = (uint16_t)dq_one(B[(size_t)(k >> 4) * N + n], k & 15, S[(size_t)(k / kGS) * N + n]);
}

template <bool BF16>
__global__ void k_int2_gemv_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D,
                                   size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    uint32_t d[8];
    uint32_t B2 = gemv_base2(BF16);
    asm volatile("" : "+v"(B2));
    gemv_decode_word<BF16>(B[i], d, B2);
#pragma unroll
    for (int j = 0; j < 8; ++j) D[i * 8 + j] = d[j];
}

int gemv_mr(int M) { return M <= 1 ? 1 : (M <= 2 ? 2 : (M <= 4 ? 4 : 8)); }

struct GemvPlan {
    int waves, lc;
    size_t lds;
};

constexpr size_t kMaxLds = 64 * 1024;

size_t gemv_lds(int MR, int waves, int lc, int groups) {
    const int ksl = waves * (64 / lc);
    const int rounds = (groups + ksl - 1) / ksl;
    const size_t stage = (size_t)(rounds > 1 ? 2 : 1) * gemv_round_dwords(MR, ksl) * 4;
    const size_t red = (size_t)waves * MR * lc * 16;
    return stage > red ? stage : red;
}

// Automatic tile: LC (lanes across a strip of 4*LC columns) as large as keeps
// >= 384 workgroups (so every CU gets one or two), then the waves that cover
// the 128-row groups in the fewest rounds with the fewest idle k-slots, within
// the 64 KiB LDS budget.
GemvPlan gemv_plan(int M, int N, int K, int waves, int lc) {
    const int MR = gemv_mr(M), groups = K / kGS;
    GemvPlan p;
    if (lc > 0) {
        p.lc = lc;
    } else {
        p.lc = 4;
        for (int c : {16, 8})
            if (N % (4 * c) == 0 && N / (4 * c) >= 384) { p.lc = c; break; }
        if (p.lc == 4 && N % 32 == 0 && N / 32 >= 192) p.lc = 8;  // 128-byte segments if >= 192 workgroups
    }
    const int lk = 64 / p.lc;
    if (waves > 0) {
        p.waves = waves;
    } else {
        int best = 1, best_cost = 1 << 30;
        for (int wv = 1; wv <= gemv_max_waves(MR); ++wv) {
            if (gemv_lds(MR, wv, p.lc, groups) > kMaxLds) break;
            const int ksl = wv * lk;
            const int rounds = (groups + ksl - 1) / ksl;
            const int cost = rounds * 1024 + (rounds * ksl - groups) * 1024 / ksl;  // rounds, then idle slots
            if (cost < best_cost) { best_cost = cost; best = wv; }
        }
        p.waves = best;
    }
    p.lds = gemv_lds(MR, p.waves, p.lc, groups);
    return p;
}

template <int MR, int LC, bool BF16>
hipError_t launch_gemv_t(const GemvPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                         const void *Other, const void *Bias, int M, int N, int K, int postop,
                         int out_f32, hipStream_t st) {
    const int strips = N / (4 * LC);
    const int swz = (LC == 4 && strips % 16 == 0) ? 1 : 0;
    hipLaunchKernelGGL((k_int2_gemv<MR, LC, BF16>), dim3(strips), dim3(64 * p.waves), p.lds, st,
                       (const uint16_t *)A, (const uint4 *)B, (const uint2 *)S, C,
                       (const uint16_t *)Other, Bias, M, N, K, postop, out_f32, swz);
    return hipGetLastError();
}

template <int MR, bool BF16>
hipError_t launch_gemv_lc(const GemvPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                          const void *Other, const void *Bias, int M, int N, int K, int postop,
                          int out_f32, hipStream_t st) {
    switch (p.lc) {
    case 8: return launch_gemv_t<MR, 8, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 16: return launch_gemv_t<MR, 16, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    default: return launch_gemv_t<MR, 4, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
}

template <bool BF16>
hipError_t launch_gemv(const GemvPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    switch (gemv_mr(M)) {
    case 1: return launch_gemv_lc<1, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return launch_gemv_lc<2, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 4: return launch_gemv_lc<4, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    default: return launch_gemv_lc<8, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
}

}  // namespace

// ---- entry points used by api.cpp -----------------------------------------

ternocl_status int2_gemv_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                             const void *Other, const void *Bias, int M, int N, int K, int postop,
                             int out_f32, int waves, int lc, hipStream_t st) {
    if (lc != 0 && lc != 4 && lc != 8 && lc != 16) {
        set_error("col_lanes must be 0 (automatic), 4, 8 or 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (waves < 0 || waves > gemv_max_waves(gemv_mr(M))) {
        set_error("waves must be 0 (automatic) .. 16 for M = 1, .. 8 for M = 2..8");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const GemvPlan p = gemv_plan(M, N, K, waves, lc);
    if (N % (4 * p.lc)) {
        set_error("N must be a multiple of 4 * col_lanes");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (p.lds > kMaxLds) {
        set_error("GEMV plan needs more than 64 KiB of LDS: use fewer waves");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const hipError_t e = dtype == TERNOCL_BF16
        ? launch_gemv<true>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st)
        : launch_gemv<false>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return launch_status(e);
}

ternocl_status int2_dequant_run(int dtype, const uint32_t *B, const void *S, void *W, int K, int N,
                                hipStream_t st) {
    const size_t total = (size_t)K * N;
    const unsigned blocks = (unsigned)((total + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_dequant<true>, dim3(blocks), dim3(256), 0, st, B,
                           (const uint16_t *)S, (uint16_t *)W, K, N);
    else
        hipLaunchKernelGGL(k_int2_dequant<false>, dim3(blocks), dim3(256), 0, st, B,
                           (const uint16_t *)S, (uint16_t *)W, K, N);
    return check_launch();
}

ternocl_status int2_gemv_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N,
                                    hipStream_t st) {
    const size_t words = (size_t)(K / 16) * N;
    const unsigned blocks = (unsigned)((words + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_gemv_decode<true>, dim3(blocks), dim3(256), 0, st, B, D, words);
    else
        hipLaunchKernelGGL(k_int2_gemv_decode<false>, dim3(blocks), dim3(256), 0, st, B, D, words);
    return check_launch();
}

}  // namespace tcl
