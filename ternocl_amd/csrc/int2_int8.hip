// int2_int8.hip -- the int2 x int8 prefill path on gfx950: the activation
// quantization pre-kernel and the s8 x s2 GEMM, replacing quant_a and
// int2_int8_{gemv,gemm_mt} of int2_via_int2_x_int8_dpas/int2_int8_dpas.cl
// (:101-123, :210-281, :313-385) in its upfront-quantization mode (QMODE 0).
//
//   SA[g, m] = DT(127 / max(absmax_{k in g} |A[m, k]|, FLT_EPSILON))
//   Aq[m, k] = sat_int8(rte(A[m, k] * SA[k/128, m]))
//   C[m, n]  = ct(epi(sum_g float(sum_{k in g} Aq[m,k] * v(B[k,n])) * (SB[g,n] * (1 / SA[g,m]))))
//
// with v the 2-bit two's-complement value of the code ({0,1,2,3} = {0,1,-2,-1}).
//
// quant_a is HBM-bound: one thread per 8 activations (one 16-byte load), the 16
// threads of a 128-group reduce the absmax with cross-lane xor shuffles.  The
// scale is 127 / x with a correctly rounded fp32 divide (the reference builds
// with -cl-fp32-correctly-rounded-divide-sqrt), q = rint(a * sa) saturated; the
// product of two 16-bit floats is exact in fp32, so q is bit-exact.
//
// The GEMM: a workgroup of 4 waves computes a 128 x 128 tile of C, each wave a
// 64 x 64 quarter as 4 x 4 v_mfma_i32_16x16x64_i8 tiles; K advances one
// 128-row scale group at a time (two MFMA k-steps of 64).
//   * B stays packed in HBM / L2: lane (c, q) of a wave loads, per k-step and
//     16-column block, the word of k rows 16*(4*ks+q) .. +15 of its column and
//     turns it into the 16 int8 of its MFMA B fragment with v_perm_b32 through
//     the byte table {0x00, 0x01, 0xFE, 0xFF} indexed by the code:
//     dword i = codes of rows i, i+4, i+8, i+12 (selector (w >> 2i) & 0x03030303);
//   * Aq goes global -> registers -> LDS once per workgroup and group, each
//     16-byte chunk 4x4 byte-transposed on the way so that its dword i holds
//     rows i, i+4, i+8, i+12 too (the same k order as B: the int32 dot is exact
//     whatever the order, as long as A and B agree);
//   * 1 / SA[g, m] of the tile's 128 rows is computed once per group into LDS;
//   * each group's dot products start from zero in int32 accumulators and are
//     folded into fp32 accumulators with acc += float(dot) * (SB * inv), the
//     order of the reference's host gold (int2_via_int2_x_int8_dpas/main.cpp:113-116).
#include "common.hpp"

#include <cfloat>

namespace tcl {
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kEps = FLT_EPSILON;  // xetla's absmax floor, int2_int8_dpas.cl:59

__host__ __device__ constexpr int ldsa_of(int M) { return (M + 31) & ~31; }

// ---- quant_a ---------------------------------------------------------------

template <bool BF16>
__global__ void __launch_bounds__(256)
k_quant_a(const uint16_t *__restrict__ A, uint16_t *__restrict__ SA, int8_t *__restrict__ Aq, int M,
          int K) {
    const int cpr = K >> 3;  // 8-element chunks per row (a multiple of 16)
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // the 16 chunks of a group are 16 aligned consecutive threads: they leave together
    if (t >= (size_t)M * cpr) return;
    const int m = (int)(t / cpr), c = (int)(t - (size_t)m * cpr);
    const uint4 v = *(const uint4 *)(A + (size_t)m * K + 8 * (size_t)c);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float a[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        a[2 * i] = dt2f<BF16>(w[i] & 0xffffu);
        a[2 * i + 1] = dt2f<BF16>(w[i] >> 16);
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(a[i]));
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
    const uint32_t sh = f2dt<BF16>(127.0f / fmaxf(mx, kEps));
    if ((c & 15) == 0) SA[(size_t)(c >> 4) * ldsa_of(M) + m] = (uint16_t)sh;
    const float s = dt2f<BF16>(sh);
    uint32_t q[2] = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // exact product, rounded to nearest even and saturated; NaN (0 * inf
        // when an fp16 scale overflows) gives 0, as convert_char8_sat_rte
        const float p = a[i] * s;
        const float r = p == p ? fminf(fmaxf(__builtin_rintf(p), -128.0f), 127.0f) : 0.0f;
        q[i >> 2] |= ((uint32_t)(int)r & 0xffu) << (8 * (i & 3));
    }
    *(uint2 *)(Aq + (size_t)m * K + 8 * (size_t)c) = make_uint2(q[0], q[1]);
}

// ---- s8 x s2 GEMM ------------------------------------------------------------

constexpr int QBM = 128, QBN = 128;
constexpr int QA_PITCH = 144;  // bytes per LDS row of the A tile (128 + 16: conflict-free b128 reads)
constexpr uint32_t kCodeLut = 0xFFFE0100u;  // int8 of code 0, 1, 2, 3

// out[i] byte b = byte i of d[b] (4 x 4 byte transpose)
__device__ __forceinline__ void transpose4x4(const uint32_t d[4], uint32_t o[4]) {
    const uint32_t p0 = __builtin_amdgcn_perm(d[1], d[0], 0x06020400u);  // d0.b0 d1.b0 d0.b2 d1.b2
    const uint32_t p1 = __builtin_amdgcn_perm(d[1], d[0], 0x07030501u);  // d0.b1 d1.b1 d0.b3 d1.b3
    const uint32_t p2 = __builtin_amdgcn_perm(d[3], d[2], 0x06020400u);
    const uint32_t p3 = __builtin_amdgcn_perm(d[3], d[2], 0x07030501u);
    o[0] = __builtin_amdgcn_perm(p2, p0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(p3, p1, 0x05040100u);
    o[2] = __builtin_amdgcn_perm(p2, p0, 0x07060302u);
    o[3] = __builtin_amdgcn_perm(p3, p1, 0x07060302u);
}

// B fragment of one word: dword i byte b = int8 value of row 4b + i.
__device__ __forceinline__ i32x4_t decode_s2(uint32_t w) {
    i32x4_t r;
    r[0] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, w & 0x03030303u);
    r[1] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 2) & 0x03030303u);
    r[2] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 4) & 0x03030303u);
    r[3] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 6) & 0x03030303u);
    return r;
}

template <bool BF16>
__global__ void __launch_bounds__(256)
k_int2_int8_gemm(const int8_t *__restrict__ Aq, const uint16_t *__restrict__ SA,
                 const uint32_t *__restrict__ B, const uint16_t *__restrict__ SB,
                 void *__restrict__ C, const uint16_t *__restrict__ Other,
                 const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32) {
    __shared__ __attribute__((aligned(16))) uint8_t lds_a[2][QBM * QA_PITCH];
    __shared__ float lds_inv[2][QBM];

    const int mt = (M + QBM - 1) / QBM, nt = (N + QBN - 1) / QBN;
    int tm, tn;
    xcd_tile_of(blockIdx.x, mt, nt, tm, tn);
    const int m0 = tm * QBM, n0 = tn * QBN;
    const int mrows = min(QBM, M - m0);
    const int groups = K / kGS;
    const int lda = ldsa_of(M);

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, q = lane >> 4;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // A staging: thread tid owns the 16-byte chunk (tid & 7) of rows (tid >> 3) + 32u
    const int arow0 = tid >> 3, achunk = tid & 7;
    uint4 av[4];
    auto a_load = [&](int g) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int r = arow0 + 32 * u;
            const int rc = r < mrows ? r : mrows - 1;
            av[u] = *(const uint4 *)(Aq + (size_t)(m0 + rc) * K + (size_t)g * kGS + 16 * achunk);
        }
    };
    uint32_t sa_raw = 0;
    auto sa_load = [&](int g) {
        if (tid < QBM) sa_raw = SA[(size_t)g * lda + m0 + (tid < mrows ? tid : mrows - 1)];
    };
    auto a_store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            // rows past mrows are zeroed here, not at the load (that would wait for it)
            const uint4 a = arow0 + 32 * u < mrows ? av[u] : make_uint4(0, 0, 0, 0);
            const uint32_t d[4] = {a.x, a.y, a.z, a.w};
            uint32_t o[4];
            transpose4x4(d, o);
            *(uint4 *)(&lds_a[buf][(arow0 + 32 * u) * QA_PITCH + 16 * achunk]) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        if (tid < QBM) {
            const float sa = dt2f<BF16>(sa_raw);
            lds_inv[buf][tid] = (tid < mrows && sa != 0.0f) ? 1.0f / sa : 0.0f;
        }
    };

    // B words of this wave for group g: block cb, k-step ks -> word kp = 8g + 4ks + q
    uint32_t bw[4][2], sbr[4];
    auto b_load = [&](int g) {
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            int n = n0 + wn + 16 * cb + c16;
            n = n < N ? n : N - 1;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) bw[cb][ks] = B[((size_t)g * 8 + 4 * ks + q) * N + n];
            sbr[cb] = SB[(size_t)g * N + n];
        }
    };

    f32x4_t acc[4][4];
#pragma unroll
    for (int mb = 0; mb < 4; ++mb)
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) acc[mb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    a_load(0);
    sa_load(0);
    b_load(0);
    a_store(0);
    for (int g = 0; g < groups; ++g) {
        __syncthreads();  // tile g staged; tile g - 1 consumed
        const int buf = g & 1;
        uint32_t bwc[4][2], sbc[4];
#pragma unroll
        for (int cb = 0; cb < 4; ++cb) {
            sbc[cb] = sbr[cb];
            bwc[cb][0] = bw[cb][0];
            bwc[cb][1] = bw[cb][1];
        }
        const bool more = g + 1 < groups;
        if (more) {  // next group's loads in flight during this group's MFMAs
            a_load(g + 1);
            sa_load(g + 1);
            b_load(g + 1);
        }
        i32x4_t dot[4][4];
#pragma unroll
        for (int ks = 0; ks < 2; ++ks) {
            i32x4_t af[4];
#pragma unroll
            for (int mb = 0; mb < 4; ++mb) {
                const uint4 v = *(const uint4 *)(&lds_a[buf][(wm + 16 * mb + c16) * QA_PITCH + (4 * ks + q) * 16]);
                af[mb] = i32x4_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const i32x4_t bf = decode_s2(bwc[cb][ks]);
#pragma unroll
                for (int mb = 0; mb < 4; ++mb)
                    dot[mb][cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(
                        af[mb], bf, ks == 0 ? i32x4_t{0, 0, 0, 0} : dot[mb][cb], 0, 0, 0);
            }
        }
        // fold the group into the fp32 accumulators: acc += float(dot) * (SB * (1 / SA))
#pragma unroll
        for (int mb = 0; mb < 4; ++mb) {
            const f32x4_t inv = *(const f32x4_t *)(&lds_inv[buf][wm + 16 * mb + 4 * q]);
#pragma unroll
            for (int cb = 0; cb < 4; ++cb) {
                const float sb = dt2f<BF16>(sbc[cb]);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb][cb][i] += (float)dot[mb][cb][i] * (sb * inv[i]);
            }
        }
        if (more) a_store(buf ^ 1);
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
                if (r < mrows) epi_store1<BF16>(C, Other, Bias, postop, out_f32, N, m0 + r, n, acc[mb][cb][i]);
            }
    }
}

// Test hook: the MFMA B fragment each word decodes to (4 dwords per word).
__global__ void k_int2_s8_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D, int words) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const i32x4_t r = decode_s2(B[i]);
    *(uint4 *)(D + (size_t)i * 4) = make_uint4((uint32_t)r[0], (uint32_t)r[1], (uint32_t)r[2], (uint32_t)r[3]);
}

}  // namespace

ternocl_status quant_a_run(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K, hipStream_t st) {
    const size_t threads = (size_t)M * (K / 8);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_quant_a<true>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)A,
                           (uint16_t *)SA, Aq, M, K);
    else
        hipLaunchKernelGGL(k_quant_a<false>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)A,
                           (uint16_t *)SA, Aq, M, K);
    return check_launch();
}

ternocl_status int2_int8_gemm_run(int dtype, const int8_t *Aq, const void *SA, const uint32_t *B,
                                  const void *SB, void *C, const void *Other, const void *Bias, int M,
                                  int N, int K, int postop, int out_f32, hipStream_t st) {
    const int mt = (M + QBM - 1) / QBM, nt = (N + QBN - 1) / QBN;
    const dim3 grid(mt * nt), block(256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_int8_gemm<true>, grid, block, 0, st, Aq, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    else
        hipLaunchKernelGGL(k_int2_int8_gemm<false>, grid, block, 0, st, Aq, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    return check_launch();
}

ternocl_status int2_s8_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st) {
    const int words = K / 16 * N;
    hipLaunchKernelGGL(k_int2_s8_decode, dim3((words + 255) / 256), dim3(256), 0, st, B, D, words);
    return check_launch();
}

}  // namespace tcl
