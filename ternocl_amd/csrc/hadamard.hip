// hadamard.hip -- fused sign flip + blockwise normalised Walsh-Hadamard
// transform on gfx950, replacing hadamard_fwht (hadamard/hadamard_fwht.cl:62-115):
//
//   y = DT(SCALE_n * H_n(s .* x))   per n = HB-wide block along K of a [rows, K] DT tensor
//
// fp32 butterflies (a + b, a - b), stages in increasing stride 1, 2, ..., n/2:
// the same fp32 operations, in the same order per element, as the reference's
// radix-8 passes and radix-2/4 tail (each pass is three consecutive radix-2
// stages), so the result is bit-identical to it.  SCALE_n = 1/sqrt(n) rounded
// to fp32.  A tail of K % HB elements (the reference leaves it unwritten) is
// transformed as one smaller block when its size is a power of two.
//
// Two kernels, the same operations per element:
//  * k_fwht_r (16-byte aligned x and y, K % 8 == 0, a tail block of 0 or >= 8
//    elements): thread t holds elements 8t .. 8t + 7 of its block in
//    registers; strides 1, 2, 4 run in registers, 8 .. 256 between the lanes
//    of a wave (lane xor stride / 8), 512 and up between the waves of the
//    workgroup through LDS.  One 16-byte load and store per thread; a 512-block
//    needs no barrier at all.
//  * k_fwht (any other case): one workgroup of 256 threads per block, the
//    block in LDS as fp32, one barrier per stage.
// Both are latency-bound at the sizes of a decode step (one row of a few
// thousand elements).
#include "common.hpp"

namespace tcl {
namespace {

constexpr int kFwhtThreads = 256;

template <bool BF16>
__global__ void __launch_bounds__(kFwhtThreads)
k_fwht(const uint16_t *__restrict__ x, const int8_t *__restrict__ signs, uint16_t *__restrict__ y,
       int K, int HB, int use_signs, float scale_full, float scale_tail) {
    extern __shared__ float v[];  // HB floats
    const int nblk = (K + HB - 1) / HB;
    const int row = blockIdx.x / nblk, b = blockIdx.x - row * nblk;
    const int k0 = b * HB;
    const int n = min(HB, K - k0);  // a power of two
    const uint16_t *xb = x + (size_t)row * K + k0;
    uint16_t *yb = y + (size_t)row * K + k0;
    const int t = threadIdx.x;

    for (int i = t; i < n; i += kFwhtThreads) {
        float f = dt2f<BF16>(xb[i]);
        if (use_signs) f *= (float)signs[k0 + i];
        v[i] = f;
    }
    __syncthreads();
    for (int h = 1; h < n; h <<= 1) {
        const int lh = __builtin_ctz(h);
        for (int p = t; p < (n >> 1); p += kFwhtThreads) {
            const int i = ((p >> lh) << (lh + 1)) | (p & (h - 1));
            const float a = v[i], c = v[i + h];
            v[i] = a + c;
            v[i + h] = a - c;
        }
        __syncthreads();
    }
    const float sc = n == HB ? scale_full : scale_tail;
    for (int i = t; i < n; i += kFwhtThreads) yb[i] = (uint16_t)f2dt<BF16>(v[i] * sc);
}

// Thread t of block (row, b): elements 8t .. 8t + 7 (threads past the block's
// n / 8 idle; the block's waves past n / 512 only meet the barriers).
template <bool BF16>
__global__ void __launch_bounds__(512)
k_fwht_r(const uint16_t *__restrict__ x, const int8_t *__restrict__ signs, uint16_t *__restrict__ y, int K, int HB,
         int use_signs, float scale_full, float scale_tail) {
    extern __shared__ float xw[];  // HB >= 1024: the block, for the strides between waves
    const int nblk = (K + HB - 1) / HB;
    const int row = blockIdx.x / nblk, b = blockIdx.x - row * nblk;
    const int k0 = b * HB;
    const int n = min(HB, K - k0);  // a power of two (>= 8)
    const int t = threadIdx.x, lane = t & 63, e0 = 8 * t;
    const bool live = e0 < n;
    float v[8];
    {
        const int ec = live ? e0 : 0;
        const uint4 raw = *(const uint4 *)(x + (size_t)row * K + k0 + ec);
        const uint2 sg = use_signs ? *(const uint2 *)(signs + k0 + ec) : make_uint2(0u, 0u);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            float f = dt2f<BF16>((w[i >> 1] >> (16 * (i & 1))) & 0xffffu);
            if (use_signs) f *= (float)(int8_t)(((i < 4 ? sg.x : sg.y) >> (8 * (i & 3))) & 0xffu);
            v[i] = f;
        }
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)  // (n >= 8)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if ((j & h) == 0) {
                const float a = v[j], c = v[j + h];
                v[j] = a + c;
                v[j + h] = a - c;
            }
    for (int h = 8; h < n && h < 512; h <<= 1) {  // partner lane ^ h / 8 holds elements i ^ h
        const int m = h >> 3;
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __shfl_xor(v[j], m);
            v[j] = up ? p - v[j] : v[j] + p;  // (a + c, a - c) with a the lower element
        }
    }
    for (int h = 512; h < n; h <<= 1) {  // partner thread t ^ h / 8, through LDS
        if (live)
#pragma unroll
            for (int j = 0; j < 8; ++j) xw[e0 + j] = v[j];
        __syncthreads();
        const bool up = (e0 & h) != 0;
        if (live)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float p = xw[(e0 ^ h) + j];
                v[j] = up ? p - v[j] : v[j] + p;
            }
        __syncthreads();
    }
    if (!live) return;
    const float sc = n == HB ? scale_full : scale_tail;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)f2dt<BF16>(v[2 * i] * sc) | ((uint32_t)f2dt<BF16>(v[2 * i + 1] * sc) << 16);
    *(uint4 *)(y + (size_t)row * K + k0 + e0) = make_uint4(o[0], o[1], o[2], o[3]);
}

}  // namespace

ternocl_status fwht_run(int dtype, const void *x, const int8_t *signs, void *y, int rows, int K,
                        int HB, int use_signs, float scale_full, float scale_tail, hipStream_t st) {
    const int nblk = (K + HB - 1) / HB, tail = K % HB;
    const dim3 grid((unsigned)(rows * nblk));
    const bool reg = ((uintptr_t)x & 15) == 0 && ((uintptr_t)y & 15) == 0 && K % 8 == 0 &&
                     (tail == 0 || tail >= 8) && (!use_signs || ((uintptr_t)signs & 7) == 0);
    if (reg) {
        const dim3 block((unsigned)(HB / 8));
        const size_t lds = HB >= 1024 ? (size_t)HB * sizeof(float) : 0;
        if (dtype == TERNOCL_BF16)
            hipLaunchKernelGGL(k_fwht_r<true>, grid, block, lds, st, (const uint16_t *)x, signs, (uint16_t *)y, K,
                               HB, use_signs, scale_full, scale_tail);
        else
            hipLaunchKernelGGL(k_fwht_r<false>, grid, block, lds, st, (const uint16_t *)x, signs, (uint16_t *)y, K,
                               HB, use_signs, scale_full, scale_tail);
        return check_launch();
    }
    const dim3 block(kFwhtThreads);
    const size_t lds = (size_t)HB * sizeof(float);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_fwht<true>, grid, block, lds, st, (const uint16_t *)x, signs, (uint16_t *)y,
                           K, HB, use_signs, scale_full, scale_tail);
    else
        hipLaunchKernelGGL(k_fwht<false>, grid, block, lds, st, (const uint16_t *)x, signs, (uint16_t *)y,
                           K, HB, use_signs, scale_full, scale_tail);
    return check_launch();
}

}  // namespace tcl
