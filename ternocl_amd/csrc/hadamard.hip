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
// One workgroup of 256 threads per block: the block lives in LDS as fp32, one
// barrier per stage.  The kernel is latency-bound at the sizes of a decode step
// (one row of a few thousand elements).
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

}  // namespace

ternocl_status fwht_run(int dtype, const void *x, const int8_t *signs, void *y, int rows, int K,
                        int HB, int use_signs, float scale_full, float scale_tail, hipStream_t st) {
    const int nblk = (K + HB - 1) / HB;
    const dim3 grid((unsigned)(rows * nblk)), block(kFwhtThreads);
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
