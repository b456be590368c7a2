// misc.hip -- small utility kernels: workspace zero-fill (used instead of
// hipMemsetAsync so a call stays capturable in a HIP graph).
#include "common.hpp"

namespace tcl {
namespace {

__global__ void k_fill_zero(uint32_t *__restrict__ p, size_t words) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < words;
         i += (size_t)gridDim.x * blockDim.x)
        p[i] = 0u;
}

__global__ void k_fill_zero_bytes(uint8_t *__restrict__ p, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = 0u;
}

}  // namespace

ternocl_status fill_zero_run(void *p, size_t bytes, hipStream_t st) {
    const size_t words = bytes / 4, tail = bytes % 4;
    if (words) {
        size_t blocks = (words + 255) / 256;
        if (blocks > 65535) blocks = 65535;
        hipLaunchKernelGGL(k_fill_zero, dim3((unsigned)blocks), dim3(256), 0, st, (uint32_t *)p, words);
    }
    if (tail)
        hipLaunchKernelGGL(k_fill_zero_bytes, dim3(1), dim3(64), 0, st, (uint8_t *)p + words * 4, tail);
    return check_launch();
}

}  // namespace tcl
