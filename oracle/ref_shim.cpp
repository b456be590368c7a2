// ref_shim.cpp -- builds oracle/_ref/libternocl_ref.so from the reference's own
// host sources, where they lie (the Makefile passes -I for common/ and each
// variant directory).  TEST INFRASTRUCTURE ONLY: used by tests/ to pin the
// oracle (ternocl_oracle.c) and by bench.py's cpu_baseline leg.
//
// The golds are `static` functions inside the drivers' main.cpp files, so each
// driver is compiled inside its own namespace here (its `main` renamed) and the
// functions are re-exported with C linkage.  The drivers' OpenCL code is
// compiled and linked (libOpenCL is in the image) but never called.
#define CL_TARGET_OPENCL_VERSION 300
#include <CL/cl.h>
#include <omp.h>

#include <algorithm>
#include <array>
#include <cfloat>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <iomanip>
#include <iostream>
#include <numeric>
#include <random>
#include <sstream>
#include <string>
#include <vector>

#include "bitcos.hpp"    // common/bitcos.hpp
#include "dt16.hpp"      // common/dt16.hpp
#include "epilogue.hpp"  // common/epilogue.hpp

namespace ref_int2 {
#define main ref_int2_main
#include "int2_fp16_upcvt/main.cpp"
#undef main
#undef CL_CHECK
}  // namespace ref_int2

namespace ref_int8 {
#define main ref_int8_main
#include "int2_via_int2_x_int8_dpas/main.cpp"
#undef main
#undef CL_CHECK
}  // namespace ref_int8

namespace ref_bitcos {
#define main ref_bitcos_main
#include "bitcos_fp16_upcvt/main.cpp"
#undef main
#undef CL_CHECK
}  // namespace ref_bitcos

extern "C" {

void ref_set_bf16(int bf16) { dt_is_bf16() = bf16 != 0; }
// OpenMP threads of the reference's gold loops (the CPU baseline times 1 core and all)
void ref_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int ref_max_threads() { return omp_get_max_threads(); }
float ref_tof(uint16_t h) { return tof(h); }
uint16_t ref_fromf(float f) { return fromf(f); }

// int2_fp16_upcvt/main.cpp:79-98
void ref_int2_gold(const uint16_t *A, const uint32_t *B, const uint16_t *S, float *C, int M,
                   int K, int N) {
    ref_int2::compute_gold(A, B, S, C, M, K, N);
}

// common/epilogue.hpp:98-115
void ref_epilogue(int postop, int out_f32, const float *acc, const uint16_t *other,
                  const unsigned char *bias, unsigned char *out, int M, int N) {
    Epilogue e;
    e.postop = postop;
    e.out_f32 = out_f32 != 0;
    epilogue_ref(e, acc, other, bias, out, M, N);
}

float ref_sigmoid(float x) { return sigmoid_ref(x); }

// int2_via_int2_x_int8_dpas/main.cpp:82-91
void ref_scale_a(const uint16_t *A, uint16_t *SA, int M, int K) {
    ref_int8::compute_scale_a(A, SA, M, K);
}

// int2_via_int2_x_int8_dpas/main.cpp:94-121
void ref_int8_gold(const uint16_t *A, const uint32_t *B, const uint16_t *SA, const uint16_t *SB,
                   float *C, int M, int K, int N) {
    ref_int8::compute_gold(A, B, SA, SB, C, M, K, N);
}

// common/bitcos.hpp:81-94, :97-106 and bitcos_fp16_upcvt/main.cpp:64-86, on a
// caller-provided BITCOS buffer
static Bitcos wrap_bitcos(const uint32_t *buf, size_t words, int K, int N) {
    Bitcos b;
    b.K = K;
    b.N = N;
    b.buf.assign(buf, buf + words);
    return b;
}

void ref_bitcos_slice_ranks(const uint32_t *buf, size_t words, int K, int N, int ls,
                            uint32_t *sr) {
    const Bitcos b = wrap_bitcos(buf, words, K, N);
    const std::vector<uint32_t> r = bitcos_slice_ranks(b, ls);
    std::copy(r.begin(), r.end(), sr);
}

void ref_bitcos_decode_col(const uint32_t *buf, size_t words, int K, int N, int n,
                           int8_t *codes) {
    const Bitcos b = wrap_bitcos(buf, words, K, N);
    bitcos_decode_col(b, n, codes);
}

void ref_bitcos_gold(const uint16_t *A, const uint32_t *buf, size_t words, const uint16_t *S,
                     float *C, int M, int K, int N) {
    const Bitcos b = wrap_bitcos(buf, words, K, N);
    ref_bitcos::compute_gold(A, b, S, C, M);
}

// common/bitcos.hpp:31-78 (random BITCOS weights, reference generator)
size_t ref_bitcos_random_words(int K, int N, double z, uint64_t seed) {
    return bitcos_random(K, N, z, seed).buf.size();
}
void ref_bitcos_random(int K, int N, double z, uint64_t seed, uint32_t *out) {
    const Bitcos b = bitcos_random(K, N, z, seed);
    std::copy(b.buf.begin(), b.buf.end(), out);
}

}  // extern "C"
