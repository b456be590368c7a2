// api.cpp -- the C ABI (include/ternocl_amd.h): host-side argument validation
// and dispatch to the kernels of the other translation units.  Nothing here
// allocates device memory or synchronises the stream.
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdio>
#include <cstring>

#include "common.hpp"

namespace tcl {

static thread_local char g_err[512] = "";

void set_error(const char *msg) { std::snprintf(g_err, sizeof g_err, "%s", msg); }

ternocl_status launch_status(hipError_t e) {
    if (e == hipSuccess) return TERNOCL_OK;
    std::snprintf(g_err, sizeof g_err, "HIP error %d: %s", (int)e, hipGetErrorString(e));
    return TERNOCL_ERR_LAUNCH;
}

ternocl_status check_launch() { return launch_status(hipGetLastError()); }

// kernels (int2_gemv.hip)
ternocl_status int2_gemv_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                             const void *Other, const void *Bias, int M, int N, int K, int postop,
                             int out_f32, int waves, int lc, hipStream_t st);
ternocl_status int2_dequant_run(int dtype, const uint32_t *B, const void *S, void *W, int K, int N,
                                hipStream_t st);
ternocl_status int2_gemv_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N,
                                    hipStream_t st);
// kernels (int2_gemv_mfma.hip)
ternocl_status int2_gemv_mfma_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K,
                                  int postop, int out_f32, int waves, int cpl, int gpw,
                                  hipStream_t st);
ternocl_status int2_mfma_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N,
                                    hipStream_t st);
// kernels (int2_gemv_f4.hip)
bool int2_gemv_f4_supports(int M, int N, const void *A);
bool int2_int8_gemv_supports(int M, int N, int K, const void *A, const int8_t *Aq);
ternocl_status int2_int8_gemv_run(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                  const uint32_t *B, const void *SB, void *C, const void *Other,
                                  const void *Bias, int M, int N, int K, int postop, int out_f32,
                                  hipStream_t st, void *ws, size_t ws_bytes);
size_t int2_int8_gemv_ws_need(int M, int N, int K);
ternocl_status int2_gemv_f4_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                const void *Other, const void *Bias, int M, int N, int K, int postop,
                                int out_f32, int waves, int cpl, int gpw, int ks, void *ws, size_t ws_bytes,
                                hipStream_t st);
size_t int2_gemv_f4_ws_need(int M, int N, int K);
ternocl_status int2_gemv_f4ms_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K, int postop,
                                  int out_f32, int cpl, int gpw, int ks, void *ws, size_t ws_bytes,
                                  hipStream_t st);
bool int2_gemv_f4ms_auto(int M, int N, int K);
ternocl_status int2_f4_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st);
ternocl_status stream_read_run(const void *src, size_t bytes, void *sink, hipStream_t st);  // misc.hip
ternocl_status int2_gemv_stream_probe_run(int dtype, const uint32_t *B, const void *S, void *C, int M, int N,
                                          int K, hipStream_t st);
// kernels (int2_gemm_mfma.hip)
ternocl_status int2_gemm_mfma_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K,
                                  int postop, int out_f32, hipStream_t st, void *ws = nullptr,
                                  size_t ws_bytes = 0);
size_t int2_gemm_ws_need(int M, int N, int K);
ternocl_status int2_gemm_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st);
// kernels (int2_int8.hip)
ternocl_status quant_a_run(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K, hipStream_t st,
                           const int *perm = nullptr, int topk = 1, const int *nrows = nullptr);
ternocl_status int2_int8_gemm_run(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                  const uint32_t *B, const void *SB, void *C, const void *Other,
                                  const void *Bias, int M, int N, int K, int postop, int out_f32,
                                  hipStream_t st, void *ws = nullptr, size_t ws_bytes = 0);
ternocl_status int2_s8_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st);
// kernels (bitcos.hip)
int bitcos_max_ls();
int bitcos_pick_ls(int N, int K);
ternocl_status bitcos_gemv_run(int dtype, const void *A, const uint32_t *Bc, const void *S,
                               const uint32_t *SR, int ls, void *C, const void *Other, const void *Bias,
                               int M, int N, int K, int postop, int out_f32, hipStream_t st, void *ws = nullptr,
                               size_t ws_bytes = 0);
size_t bitcos_gemv_ws_need(int N, int ls);
ternocl_status bitcos_gemm_mt_run(int dtype, const void *A, const uint32_t *Bc, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K, int postop,
                                  int out_f32, hipStream_t st);
ternocl_status bitcos_slice_ranks_run(const uint32_t *Bc, uint32_t *SR, int N, int K, int ls,
                                      hipStream_t st);
ternocl_status bitcos_dequant_run(int dtype, const uint32_t *Bc, const void *S, void *W, int N, int K,
                                  hipStream_t st);
ternocl_status bitcos_to_int2_run(const uint32_t *Bc, const uint32_t *SR, int ls, uint32_t *W2, int N, int K,
                                  hipStream_t st);
// kernels (hadamard.hip)
ternocl_status fwht_run(int dtype, const void *x, const int8_t *signs, void *y, int rows, int K,
                        int HB, int use_signs, float scale_full, float scale_tail, hipStream_t st);
ternocl_status bitcos_fwht_gemv_run(int dtype, const void *x, const int8_t *signs, int HB, int use_signs,
                                    float scale_full, float scale_tail, const uint32_t *Bc, const void *S,
                                    const uint32_t *SR, int ls, void *C, const void *Other, const void *Bias, int M,
                                    int N, int K, int postop, int out_f32, hipStream_t st, void *ws,
                                    size_t ws_bytes);  // bitcos.hip
// kernels (moe.hip, int2_gemm_mfma.hip)
int moe_tile_rows();
ternocl_status moe_route_run(const int *ids, int *meta, int *perm, int *inv, int G, int E, hipStream_t st,
                             int4 *desc = nullptr);
ternocl_status moe_gather_run(const void *X, const int *perm, void *Xs, int G, int K, int topk, hipStream_t st);
ternocl_status moe_combine_run(int dtype, const float *Y, const int *inv, const void *RW, void *O, int T,
                               int topk, int N, hipStream_t st);
ternocl_status moe_gemm_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                            const uint32_t *B_all, const void *S_all, void *C_all, const void *Other_all,
                            int E, int G, int N, int K, int postop, int out_f32, hipStream_t st,
                            const int4 *desc = nullptr);
MoeWs moe_ws_layout(int T, int E, int topk, int H, int I);  // moe.hip
ternocl_status moe_prefill_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                               int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                               const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                               void *O, void *ws, hipStream_t st);
MoeI8Ws moe_i8_ws_layout(int T, int E, int topk, int H, int I);  // moe.hip
ternocl_status moe_prefill_int8_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                                    int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                    const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                                    void *O, void *ws, hipStream_t st);
int int8_moe_tile_rows();  // int2_int8.hip
size_t moe_decode_ws_bytes(int T, int topk, int H, int I);
ternocl_status moe_decode_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                              int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                              const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                              void *O, void *ws, hipStream_t st);
ternocl_status moe_decode_noalloc_run(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                                      int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                      const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                                      void *O, hipStream_t st);
// kernels (misc.hip)
ternocl_status fill_zero_run(void *p, size_t bytes, hipStream_t st);

}  // namespace tcl

using namespace tcl;

#define FAIL(code, msg)          \
    do {                         \
        set_error(msg);          \
        return (code);           \
    } while (0)

// Operands the MFMA GEMMs address through 32-bit buffer offsets stay below this.
constexpr size_t kMaxBufBytes = (size_t)1 << 31;

static ternocl_status check_dtype(int dtype) {
    if (dtype != TERNOCL_FP16 && dtype != TERNOCL_BF16) FAIL(TERNOCL_ERR_INVALID_ARG, "dtype must be TERNOCL_FP16 or TERNOCL_BF16");
    return TERNOCL_OK;
}

// Shared checks of the int2 / int8 / BITCOS GEMM family.
static ternocl_status check_gemm_common(int dtype, const void *A, const void *B, const void *S,
                                        const void *C, const void *Other, const void *Bias, int M,
                                        int N, int K, int postop, int out_f32) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!A || !B || !S || !C) FAIL(TERNOCL_ERR_INVALID_ARG, "A, B, S and C must be non-null");
    if (M < 1 || N < 1 || K < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "M, N and K must be positive");
    if (N % 16) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "N must be a multiple of 16");
    if (K % kGS) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "K must be a multiple of 128");
    if (postop < 0 || postop > 5) FAIL(TERNOCL_ERR_INVALID_ARG, "postop must be 0..5");
    if (out_f32 != 0 && out_f32 != 1) FAIL(TERNOCL_ERR_INVALID_ARG, "out_f32 must be 0 or 1");
    if (postop_needs_other(postop) && !Other) FAIL(TERNOCL_ERR_INVALID_ARG, "this postop reads Other: it must be non-null");
    if (postop_needs_bias(postop) && !Bias) FAIL(TERNOCL_ERR_INVALID_ARG, "this postop reads Bias: it must be non-null");
    return TERNOCL_OK;
}

extern "C" {

const char *ternocl_status_string(int status) {
    switch (status) {
    case TERNOCL_OK: return "ok";
    case TERNOCL_ERR_INVALID_ARG: return "invalid argument";
    case TERNOCL_ERR_UNSUPPORTED_SHAPE: return "unsupported shape";
    case TERNOCL_ERR_WORKSPACE: return "workspace missing or too small";
    case TERNOCL_ERR_LAUNCH: return "HIP launch error";
    default: return "unknown status";
    }
}

const char *ternocl_last_error(void) { return g_err; }
const char *ternocl_version(void) { return "0.1.0"; }

size_t ternocl_int2_gemm_ws_bytes(int M, int N, int K) {
    if (M < 1 || N < 16 || N % 16 || K < kGS || K % kGS) return 0;
    // the fp8 x fp4 GEMV's K split: slice sums and a counter per strip
    if (M <= 16) return int2_gemv_f4_ws_need(M, N, K);
    // the prefill GEMM's split-K partials (shapes whose 128 x 512 tiles leave CUs idle)
    return int2_gemm_ws_need(M, N, K);
}

ternocl_status ternocl_workspace_zero(void *ws, size_t ws_bytes, void *stream) {
    if (!ws || !ws_bytes) return TERNOCL_OK;
    return fill_zero_run(ws, ws_bytes, (hipStream_t)stream);
}

ternocl_status ternocl_int2_fp16_upcvt_gemm_ex(int dtype, const void *A, const uint32_t *B,
                                               const void *S, void *C, const void *Other,
                                               const void *Bias, int M, int N, int K, int postop,
                                               int out_f32, void *ws, size_t ws_bytes,
                                               const ternocl_gemv_tile *tile, void *stream) {
    ternocl_status s = check_gemm_common(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32);
    if (s != TERNOCL_OK) return s;
    const ternocl_gemv_tile t = tile ? *tile : ternocl_gemv_tile{0, 0, 0, 0, 0, 0};
    if (t.engine < 0 || t.engine > 5) FAIL(TERNOCL_ERR_INVALID_ARG, "tile engine must be 0..5");
    if (t.k_slices < 0 || t.k_slices > 16) FAIL(TERNOCL_ERR_INVALID_ARG, "k_slices must be 0..16");
    if (t.engine == 3 || (M > 16 && t.engine == 0)) {
        if (t.k_slices > 1) FAIL(TERNOCL_ERR_INVALID_ARG, "k_slices > 1: the fp8 x fp4 GEMV (engine 4) only");
        // the GEMM addresses the packed weights with 32-bit buffer offsets
        if ((size_t)(K / 16) * (size_t)N * 4 >= kMaxBufBytes)
            FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the prefill GEMM takes packed weights (K * N / 4 bytes) below 2^31 bytes");
        return int2_gemm_mfma_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32,
                                  (hipStream_t)stream, ws, ws_bytes);
    }
    if (M <= 16) {
        // automatic: the fp8 x fp4 engine where it applies (its multi-strip
        // kernel on many strips), else the bf16/fp16 MFMA GEMV
        const bool auto_tile = t.engine == 0 && t.waves == 0 && t.cols_per_lane == 0 && t.groups_per_wave == 0 &&
                               t.k_slices == 0;
        if (t.engine == 5 || (auto_tile && int2_gemv_f4_supports(M, N, A) && int2_gemv_f4ms_auto(M, N, K))) {
            if (t.waves)
                FAIL(TERNOCL_ERR_INVALID_ARG, "the multi-strip GEMV (engine 5) takes cols_per_lane, "
                                              "groups_per_wave and k_slices (its waves follow from them)");
            if (!int2_gemv_f4_supports(M, N, A))
                FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the multi-strip GEMV takes M <= 8 and A 16-byte aligned");
            return int2_gemv_f4ms_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, t.cols_per_lane,
                                      t.groups_per_wave, t.k_slices, ws, ws_bytes, (hipStream_t)stream);
        }
        if (t.engine == 4 || (t.engine == 0 && int2_gemv_f4_supports(M, N, A)))
            return int2_gemv_f4_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, t.waves,
                                    t.cols_per_lane, t.groups_per_wave, t.k_slices, ws, ws_bytes,
                                    (hipStream_t)stream);
        if (t.k_slices > 1) FAIL(TERNOCL_ERR_INVALID_ARG, "k_slices > 1: the fp8 x fp4 GEMV (engine 4) only");
        if (t.engine == 1) {
            if (M > 8) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the VALU GEMV takes M <= 8");
            return int2_gemv_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, t.waves,
                                 t.col_lanes, (hipStream_t)stream);
        }
        return int2_gemv_mfma_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, t.waves,
                                  t.cols_per_lane, t.groups_per_wave, (hipStream_t)stream);
    }
    FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the GEMV engines take M <= 16 (use engine 0 or 3)");
}

ternocl_status ternocl_int2_fp16_upcvt_gemm(int dtype, const void *A, const uint32_t *B,
                                            const void *S, void *C, const void *Other,
                                            const void *Bias, int M, int N, int K, int postop,
                                            int out_f32, void *ws, size_t ws_bytes, void *stream) {
    return ternocl_int2_fp16_upcvt_gemm_ex(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32,
                                           ws, ws_bytes, nullptr, stream);
}

ternocl_status ternocl_int2_dequant(int dtype, const uint32_t *B, const void *S, void *W, int K,
                                    int N, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!B || !S || !W) FAIL(TERNOCL_ERR_INVALID_ARG, "B, S and W must be non-null");
    if (N < 16 || N % 16 || K < kGS || K % kGS) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % 128 == 0");
    return int2_dequant_run(dtype, B, S, W, K, N, (hipStream_t)stream);
}

ternocl_status ternocl_int2_gemv_decode(int dtype, int engine, const uint32_t *B, uint32_t *D,
                                        int K, int N, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!B || !D) FAIL(TERNOCL_ERR_INVALID_ARG, "B and D must be non-null");
    if (engine < 1 || engine > 4) FAIL(TERNOCL_ERR_INVALID_ARG, "engine must be 1 (VALU), 2 (MFMA GEMV), 3 (GEMM) or 4 (fp8 x fp4 GEMV)");
    if (N < 16 || N % 16 || K < 16 || K % 16) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % 16 == 0");
    if (engine == 4) return int2_f4_decode_run(B, D, K, N, (hipStream_t)stream);
    if (engine == 3) return int2_gemm_decode_run(dtype, B, D, K, N, (hipStream_t)stream);
    if (engine == 2) return int2_mfma_decode_run(dtype, B, D, K, N, (hipStream_t)stream);
    return int2_gemv_decode_run(dtype, B, D, K, N, (hipStream_t)stream);
}

ternocl_status ternocl_stream_read_probe(const void *src, size_t bytes, void *sink, void *stream) {
    if (!src || !sink) FAIL(TERNOCL_ERR_INVALID_ARG, "src and sink must be non-null");
    if (((uintptr_t)src & 15) != 0) FAIL(TERNOCL_ERR_INVALID_ARG, "src must be 16-byte aligned");
    if (bytes / 16 / 1024 >= 0x7fffffffu) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "bytes too large for one launch");
    return stream_read_run(src, bytes, sink, (hipStream_t)stream);
}

ternocl_status ternocl_int2_gemv_stream_probe(int dtype, const uint32_t *B, const void *S, void *C, int M,
                                             int N, int K, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!B || !S || !C) FAIL(TERNOCL_ERR_INVALID_ARG, "B, S and C must be non-null");
    if (M < 1 || N < 16 || N % 16 || K < kGS || K % kGS)
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need M >= 1, N % 16 == 0 and K % 128 == 0");
    if ((size_t)(K / 16) * N * 4 >= 0x80000000u) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "B must be below 2^31 bytes");
    return int2_gemv_stream_probe_run(dtype, B, S, C, M, N, K, (hipStream_t)stream);
}

int ternocl_ldsa(int M) { return (M + 31) & ~31; }

ternocl_status ternocl_quant_a(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K,
                               void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!A || !SA) FAIL(TERNOCL_ERR_INVALID_ARG, "A and SA must be non-null");
    if (M < 1 || K < kGS || K % kGS) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need M >= 1 and K % 128 == 0");
    return quant_a_run(dtype, A, SA, Aq, M, K, (hipStream_t)stream);
}

ternocl_status ternocl_int2_int8_gemm_ws(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                         const uint32_t *B, const void *SB, void *C, const void *Other,
                                         const void *Bias, int M, int N, int K, int postop, int out_f32, void *ws,
                                         size_t ws_bytes, void *stream) {
    if (!Aq && !A) FAIL(TERNOCL_ERR_INVALID_ARG, "Aq (upfront quantization) or A (in-GEMM quantization) must be non-null");
    ternocl_status s = check_gemm_common(dtype, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32);
    if (s != TERNOCL_OK) return s;
    if (int2_int8_gemv_supports(M, N, K, A, Aq))  // decode: the fp8 x fp4 block-scaled GEMV
        return int2_int8_gemv_run(dtype, A, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32,
                                  (hipStream_t)stream, ws, ws_bytes);
    return int2_int8_gemm_run(dtype, A, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32,
                              (hipStream_t)stream, ws, ws_bytes);
}

ternocl_status ternocl_int2_int8_gemm(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                      const uint32_t *B, const void *SB, void *C,
                                      const void *Other, const void *Bias, int M, int N, int K,
                                      int postop, int out_f32, void *stream) {
    return ternocl_int2_int8_gemm_ws(dtype, A, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, nullptr, 0,
                                     stream);
}

size_t ternocl_int2_int8_gemm_ws_bytes(int M, int N, int K) {
    if (M < 1 || N < 16 || N % 16 || K < kGS || K % kGS) return 0;
    if (M <= 4) return int2_int8_gemv_ws_need(M, N, K);  // the decode GEMV's K split
    return int2_gemm_ws_need(M, N, K);
}

ternocl_status ternocl_int2_s8_decode(const uint32_t *B, uint32_t *D, int K, int N, void *stream) {
    if (!B || !D) FAIL(TERNOCL_ERR_INVALID_ARG, "B and D must be non-null");
    if (N < 16 || N % 16 || K < 16 || K % 16) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % 16 == 0");
    return int2_s8_decode_run(B, D, K, N, (hipStream_t)stream);
}

ternocl_status ternocl_bitcos_fp16_upcvt_gemm_ws(int dtype, const void *A, const uint32_t *B,
                                                 const void *S, const uint32_t *SR, int ls, void *C,
                                                 const void *Other, const void *Bias, int M, int N,
                                                 int K, int postop, int out_f32, void *ws, size_t ws_bytes,
                                                 void *stream) {
    ternocl_status s = check_gemm_common(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32);
    if (s != TERNOCL_OK) return s;
    if (ls < 1 || ls > bitcos_max_ls()) FAIL(TERNOCL_ERR_INVALID_ARG, "ls must be 1..16");
    if (K % (64 * ls)) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "BITCOS needs K % (64 * ls) == 0");
    if (ls > 1 && !SR) FAIL(TERNOCL_ERR_INVALID_ARG, "SR (slice ranks for ls slices) must be non-null when ls > 1");
    return bitcos_gemv_run(dtype, A, B, S, SR, ls, C, Other, Bias, M, N, K, postop, out_f32,
                           (hipStream_t)stream, ws, ws_bytes);
}

ternocl_status ternocl_bitcos_fwht_gemm_ws(int dtype, const void *x, const int8_t *signs, int HB, int use_signs,
                                          const uint32_t *B, const void *S, const uint32_t *SR, int ls, void *C,
                                          const void *Other, const void *Bias, int M, int N, int K, int postop,
                                          int out_f32, void *ws, size_t ws_bytes, void *stream) {
    ternocl_status s = check_gemm_common(dtype, x, B, S, C, Other, Bias, M, N, K, postop, out_f32);
    if (s != TERNOCL_OK) return s;
    if (ls < 1 || ls > bitcos_max_ls()) FAIL(TERNOCL_ERR_INVALID_ARG, "ls must be 1..16");
    if (K % (64 * ls)) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "BITCOS needs K % (64 * ls) == 0");
    if (ls > 1 && !SR) FAIL(TERNOCL_ERR_INVALID_ARG, "SR (slice ranks for ls slices) must be non-null when ls > 1");
    if (use_signs && !signs) FAIL(TERNOCL_ERR_INVALID_ARG, "use_signs needs a signs vector");
    if (HB < 256 || HB > 512 || (HB & (HB - 1)))
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the fused transform takes HB 256 or 512 (one wave per block)");
    const int tail = K % HB;
    if ((tail & (tail - 1)) || (tail && tail < 8))
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the fused transform takes K % HB of 0 or a power of two >= 8");
    if (((uintptr_t)x & 15) || (use_signs && ((uintptr_t)signs & 7)))
        FAIL(TERNOCL_ERR_INVALID_ARG, "the fused transform reads x 16-byte and signs 8-byte aligned");
    const float full = (float)(1.0 / std::sqrt((double)HB));
    const float part = tail ? (float)(1.0 / std::sqrt((double)tail)) : full;
    return bitcos_fwht_gemv_run(dtype, x, signs, HB, use_signs ? 1 : 0, full, part, B, S, SR, ls, C, Other, Bias,
                                M, N, K, postop, out_f32, (hipStream_t)stream, ws, ws_bytes);
}

ternocl_status ternocl_bitcos_fp16_upcvt_gemm(int dtype, const void *A, const uint32_t *B,
                                              const void *S, const uint32_t *SR, int ls, void *C,
                                              const void *Other, const void *Bias, int M, int N,
                                              int K, int postop, int out_f32, void *stream) {
    return ternocl_bitcos_fp16_upcvt_gemm_ws(dtype, A, B, S, SR, ls, C, Other, Bias, M, N, K, postop, out_f32,
                                             nullptr, 0, stream);
}

size_t ternocl_bitcos_gemv_ws_bytes(int N, int ls) {
    if (N < 16 || N % 16 || ls < 1 || ls > bitcos_max_ls()) return 0;
    return bitcos_gemv_ws_need(N, ls);
}

static ternocl_status check_bitcos_slices(int N, int K, int ls, const uint32_t *SR) {
    if (ls < 1 || ls > bitcos_max_ls()) FAIL(TERNOCL_ERR_INVALID_ARG, "ls must be 1..16");
    if (N < 16 || N % 16 || K < 64 || K % (64 * ls)) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % (64 * ls) == 0");
    if (ls > 1 && !SR) FAIL(TERNOCL_ERR_INVALID_ARG, "SR (slice ranks for ls slices) must be non-null when ls > 1");
    return TERNOCL_OK;
}

size_t ternocl_bitcos_gemm_mt_ws_bytes(int K, int N) {
    if (K < 16 || N < 1) return 0;
    return kWsHeader + (size_t)(K / 16) * (size_t)N * 4;  // the header, then the re-packed words
}

ternocl_status ternocl_bitcos_to_int2(const uint32_t *B, const uint32_t *SR, int ls, uint32_t *W2, int K,
                                      int N, void *stream) {
    if (!B || !W2) FAIL(TERNOCL_ERR_INVALID_ARG, "B and W2 must be non-null");
    ternocl_status s = check_bitcos_slices(N, K, ls, SR);
    if (s != TERNOCL_OK) return s;
    return bitcos_to_int2_run(B, SR, ls, W2, N, K, (hipStream_t)stream);
}

ternocl_status ternocl_bitcos_fp16_upcvt_gemm_mt(int dtype, const void *A, const uint32_t *B,
                                                 const void *S, const uint32_t *SR, int ls, void *C,
                                                 const void *Other, const void *Bias, int M, int N,
                                                 int K, int postop, int out_f32, void *ws,
                                                 size_t ws_bytes, void *stream) {
    ternocl_status s = check_gemm_common(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32);
    if (s != TERNOCL_OK) return s;
    if ((s = check_bitcos_slices(N, K, ls, SR)) != TERNOCL_OK) return s;
    if (!ws) {  // the tiles decode the BITCOS weights themselves
        if ((size_t)M * K * 2 >= kMaxBufBytes)
            FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the M-tiled BITCOS GEMM takes A below 2^31 bytes");
        return bitcos_gemm_mt_run(dtype, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, (hipStream_t)stream);
    }
    const size_t need = ternocl_bitcos_gemm_mt_ws_bytes(K, N);
    if (ws_bytes < need) FAIL(TERNOCL_ERR_WORKSPACE, "ws must hold ternocl_bitcos_gemm_mt_ws_bytes(K, N) bytes");
    if (((uintptr_t)ws & 15) != 0) FAIL(TERNOCL_ERR_INVALID_ARG, "ws must be 16-byte aligned");
    if (need - kWsHeader >= kMaxBufBytes || (size_t)M * K * 2 >= kMaxBufBytes)
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the M-tiled BITCOS path takes A and the re-packed weights below 2^31 bytes");
    const hipStream_t st = (hipStream_t)stream;
    uint32_t *W2 = (uint32_t *)((uint8_t *)ws + kWsHeader);
    if ((s = bitcos_to_int2_run(B, SR, ls, W2, N, K, st)) != TERNOCL_OK) return s;
    return int2_gemm_mfma_run(dtype, A, W2, S, C, Other, Bias, M, N, K, postop, out_f32, st);
}

ternocl_status ternocl_bitcos_slice_ranks(const uint32_t *B, uint32_t *SR, int K, int N, int ls,
                                          void *stream) {
    if (!B) FAIL(TERNOCL_ERR_INVALID_ARG, "B must be non-null");
    if (ls < 1 || ls > bitcos_max_ls()) FAIL(TERNOCL_ERR_INVALID_ARG, "ls must be 1..16");
    if (N < 16 || N % 16 || K < 64 || K % (64 * ls)) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % (64 * ls) == 0");
    if (ls == 1) return TERNOCL_OK;
    if (!SR) FAIL(TERNOCL_ERR_INVALID_ARG, "SR must be non-null");
    return bitcos_slice_ranks_run(B, SR, N, K, ls, (hipStream_t)stream);
}

int ternocl_bitcos_pick_ls(int M, int N, int K) {
    (void)M;
    if (N < 1 || K < 64) return 1;
    return bitcos_pick_ls(N, K);
}

ternocl_status ternocl_bitcos_dequant(int dtype, const uint32_t *B, const void *S, void *W, int K,
                                      int N, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!B || !S || !W) FAIL(TERNOCL_ERR_INVALID_ARG, "B, S and W must be non-null");
    if (N < 16 || N % 16 || K < kGS || K % kGS) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need N % 16 == 0 and K % 128 == 0");
    return bitcos_dequant_run(dtype, B, S, W, N, K, (hipStream_t)stream);
}

ternocl_status ternocl_hadamard_fwht(int dtype, const void *x, const int8_t *signs, void *y,
                                     int rows, int K, int HB, int use_signs, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!x || !y) FAIL(TERNOCL_ERR_INVALID_ARG, "x and y must be non-null");
    if (use_signs && !signs) FAIL(TERNOCL_ERR_INVALID_ARG, "use_signs needs a signs vector");
    if (HB < 256 || HB > 4096 || (HB & (HB - 1))) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "HB must be a power of two in [256, 4096]");
    if (rows < 1 || K < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "rows and K must be positive");
    const int tail = K % HB;
    if (tail & (tail - 1)) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "K % HB must be 0 or a power of two");
    const float full = (float)(1.0 / std::sqrt((double)HB));
    const float part = tail ? (float)(1.0 / std::sqrt((double)tail)) : full;
    return fwht_run(dtype, x, signs, y, rows, K, HB, use_signs ? 1 : 0, full, part, (hipStream_t)stream);
}

constexpr int kMoeMaxExperts = 512;  // route LDS: 18 ints per expert (36 KiB)

int ternocl_moe_tile_rows(void) { return moe_tile_rows(); }

ternocl_status ternocl_int2_moe_route(const int *ids, int *meta, int *perm, int *inv, int G, int E,
                                      void *stream) {
    if (!ids || !meta || !perm || !inv) FAIL(TERNOCL_ERR_INVALID_ARG, "ids, meta, perm and inv must be non-null");
    if (G < 1 || E < 1 || E > kMoeMaxExperts) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need G >= 1 and 1 <= E <= 512");
    return moe_route_run(ids, meta, perm, inv, G, E, (hipStream_t)stream);
}

ternocl_status ternocl_int2_moe_gather(int dtype, const void *X, const int *perm, void *Xs, int G,
                                       int K, int topk, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!X || !perm || !Xs) FAIL(TERNOCL_ERR_INVALID_ARG, "X, perm and Xs must be non-null");
    if (G < 1 || K < 1 || topk < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need G, K, topk >= 1");
    return moe_gather_run(X, perm, Xs, G, K, topk, (hipStream_t)stream);
}

ternocl_status ternocl_int2_moe_gemm(int dtype, const int *meta, const void *A_all, const int *perm,
                                     int topk, const uint32_t *B_all, const void *S_all, void *C_all,
                                     const void *Other_all, int E, int G, int N, int K, int postop,
                                     int out_f32, void *stream) {
    ternocl_status s = check_gemm_common(dtype, A_all, B_all, S_all, C_all, Other_all, nullptr, G, N, K,
                                         postop == 3 || postop == 5 ? 0 : postop, out_f32);
    if (s != TERNOCL_OK) return s;
    if (!meta) FAIL(TERNOCL_ERR_INVALID_ARG, "meta must be non-null");
    if (postop == 3 || postop == 5) FAIL(TERNOCL_ERR_INVALID_ARG, "the MoE GEMM has no bias: postop 0, 1, 2 or 4");
    if (E < 1 || E > kMoeMaxExperts || topk < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need 1 <= E <= 512 and topk >= 1");
    if ((size_t)(perm ? G / topk : G) * (size_t)K * 2 >= kMaxBufBytes || (size_t)(K / 16) * (size_t)N * 4 >= kMaxBufBytes)
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the A rows and each expert's packed weights must be below 2^31 bytes");
    return moe_gemm_run(dtype, meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop,
                        out_f32, (hipStream_t)stream);
}

ternocl_status ternocl_int2_moe_combine(int dtype, const float *Y, const int *inv, const void *RW,
                                        void *O, int T, int topk, int N, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!Y || !inv || !RW || !O) FAIL(TERNOCL_ERR_INVALID_ARG, "Y, inv, RW and O must be non-null");
    if (T < 1 || topk < 1 || N < 4 || N % 4) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need T, topk >= 1 and N % 4 == 0");
    return moe_combine_run(dtype, Y, inv, RW, O, T, topk, N, (hipStream_t)stream);
}

size_t ternocl_int2_moe_prefill_ws_bytes(int T, int E, int topk, int H, int I) {
    if (T < 1 || E < 1 || topk < 1 || H < 1 || I < 1) return 0;
    return moe_ws_layout(T, E, topk, H, I).total;
}

ternocl_status ternocl_int2_moe_prefill(int dtype, const void *X, const int *ids, const void *RW,
                                        int T, int E, int topk, int H, int I, const uint32_t *Bg,
                                        const void *Sg, const uint32_t *Bu, const void *Su,
                                        const uint32_t *Bd, const void *Sd, void *O, void *ws,
                                        size_t ws_bytes, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!X || !ids || !RW || !Bg || !Sg || !Bu || !Su || !Bd || !Sd || !O)
        FAIL(TERNOCL_ERR_INVALID_ARG, "X, ids, RW, the six weight tensors and O must be non-null");
    if (T < 1 || E < 1 || E > kMoeMaxExperts || topk < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need T, topk >= 1 and 1 <= E <= 512");
    if (H % 128 || I % 128) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "H and I must be multiples of 128");
    {
        const size_t G = (size_t)T * topk;
        if ((size_t)T * H * 2 >= kMaxBufBytes || G * I * 2 >= kMaxBufBytes ||
            (size_t)(H / 16) * I * 4 >= kMaxBufBytes || (size_t)(I / 16) * H * 4 >= kMaxBufBytes)
            FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE,
                 "X (T * H * 2 bytes), the expert-sorted rows (T * topk * I * 2) and each expert's packed weights must be below 2^31 bytes");
    }
    if (!ws || ws_bytes < moe_ws_layout(T, E, topk, H, I).total)
        FAIL(TERNOCL_ERR_WORKSPACE, "ws must hold ternocl_int2_moe_prefill_ws_bytes() bytes");
    return moe_prefill_run(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws, (hipStream_t)stream);
}

size_t ternocl_int2_moe_prefill_int8_ws_bytes(int T, int E, int topk, int H, int I) {
    if (T < 1 || E < 1 || topk < 1 || H < 1 || I < 1) return 0;
    return moe_i8_ws_layout(T, E, topk, H, I).total;
}

ternocl_status ternocl_int2_moe_prefill_int8(int dtype, const void *X, const int *ids, const void *RW,
                                             int T, int E, int topk, int H, int I, const uint32_t *Bg,
                                             const void *Sg, const uint32_t *Bu, const void *Su,
                                             const uint32_t *Bd, const void *Sd, void *O, void *ws,
                                             size_t ws_bytes, void *stream) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!X || !ids || !RW || !Bg || !Sg || !Bu || !Su || !Bd || !Sd || !O)
        FAIL(TERNOCL_ERR_INVALID_ARG, "X, ids, RW, the six weight tensors and O must be non-null");
    if (T < 1 || E < 1 || E > kMoeMaxExperts || topk < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need T, topk >= 1 and 1 <= E <= 512");
    if (H % 128 || I % 128) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "H and I must be multiples of 128");
    if (int8_moe_tile_rows() != moe_tile_rows()) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "int8 tile rows differ from the route's");
    const size_t G = (size_t)T * topk;
    if (G * H * 4 >= kMaxBufBytes || G * I * 2 >= kMaxBufBytes || (size_t)(H / 16) * I * 4 >= kMaxBufBytes ||
        (size_t)(I / 16) * H * 4 >= kMaxBufBytes)
        FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "the gathered rows and each expert's weights must be below 2^31 bytes");
    if (!ws || ws_bytes < moe_i8_ws_layout(T, E, topk, H, I).total)
        FAIL(TERNOCL_ERR_WORKSPACE, "ws must hold ternocl_int2_moe_prefill_int8_ws_bytes() bytes");
    return moe_prefill_int8_run(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws,
                                (hipStream_t)stream);
}

size_t ternocl_int2_moe_decode_ws_bytes(int T, int topk, int H, int I) {
    if (T < 1 || topk < 1 || H < 1 || I < 1) return 0;
    return moe_decode_ws_bytes(T, topk, H, I);
}

static ternocl_status check_moe_decode(int dtype, const void *X, const int *ids, const void *RW, int T, int E,
                                       int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                       const uint32_t *Bu, const void *Su, const uint32_t *Bd, const void *Sd,
                                       const void *O) {
    ternocl_status s = check_dtype(dtype);
    if (s != TERNOCL_OK) return s;
    if (!X || !ids || !RW || !Bg || !Sg || !Bu || !Su || !Bd || !Sd || !O)
        FAIL(TERNOCL_ERR_INVALID_ARG, "X, ids, RW, the six weight tensors and O must be non-null");
    if (T < 1 || E < 1 || topk < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need T, E, topk >= 1");
    if (H % 128 || I % 128) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "H and I must be multiples of 128");
    if ((size_t)T * topk > 32767) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "T * topk must be below 32768 (decode)");
    if (((uintptr_t)X & 15) != 0) FAIL(TERNOCL_ERR_INVALID_ARG, "X must be 16-byte aligned");
    return TERNOCL_OK;
}

ternocl_status ternocl_int2_moe_decode(int dtype, const void *X, const int *ids, const void *RW, int T,
                                       int E, int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                       const uint32_t *Bu, const void *Su, const uint32_t *Bd,
                                       const void *Sd, void *O, void *ws, size_t ws_bytes, void *stream) {
    ternocl_status s = check_moe_decode(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O);
    if (s != TERNOCL_OK) return s;
    if (!ws || ws_bytes < moe_decode_ws_bytes(T, topk, H, I))
        FAIL(TERNOCL_ERR_WORKSPACE, "ws must hold ternocl_int2_moe_decode_ws_bytes() bytes");
    if (((uintptr_t)ws & 255) != 0) FAIL(TERNOCL_ERR_INVALID_ARG, "ws must be 256-byte aligned");
    return moe_decode_run(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O, ws, (hipStream_t)stream);
}

ternocl_status ternocl_int2_moe_decode_noalloc(int dtype, const void *X, const int *ids, const void *RW, int T,
                                               int E, int topk, int H, int I, const uint32_t *Bg,
                                               const void *Sg, const uint32_t *Bu, const void *Su,
                                               const uint32_t *Bd, const void *Sd, void *O, void *stream) {
    ternocl_status s = check_moe_decode(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O);
    if (s != TERNOCL_OK) return s;
    if (moe_decode_ws_bytes(T, topk, H, I) > kNoAllocScratchBytes)
        FAIL(TERNOCL_ERR_WORKSPACE, "this layer needs more scratch than the allocation-free entry holds "
                                    "(ternocl_int2_moe_decode_ws_bytes() > TERNOCL_NOALLOC_SCRATCH_BYTES, 16 MiB): "
                                    "call ternocl_int2_moe_decode with a workspace");
    return moe_decode_noalloc_run(dtype, X, ids, RW, T, E, topk, H, I, Bg, Sg, Bu, Su, Bd, Sd, O,
                                  (hipStream_t)stream);
}

}  // extern "C"
