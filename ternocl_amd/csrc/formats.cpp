// formats.cpp -- host (CPU) packers of the weight formats, so that a C, Go or
// Rust caller of include/ternocl_amd.h can produce the buffers the kernels
// read from dense ternary weights (int8 [K, N], row-major, values -1, 0, +1):
//   * int2: word (kp, n) bits 2j..2j+1 = code of row 16 kp + j, codes 0, 1, 3
//     for 0, +1, -1 (int2_fp16_upcvt/int2_fp16_upcvt.cl:6-19, the generator of
//     int2_fp16_upcvt/main.cpp:238-242 draws the same codes);
//   * BITCOS (common/bitcos.hpp:1-8): presence bitmap [K/32][N] (bit c of word
//     (kp, n) = weight (32 kp + c, n) != 0), per-column offsets of the sign
//     streams, the sign streams (one bit per non-zero in k order, 1 = -1,
//     column after column, each padded to whole words with zeros) and 4 zero
//     pad words; slice ranks [ls-1][N] = non-zeros of column n in the bitmap
//     words below s * ceil(K / ls) / 32 (common/bitcos.hpp:81-94).
// Nothing here touches the GPU.
#include <cstdint>
#include <cstring>
#include <vector>

#include "common.hpp"

namespace {

using tcl::set_error;

constexpr size_t kBitcosPadWords = 4;

#define FAIL(code, msg)    \
    do {                   \
        set_error(msg);    \
        return code;       \
    } while (0)

// Code of a ternary value, or -1 for a value outside {-1, 0, +1}.
inline int code_of(int8_t v) { return v == 0 ? 0 : v == 1 ? 1 : v == -1 ? 3 : -1; }

bool ternary(const int8_t *W, size_t n) {
    for (size_t i = 0; i < n; ++i)
        if (W[i] < -1 || W[i] > 1) return false;
    return true;
}

// Non-zeros per column and the presence bitmap (row-major pass).
void bitcos_presence(const int8_t *W, int K, int N, uint32_t *bitmap, std::vector<uint32_t> &nnz) {
    nnz.assign((size_t)N, 0u);
    std::memset(bitmap, 0, (size_t)K / 32 * N * sizeof(uint32_t));
    for (int k = 0; k < K; ++k) {
        const int8_t *row = W + (size_t)k * N;
        uint32_t *bw = bitmap + (size_t)(k / 32) * N;
        const uint32_t bit = 1u << (k % 32);
        for (int n = 0; n < N; ++n)
            if (row[n] != 0) {
                bw[n] |= bit;
                ++nnz[n];
            }
    }
}

}  // namespace

extern "C" {

ternocl_status ternocl_int2_pack(const int8_t *W, uint32_t *B, int K, int N) {
    if (!W || !B) FAIL(TERNOCL_ERR_INVALID_ARG, "W and B must be non-null");
    if (K < 16 || K % 16 || N < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need K % 16 == 0 and N >= 1");
    if (!ternary(W, (size_t)K * N)) FAIL(TERNOCL_ERR_INVALID_ARG, "W holds a value outside {-1, 0, +1}");
    for (int kp = 0; kp < K / 16; ++kp) {
        uint32_t *out = B + (size_t)kp * N;
        for (int n = 0; n < N; ++n) out[n] = 0u;
        for (int j = 0; j < 16; ++j) {
            const int8_t *row = W + (size_t)(16 * kp + j) * N;
            for (int n = 0; n < N; ++n) out[n] |= (uint32_t)code_of(row[n]) << (2 * j);
        }
    }
    return TERNOCL_OK;
}

ternocl_status ternocl_int2_unpack(const uint32_t *B, int8_t *W, int K, int N) {
    if (!W || !B) FAIL(TERNOCL_ERR_INVALID_ARG, "W and B must be non-null");
    if (K < 16 || K % 16 || N < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need K % 16 == 0 and N >= 1");
    // the 2-bit two's complement value: code 2 (outside the format) reads as -2,
    // as code_to_value does (int2_fp16_upcvt/main.cpp:76)
    static const int8_t val[4] = {0, 1, -2, -1};
    for (int k = 0; k < K; ++k) {
        const uint32_t *in = B + (size_t)(k / 16) * N;
        int8_t *row = W + (size_t)k * N;
        const int sh = 2 * (k % 16);
        for (int n = 0; n < N; ++n) row[n] = val[(in[n] >> sh) & 3u];
    }
    return TERNOCL_OK;
}

size_t ternocl_bitcos_pack_words(const int8_t *W, int K, int N) {
    if (!W || K < 32 || K % 32 || N < 1 || !ternary(W, (size_t)K * N)) return 0;
    std::vector<uint32_t> nnz((size_t)N, 0u);
    for (int k = 0; k < K; ++k) {
        const int8_t *row = W + (size_t)k * N;
        for (int n = 0; n < N; ++n) nnz[n] += row[n] != 0;
    }
    size_t signs = 0;
    for (int n = 0; n < N; ++n) signs += (nnz[n] + 31) / 32;
    return (size_t)K / 32 * N + N + signs + kBitcosPadWords;
}

ternocl_status ternocl_bitcos_pack(const int8_t *W, int K, int N, uint32_t *buf, size_t words) {
    if (!W || !buf) FAIL(TERNOCL_ERR_INVALID_ARG, "W and buf must be non-null");
    if (K < 32 || K % 32 || N < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need K % 32 == 0 and N >= 1");
    if (!ternary(W, (size_t)K * N)) FAIL(TERNOCL_ERR_INVALID_ARG, "W holds a value outside {-1, 0, +1}");
    const size_t bw = (size_t)K / 32 * N;
    std::vector<uint32_t> nnz;
    std::vector<uint32_t> bitmap(bw);
    bitcos_presence(W, K, N, bitmap.data(), nnz);
    size_t signs = 0;
    std::vector<uint32_t> off((size_t)N);
    for (int n = 0; n < N; ++n) {
        if (signs > 0xffffffffu) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "sign streams beyond 2^32 words");
        off[n] = (uint32_t)signs;
        signs += (nnz[n] + 31) / 32;
    }
    const size_t total = bw + N + signs + kBitcosPadWords;
    if (words < total) FAIL(TERNOCL_ERR_INVALID_ARG, "buf is shorter than ternocl_bitcos_pack_words");
    std::memcpy(buf, bitmap.data(), bw * sizeof(uint32_t));
    std::memcpy(buf + bw, off.data(), (size_t)N * sizeof(uint32_t));
    uint32_t *sg = buf + bw + N;
    std::memset(sg, 0, (signs + kBitcosPadWords) * sizeof(uint32_t));
    // sign bits in k order per column: one rank cursor per column, rows in order
    std::vector<uint32_t> rank((size_t)N, 0u);
    for (int k = 0; k < K; ++k) {
        const int8_t *row = W + (size_t)k * N;
        for (int n = 0; n < N; ++n) {
            if (row[n] == 0) continue;
            const uint32_t r = rank[n]++;
            if (row[n] < 0) sg[off[n] + r / 32] |= 1u << (r % 32);
        }
    }
    return TERNOCL_OK;
}

ternocl_status ternocl_bitcos_unpack(const uint32_t *buf, size_t words, int K, int N, int8_t *W) {
    if (!W || !buf) FAIL(TERNOCL_ERR_INVALID_ARG, "W and buf must be non-null");
    if (K < 32 || K % 32 || N < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need K % 32 == 0 and N >= 1");
    const size_t bw = (size_t)K / 32 * N;
    if (words < bw + N + kBitcosPadWords) FAIL(TERNOCL_ERR_INVALID_ARG, "buf is too short for K x N");
    const uint32_t *off = buf + bw, *sg = buf + bw + N;
    std::vector<uint32_t> rank((size_t)N, 0u);
    for (int k = 0; k < K; ++k) {
        const uint32_t *bm = buf + (size_t)(k / 32) * N;
        const uint32_t bit = 1u << (k % 32);
        int8_t *row = W + (size_t)k * N;
        for (int n = 0; n < N; ++n) {
            if (!(bm[n] & bit)) {
                row[n] = 0;
                continue;
            }
            const size_t w = (size_t)off[n] + rank[n] / 32;
            if (bw + N + w >= words) FAIL(TERNOCL_ERR_INVALID_ARG, "a sign stream runs past buf's end");
            row[n] = ((sg[w] >> (rank[n] % 32)) & 1u) ? -1 : 1;
            ++rank[n];
        }
    }
    return TERNOCL_OK;
}

ternocl_status ternocl_bitcos_slice_ranks_host(const uint32_t *buf, int K, int N, int ls, uint32_t *SR) {
    if (!buf || (ls > 1 && !SR)) FAIL(TERNOCL_ERR_INVALID_ARG, "buf and SR must be non-null");
    if (K < 32 || K % 32 || N < 1) FAIL(TERNOCL_ERR_UNSUPPORTED_SHAPE, "need K % 32 == 0 and N >= 1");
    if (ls < 1) FAIL(TERNOCL_ERR_INVALID_ARG, "ls must be >= 1");
    const int slice_k = (K + ls - 1) / ls;
    std::vector<uint32_t> run((size_t)N, 0u);
    int kp = 0;
    for (int s = 1; s < ls; ++s) {
        for (; kp < s * slice_k / 32; ++kp) {
            const uint32_t *bm = buf + (size_t)kp * N;
            for (int n = 0; n < N; ++n) run[n] += (uint32_t)__builtin_popcount(bm[n]);
        }
        std::memcpy(SR + (size_t)(s - 1) * N, run.data(), (size_t)N * sizeof(uint32_t));
    }
    return TERNOCL_OK;
}

}  // extern "C"
