/*
 * ternocl_oracle.c -- CPU restatement of TernOCL's host reference numerics.
 *
 * TEST INFRASTRUCTURE ONLY: results of the HIP library are checked against it.  Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.
 *
 * Built with gcc -O2 -fopenmp -ffp-contract=off and no -march flags, so that
 * every fp32 multiply and add rounds separately, in the order the reference's
 * loops give them (the reference host code is built the same way: no FMA
 * contraction on baseline x86-64).  OpenMP only splits independent outputs;
 * each output is a sequential loop, so results do not depend on the thread count.
 *
 * Parity pins (tests/test_oracle.py, tests/test_oracle_vs_ref.py):
 *   orc_tof / orc_fromf     exhaustive over all 65,536 codes against the compiled
 *                           reference dt16.hpp (oracle/_ref) and the IEEE closed
 *                           form; rounding ties / overflow / subnormals / NaN.
 *   orc_int2_gold           bit-identical to the compiled reference compute_gold
 *                           (int2_fp16_upcvt/main.cpp:79-98); brute-force dense
 *                           float64 product within fp32 rounding.
 *   orc_int2_dequant        closed form (+s, s^0x8000, 0), exhaustive over codes.
 *   orc_epilogue            bit-identical to the compiled epilogue_ref for
 *                           postop 0..4 x {DT, fp32}; postop 5 (bias + residual,
 *                           no single reference postop) bit-identical to the
 *                           compiled epilogue_ref run twice: postop 3 into fp32,
 *                           then postop 2 into the output type.
 *   orc_scale_a/quant_a     bit-identical to the compiled compute_scale_a and the
 *                           lrintf quantization for finite products; closed-form
 *                           checks (RTE ties, saturation, FLT_EPSILON floor).
 *                           Infinite / NaN products (fp16 SA = inf) follow the
 *                           reference device kernel's saturating conversion
 *                           (closed-form test), not the host's undefined lrintf.
 *   orc_int8_gold           bit-identical to the compiled compute_gold
 *                           (int2_via_int2_x_int8_dpas/main.cpp:94-121).
 *   orc_bitcos_*            pack/decode round trip; slice ranks and decode and
 *                           gold bit-identical to the compiled bitcos.hpp and
 *                           bitcos_fp16_upcvt/main.cpp:64-86 on the same buffers.
 *   orc_fwht                Sylvester-matrix brute force (float64) for small HB,
 *                           involution H*H = I, stage-order restatement of
 *                           hadamard_fwht.cl (no reference host code exists; the
 *                           K % HB tail block is an extension, parity unpinned).
 *   orc_moe_*               route: permutation invariants and brute force;
 *                           combine: closed form; token check: restated from
 *                           int2_moe/prefill.cpp:288-319 (pinned by brute force
 *                           against a dense float64 evaluation).
 */
#include "ternocl_oracle.h"

#include <float.h>
#include <math.h>
#include <omp.h>
#include <stdlib.h>
#include <string.h>

#define GS 128

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* ---- DT conversions: common/dt16.hpp:18-42 ---------------------------- */

float orc_tof(uint16_t h, int bf16) {
    if (bf16) return u2f((uint32_t)h << 16);
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    const uint32_t e = (h >> 10) & 0x1fu, m = h & 0x3ffu;
    if (e == 0) {
        /* zero or subnormal: m * 2^-24 is exact in fp32 */
        const float v = (float)m * 5.9604644775390625e-08f;
        return u2f(f2u(v) | sign);
    }
    if (e == 31) return u2f(sign | 0x7f800000u | (m << 13));
    return u2f(sign | ((e + 112u) << 23) | (m << 13));
}

uint16_t orc_fromf(float f, int bf16) {
    uint32_t u = f2u(f);
    if (bf16) {
        if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u); /* NaN */
        u += 0x7fffu + ((u >> 16) & 1u);
        return (uint16_t)(u >> 16);
    }
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7fffffffu;
    if (a > 0x7f800000u) /* NaN: quiet, payload truncated */
        return (uint16_t)(sign | 0x7e00u | ((a >> 13) & 0x3ffu));
    if (a >= 0x47800000u) return (uint16_t)(sign | 0x7c00u); /* >= 65536 (and inf) */
    if (a < 0x38800000u) {                                   /* below 2^-14 */
        if (a <= 0x33000000u) return (uint16_t)sign;         /* <= 2^-25: ties to 0 */
        const float v = u2f(a) * 16777216.0f;                /* exact scaling by 2^24 */
        return (uint16_t)(sign | (uint32_t)rintf(v));        /* RTE (default mode) */
    }
    uint32_t h = ((((a >> 23) - 112u) << 10) | ((a & 0x7fffffu) >> 13));
    const uint32_t rem = a & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) ++h; /* carries into the exponent */
    return (uint16_t)(sign | h);
}

void orc_tof_n(const uint16_t *h, float *f, size_t n, int bf16) {
#pragma omp parallel for
    for (long long i = 0; i < (long long)n; ++i) f[i] = orc_tof(h[i], bf16);
}

void orc_fromf_n(const float *f, uint16_t *h, size_t n, int bf16) {
#pragma omp parallel for
    for (long long i = 0; i < (long long)n; ++i) h[i] = orc_fromf(f[i], bf16);
}

/* ---- int2 format and gold: int2_fp16_upcvt/main.cpp:76-98 ------------- */

int orc_code_to_value(uint32_t c) { return (int)(int8_t)((int8_t)(c << 6) >> 6); }

void orc_int2_gold(int bf16, const uint16_t *A, const uint32_t *B, const uint16_t *S, float *C,
                   int M, int K, int N) {
    const int groups = K / GS;
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int g = 0; g < groups; ++g) {
                float partial = 0.0f;
                for (int p = 0; p < GS; ++p) {
                    const int ik = g * GS + p;
                    const uint32_t code = (B[(size_t)(ik / 16) * N + j] >> (2 * (ik % 16))) & 3u;
                    const int bv = orc_code_to_value(code);
                    if (bv) partial += orc_tof(A[(size_t)i * K + ik], bf16) * (float)bv;
                }
                acc += partial * orc_tof(S[(size_t)g * N + j], bf16);
            }
            C[(size_t)i * N + j] = acc;
        }
}

/* int2_fp16_upcvt.cl:95-116 (INT_DQ) and :118-150 (select): code 1 -> +s,
 * code 3 -> s with the sign bit flipped, code 0 -> +0.  Code 2 tests only the
 * low bit on the device and gives +0 here too (the codes contract is {0,1,3}). */
void orc_int2_dequant(const uint32_t *B, const uint16_t *S, uint16_t *W, int K, int N) {
#pragma omp parallel for schedule(static)
    for (int k = 0; k < K; ++k)
        for (int n = 0; n < N; ++n) {
            const uint32_t c = (B[(size_t)(k / 16) * N + n] >> (2 * (k % 16))) & 3u;
            const uint16_t s = S[(size_t)(k / GS) * N + n];
            W[(size_t)k * N + n] = (c & 1u) ? (uint16_t)(s ^ ((c & 2u) ? 0x8000u : 0u)) : 0u;
        }
}

/* ---- epilogue: common/epilogue.hpp:82, :98-115 ------------------------ */

float orc_sigmoid(float x) { return x <= -10.0f ? 0.0f : 1.0f / (expf(-x) + 1.0f); }

void orc_epilogue(int bf16, int postop, int out_f32, const float *acc, const uint16_t *other,
                  const void *bias, void *out, int M, int N) {
    const unsigned char *bb = (const unsigned char *)bias;
    unsigned char *o = (unsigned char *)out;
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)M * N; ++i) {
        float v = acc[i];
        const int n = (int)(i % N);
        float b = 0.0f;
        if (postop == 3 || postop == 5) {
            if (out_f32) memcpy(&b, bb + 4 * (size_t)n, 4);
            else { uint16_t h; memcpy(&h, bb + 2 * (size_t)n, 2); b = orc_tof(h, bf16); }
        }
        if (postop == 1) v = v * orc_sigmoid(v) * orc_tof(other[i], bf16);
        else if (postop == 2) v += orc_tof(other[i], bf16);
        else if (postop == 3) v += b;
        else if (postop == 4) v = orc_sigmoid(v);
        else if (postop == 5) { v += b; v += orc_tof(other[i], bf16); }
        if (out_f32) memcpy(o + 4 * (size_t)i, &v, 4);
        else { const uint16_t h = orc_fromf(v, bf16); memcpy(o + 2 * (size_t)i, &h, 2); }
    }
}

/* ---- int8 path: int2_via_int2_x_int8_dpas/main.cpp:79-121 ------------- */

int orc_ldsa(int M) { return (M + 31) & ~31; }

void orc_scale_a(int bf16, const uint16_t *A, uint16_t *SA, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int g = 0; g < K / GS; ++g) {
            float mx = FLT_EPSILON;
            for (int p = 0; p < GS; ++p) {
                const float v = fabsf(orc_tof(A[(size_t)m * K + g * GS + p], bf16));
                mx = (mx < v) ? v : mx; /* std::max(mx, v) */
            }
            SA[(size_t)g * orc_ldsa(M) + m] = orc_fromf(127.0f / mx, bf16);
        }
}

void orc_quant_a(int bf16, const uint16_t *A, const uint16_t *SA, int8_t *Aq, int M, int K) {
#pragma omp parallel for schedule(static)
    for (int m = 0; m < M; ++m)
        for (int k = 0; k < K; ++k) {
            const float p = orc_tof(A[(size_t)m * K + k], bf16) *
                            orc_tof(SA[(size_t)(k / GS) * orc_ldsa(M) + m], bf16);
            /* lrintf + clamp to [-128, 127] as main.cpp:101-102 for every finite
             * product; a product of +-inf (fp16 SA overflows to inf when a
             * group's absmax is below 127 / 65504) saturates and NaN (0 * inf)
             * gives 0, as the reference device kernel's convert_char8_sat_rte
             * (int2_int8_dpas.cl:120) does: lrintf is undefined there. */
            long v;
            if (p != p) v = 0;
            else if (p >= 127.0f) v = 127;
            else if (p <= -128.0f) v = -128;
            else v = lrintf(p);
            Aq[(size_t)m * K + k] = (int8_t)v;
        }
}

void orc_int8_gold(int bf16, const uint16_t *A, const uint32_t *B, const uint16_t *SA,
                   const uint16_t *SB, float *C, int M, int K, int N) {
    const int groups = K / GS;
    int8_t *q = (int8_t *)malloc((size_t)M * K);
    orc_quant_a(bf16, A, SA, q, M, K);
#pragma omp parallel for collapse(2) schedule(static)
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            float acc = 0.0f;
            for (int g = 0; g < groups; ++g) {
                int32_t dot = 0;
                for (int p = 0; p < GS; ++p) {
                    const int ik = g * GS + p;
                    const uint32_t code = (B[(size_t)(ik / 16) * N + j] >> (2 * (ik % 16))) & 3u;
                    dot += (int)q[(size_t)i * K + ik] * orc_code_to_value(code);
                }
                const float sa = orc_tof(SA[(size_t)g * orc_ldsa(M) + i], bf16);
                const float inv = sa == 0.0f ? 0.0f : 1.0f / sa;
                acc += (float)dot * (orc_tof(SB[(size_t)g * N + j], bf16) * inv);
            }
            C[(size_t)i * N + j] = acc;
        }
    free(q);
}

/* ---- BITCOS: common/bitcos.hpp ----------------------------------------- */

#define BITCOS_PAD 4 /* kBitcosPad, common/bitcos.hpp:27 */

static uint32_t col_nnz(const int8_t *codes, int K, int N, int n) {
    uint32_t s = 0;
    for (int k = 0; k < K; ++k) s += codes[(size_t)k * N + n] != 0;
    return s;
}

size_t orc_bitcos_words(const int8_t *codes, int K, int N) {
    size_t words = 0;
    for (int n = 0; n < N; ++n) words += (col_nnz(codes, K, N, n) + 31) / 32;
    return (size_t)K / 32 * N + N + words + BITCOS_PAD;
}

/* The packer of common/bitcos.hpp:1-8 / bitcos_random :31-78, from a dense
 * code matrix codes[k][n] in {-1, 0, +1} instead of random draws. */
size_t orc_bitcos_pack(const int8_t *codes, int K, int N, uint32_t *buf) {
    const size_t bw = (size_t)K / 32 * N;
    size_t total = orc_bitcos_words(codes, K, N);
    memset(buf, 0, total * 4);
#pragma omp parallel for schedule(static)
    for (long long i = 0; i < (long long)bw; ++i) {
        const int kp = (int)(i / N), n = (int)(i % N);
        uint32_t w = 0;
        for (int c = 0; c < 32; ++c) w |= (uint32_t)(codes[(size_t)(kp * 32 + c) * N + n] != 0) << c;
        buf[i] = w;
    }
    uint32_t off = 0;
    for (int n = 0; n < N; ++n) {
        buf[bw + n] = off;
        off += (col_nnz(codes, K, N, n) + 31) / 32;
    }
    uint32_t *sg = buf + bw + N;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        uint32_t r = 0;
        uint32_t *col = sg + buf[bw + n];
        for (int k = 0; k < K; ++k) {
            const int8_t c = codes[(size_t)k * N + n];
            if (!c) continue;
            if (c < 0) col[r / 32] |= 1u << (r % 32);
            ++r;
        }
    }
    return total;
}

void orc_bitcos_slice_ranks(const uint32_t *buf, int K, int N, int ls, uint32_t *r) {
    const int slice_k = (K + ls - 1) / ls;
#pragma omp parallel for schedule(static)
    for (int n = 0; n < N; ++n) {
        uint32_t s = 0;
        int kp = 0;
        for (int sl = 1; sl < ls; ++sl) {
            for (; kp < sl * slice_k / 32; ++kp) s += (uint32_t)__builtin_popcount(buf[(size_t)kp * N + n]);
            r[(size_t)(sl - 1) * N + n] = s;
        }
    }
}

void orc_bitcos_decode_col(const uint32_t *buf, int K, int N, int n, int8_t *codes) {
    const size_t bw = (size_t)K / 32 * N;
    const uint32_t *sg = buf + bw + N + buf[bw + n];
    uint32_t rank = 0;
    for (int k = 0; k < K; ++k) {
        const int p = (buf[(size_t)(k / 32) * N + n] >> (k % 32)) & 1u;
        if (!p) { codes[k] = 0; continue; }
        codes[k] = ((sg[rank / 32] >> (rank % 32)) & 1u) ? -1 : 1;
        ++rank;
    }
}

void orc_bitcos_gold(int bf16, const uint16_t *A, const uint32_t *buf, const uint16_t *S,
                     float *C, int M, int K, int N) {
#pragma omp parallel
    {
        int8_t *codes = (int8_t *)malloc((size_t)K);
#pragma omp for schedule(dynamic, 16)
        for (int j = 0; j < N; ++j) {
            orc_bitcos_decode_col(buf, K, N, j, codes);
            for (int i = 0; i < M; ++i) {
                float acc = 0.0f;
                for (int g = 0; g < K / GS; ++g) {
                    float partial = 0.0f;
                    for (int p = 0; p < GS; ++p) {
                        const int k = g * GS + p;
                        if (codes[k]) partial += orc_tof(A[(size_t)i * K + k], bf16) * (float)codes[k];
                    }
                    acc += partial * orc_tof(S[(size_t)g * N + j], bf16);
                }
                C[(size_t)i * N + j] = acc;
            }
        }
        free(codes);
    }
}

void orc_bitcos_dequant(const uint32_t *buf, const uint16_t *S, uint16_t *W, int K, int N) {
#pragma omp parallel
    {
        int8_t *codes = (int8_t *)malloc((size_t)K);
#pragma omp for schedule(static)
        for (int n = 0; n < N; ++n) {
            orc_bitcos_decode_col(buf, K, N, n, codes);
            for (int k = 0; k < K; ++k) {
                const uint16_t s = S[(size_t)(k / GS) * N + n];
                W[(size_t)k * N + n] = codes[k] == 0 ? 0 : (codes[k] > 0 ? s : (uint16_t)(s ^ 0x8000u));
            }
        }
        free(codes);
    }
}

/* ---- FWHT: hadamard/hadamard_fwht.cl ----------------------------------- */

/* SCALE = 1/sqrt(n) as the fp32 constants of hadamard_fwht.cl:17-31. */
float orc_fwht_scale(int n) {
    switch (n) {
    case 1: return 1.0f;
    case 2: return 0.70710678118654752f;
    case 4: return 0.5f;
    case 8: return 0.35355339059327376f;
    case 16: return 0.25f;
    case 32: return 0.17677669529663688f;
    case 64: return 0.125f;
    case 128: return 0.088388347648318441f;
    case 256: return 0.0625f;
    case 512: return 0.044194173824159216f;
    case 1024: return 0.03125f;
    case 2048: return 0.022097086912079608f;
    case 4096: return 0.015625f;
    default: return 0.0f;
    }
}

static int is_pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }

static void fwht_block(const uint16_t *x, const int8_t *s, uint16_t *y, int n, int use_signs,
                       int bf16, float *v) {
    for (int i = 0; i < n; ++i)
        v[i] = use_signs ? orc_tof(x[i], bf16) * (float)s[i] : orc_tof(x[i], bf16);
    /* stages of stride 1, 2, 4, ..., n/2: the reference's radix-8 passes
     * (wht8, strides 8^p * {1,2,4}) then its radix-2 / radix-4 tail */
    for (int h = 1; h < n; h <<= 1)
        for (int i = 0; i < n; ++i)
            if ((i & h) == 0) {
                const float a = v[i], b = v[i + h];
                v[i] = a + b;
                v[i + h] = a - b;
            }
    const float sc = orc_fwht_scale(n);
    for (int i = 0; i < n; ++i) y[i] = orc_fromf(v[i] * sc, bf16);
}

int orc_fwht(int bf16, const uint16_t *x, const int8_t *signs, uint16_t *y, int rows, int K,
             int HB, int use_signs) {
    if (!is_pow2(HB) || HB < 256 || HB > 4096 || K <= 0) return -1;
    const int tail = K % HB;
    if (tail && !is_pow2(tail)) return -1;
    const int nblk = K / HB + (tail ? 1 : 0);
#pragma omp parallel
    {
        float *v = (float *)malloc((size_t)HB * sizeof(float));
#pragma omp for schedule(static) collapse(2)
        for (int r = 0; r < rows; ++r)
            for (int b = 0; b < nblk; ++b) {
                const int k0 = b * HB, n = (k0 + HB <= K) ? HB : tail;
                fwht_block(x + (size_t)r * K + k0, signs ? signs + k0 : NULL, y + (size_t)r * K + k0,
                           n, use_signs && signs, bf16, v);
            }
        free(v);
    }
    return 0;
}

/* ---- MoE: int2_moe/int2_moe_prefill.cl, int2_moe/prefill.cpp ----------- */

void orc_moe_route(const int *ids, int G, int E, int rows_per_tile, int *meta, int *perm,
                   int *inv) {
    int *cnt = (int *)calloc((size_t)E, sizeof(int));
    for (int g = 0; g < G; ++g) cnt[ids[g]]++;
    int r = 0, t = 0;
    for (int e = 0; e < E; ++e) {
        meta[e] = r;
        meta[E + 1 + e] = t;
        r += cnt[e];
        t += (cnt[e] + rows_per_tile - 1) / rows_per_tile;
    }
    meta[E] = r;
    meta[2 * E + 1] = t;
    for (int e = 0; e < E; ++e) cnt[e] = 0;
    for (int g = 0; g < G; ++g) { /* stable: rows of an expert in g order */
        const int e = ids[g], p = meta[e] + cnt[e]++;
        perm[p] = g;
        inv[g] = p;
    }
    free(cnt);
}

void orc_moe_gather(const uint16_t *X, const int *perm, uint16_t *Xs, int G, int K, int topk) {
#pragma omp parallel for schedule(static)
    for (int p = 0; p < G; ++p)
        memcpy(Xs + (size_t)p * K, X + (size_t)(perm[p] / topk) * K, (size_t)K * 2);
}

void orc_moe_combine(int bf16, const float *Y, const int *inv, const uint16_t *RW, uint16_t *O,
                     int T, int topk, int N) {
#pragma omp parallel for collapse(2) schedule(static)
    for (int t = 0; t < T; ++t)
        for (int n = 0; n < N; ++n) {
            float s = 0.0f;
            for (int j = 0; j < topk; ++j) {
                const int g = t * topk + j;
                s += orc_tof(RW[g], bf16) * Y[(size_t)inv[g] * N + n];
            }
            O[(size_t)t * N + n] = orc_fromf(s, bf16);
        }
}

/* Proj::w, int2_moe/prefill.cpp:63-66: code * scale as a float product. */
static inline float moe_w(int bf16, const uint32_t *B, const uint16_t *S, int K, int N, int e,
                          int k, int n) {
    const uint32_t word = B[((size_t)e * (K / 16) + k / 16) * N + n];
    return (float)orc_code_to_value((word >> (2 * (k % 16))) & 3u) *
           orc_tof(S[((size_t)e * (K / GS) + k / GS) * N + n], bf16);
}

/* int2_moe/prefill.cpp:291-315: double-precision reference of tokens
 * [T0, T1): O[(t - T0) * H + n].  round_up = 1: the up product is rounded to DT
 * before silu(gate) * up (the prefill check); 0: it is not (the decode check,
 * int2_moe/main.cpp:276-281). */
void orc_moe_ref_tokens(int bf16, const uint16_t *X, const int *ids, const uint16_t *RW, int T0,
                        int T1, int topk, int H, int I, const uint32_t *Bg, const uint16_t *Sg,
                        const uint32_t *Bu, const uint16_t *Su, const uint32_t *Bd,
                        const uint16_t *Sd, double *O, int round_up) {
#pragma omp parallel for schedule(dynamic, 1)
    for (int t = T0; t < T1; ++t) {
        double *o = O + (size_t)(t - T0) * H;
        float *h = (float *)malloc((size_t)I * sizeof(float));
        for (int n = 0; n < H; ++n) o[n] = 0.0;
        for (int j = 0; j < topk; ++j) {
            const int g = t * topk + j, e = ids[g];
            for (int n = 0; n < I; ++n) {
                double sg = 0.0, su = 0.0;
                for (int k = 0; k < H; ++k) {
                    const double x = orc_tof(X[(size_t)t * H + k], bf16);
                    sg += x * moe_w(bf16, Bg, Sg, H, I, e, k, n);
                    su += x * moe_w(bf16, Bu, Su, H, I, e, k, n);
                }
                const double up = round_up ? (double)orc_tof(orc_fromf((float)su, bf16), bf16) : su;
                h[n] = orc_tof(orc_fromf((float)(sg / (1.0 + exp(-sg)) * up), bf16), bf16);
            }
            for (int n = 0; n < H; ++n) {
                double s = 0.0;
                for (int k = 0; k < I; ++k) s += h[k] * moe_w(bf16, Bd, Sd, I, H, e, k, n);
                o[n] += s * orc_tof(RW[g], bf16);
            }
        }
        free(h);
    }
}

/* OpenMP threads of the oracle's loops (the CPU baseline times 1 core and all). */
void orc_set_threads(int n) { omp_set_num_threads(n > 0 ? n : 1); }
int orc_max_threads(void) { return omp_get_max_threads(); }
