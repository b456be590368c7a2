/*
 * ternocl_oracle.h -- CPU restatement of TernOCL's host reference path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (the HIP library, the
 * Python mirror of the kernel interface) may call, link or load this code:
 * only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg use it,
 * and only to check results against.
 *
 * Every function cites the reference file:line whose behaviour it restates.
 * Values of the 16-bit activation / scale / output dtype ("DT") travel as raw
 * uint16 bits, fp16 when bf16 == 0 and bf16 when bf16 != 0, like the
 * reference's dt16 (common/dt16.hpp:10).
 *
 * Parity status of each function is listed in the header of ternocl_oracle.c.
 */
#ifndef TERNOCL_ORACLE_H
#define TERNOCL_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* common/dt16.hpp:18-42 */
float orc_tof(uint16_t h, int bf16);
uint16_t orc_fromf(float f, int bf16);
void orc_tof_n(const uint16_t *h, float *f, size_t n, int bf16);
void orc_fromf_n(const float *f, uint16_t *h, size_t n, int bf16);

/* int2_fp16_upcvt/main.cpp:76 code_to_value, :79-98 compute_gold */
int orc_code_to_value(uint32_t c);
void orc_int2_gold(int bf16, const uint16_t *A, const uint32_t *B, const uint16_t *S,
                   float *C, int M, int K, int N);

/* Device decode of one int2 code into the B operand (int2_fp16_upcvt.cl:118-150,
 * :95-116): W[k][n] = 0 for code 0, S for code 1, S ^ 0x8000 for code 3. */
void orc_int2_dequant(const uint32_t *B, const uint16_t *S, uint16_t *W, int K, int N);

/* common/epilogue.hpp:82 sigmoid_ref, :98-115 epilogue_ref.  postop 0..4 as the
 * reference; postop 5 (an extension: acc + bias[n] + other[m,n], in that order,
 * fp32) is the bias-plus-residual composition this library adds. */
float orc_sigmoid(float x);
void orc_epilogue(int bf16, int postop, int out_f32, const float *acc, const uint16_t *other,
                  const void *bias, void *out, int M, int N);

/* int2_via_int2_x_int8_dpas/main.cpp:79 ldsa, :82-91 compute_scale_a,
 * :97-103 quantization, :94-121 compute_gold. SA is [K/128][ldsa(M)]. */
int orc_ldsa(int M);
void orc_scale_a(int bf16, const uint16_t *A, uint16_t *SA, int M, int K);
void orc_quant_a(int bf16, const uint16_t *A, const uint16_t *SA, int8_t *Aq, int M, int K);
void orc_int8_gold(int bf16, const uint16_t *A, const uint32_t *B, const uint16_t *SA,
                   const uint16_t *SB, float *C, int M, int K, int N);

/* BITCOS container, common/bitcos.hpp:1-114.  Layout of buf (uint32 words):
 * bitmap [K/32][N] | offsets [N] | signs | 4 pad words. */
size_t orc_bitcos_words(const int8_t *codes, int K, int N);
size_t orc_bitcos_pack(const int8_t *codes, int K, int N, uint32_t *buf);
void orc_bitcos_slice_ranks(const uint32_t *buf, int K, int N, int ls, uint32_t *sr);
void orc_bitcos_decode_col(const uint32_t *buf, int K, int N, int n, int8_t *codes);
void orc_bitcos_gold(int bf16, const uint16_t *A, const uint32_t *buf, const uint16_t *S,
                     float *C, int M, int K, int N);
/* Decoded B operand of the BITCOS kernels (bitcos_fp16_upcvt.cl:88-94, :153-175):
 * W[k][n] = 0 / S / S ^ 0x8000 for code 0 / +1 / -1. */
void orc_bitcos_dequant(const uint32_t *buf, const uint16_t *S, uint16_t *W, int K, int N);

/* hadamard/hadamard_fwht.cl:1-115: y = DT(SCALE * H_HB(s .* x)), fp32 radix-2
 * stages in increasing stride order.  A tail K % HB (which the reference leaves
 * unwritten) is transformed as one smaller block of size K % HB when that is a
 * power of two (an extension, parity unpinned). Returns 0, or -1 on bad args. */
int orc_fwht(int bf16, const uint16_t *x, const int8_t *signs, uint16_t *y, int rows, int K,
             int HB, int use_signs);
float orc_fwht_scale(int n);

/* int2_moe/int2_moe_prefill.cl:29-61 route (stable order), :63-70 gather,
 * :143-156 combine; int2_moe/prefill.cpp:288-319 double-precision token check. */
void orc_moe_route(const int *ids, int G, int E, int rows_per_tile, int *meta, int *perm,
                   int *inv);
void orc_moe_gather(const uint16_t *X, const int *perm, uint16_t *Xs, int G, int K, int topk);
void orc_moe_combine(int bf16, const float *Y, const int *inv, const uint16_t *RW, uint16_t *O,
                     int T, int topk, int N);
void orc_moe_ref_tokens(int bf16, const uint16_t *X, const int *ids, const uint16_t *RW, int T0,
                        int T1, int topk, int H, int I, const uint32_t *Bg, const uint16_t *Sg,
                        const uint32_t *Bu, const uint16_t *Su, const uint32_t *Bd,
                        const uint16_t *Sd, double *O, int round_up);

void orc_set_threads(int n);
int orc_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
