/*
 * ternocl_amd.h -- C ABI of the MI355X (gfx950) ternary GEMV/GEMM library.
 *
 * Drop-in for the kernel surface of TernOCL (OpenCL kernels for Intel Xe2).
 * Every entry point keeps the reference kernel's tensors, layouts and argument
 * order; the OpenCL build-time switches (-DBF16, -DPOSTOP, -DOUT_F32, -DHB, ...)
 * become ordinary arguments.  All pointers are device pointers (hipMalloc'd),
 * `stream` is a hipStream_t (NULL = the default stream); every call is
 * stream-ordered and asynchronous and validates its arguments on the host
 * before any launch, returning a status (it never exits the process).
 *
 * Data formats (shared with the reference):
 *   A    : DT [M, K] row-major (DT = fp16 or bf16 raw bits)
 *   B    : uint32 [K/16, N]; word (kp, n) holds the 2-bit codes of rows
 *          16*kp .. 16*kp+15 of column n, row 16*kp+j at bits 2j..2j+1;
 *          codes {0, 1, 3} = {0, +1, -1} (code 2 is unspecified)
 *   S    : DT [K/128, N] per-128-group scales
 *   C    : DT [M, N], or fp32 with out_f32
 *   Other: DT [M, N]   (postop 1, 2, 5)     Bias: C's type [N] (postop 3, 5)
 * Constraints: N % 16 == 0, K % 128 == 0, M >= 1 (ragged M is fine).
 * The MFMA GEMMs (prefill, grouped MoE) address their operands with 32-bit
 * buffer offsets: packed weights (K * N / 4 bytes per matrix) and activation
 * rows stay below 2^31 bytes, or the entry returns TERNOCL_ERR_UNSUPPORTED_SHAPE.
 * The fp16 prefill GEMM (M > 16) forms 2 * S in fp16: it takes |S| < 32768.
 *
 * Epilogue (postop), applied to the fp32 accumulator before the output cast,
 * as common/epilogue.clh:27-37 and common/epilogue.hpp:98-115:
 *   0 none, 1 silu(acc)*other, 2 acc+other, 3 acc+bias[n], 4 sigmoid(acc)
 *   (0 for acc <= -10), and 5 = (acc + bias[n]) + other[m,n] (an extension:
 *   bias add and residual add fused in one pass; no reference counterpart).
 *   The sigmoid is the reference kernels' native form (common/epilogue.clh:25,
 *   the hardware's exp2 and reciprocal), within ~1e-6 relative of the exact one.
 */
#ifndef TERNOCL_AMD_H
#define TERNOCL_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    TERNOCL_OK = 0,
    TERNOCL_ERR_INVALID_ARG = 1,       /* null pointer, bad enum, bad postop */
    TERNOCL_ERR_UNSUPPORTED_SHAPE = 2, /* N % 16, K % 128, BITCOS K % (64*ls), ... */
    TERNOCL_ERR_WORKSPACE = 3,         /* workspace missing or too small */
    TERNOCL_ERR_LAUNCH = 4             /* the HIP runtime reported an error */
} ternocl_status;

typedef enum { TERNOCL_FP16 = 0, TERNOCL_BF16 = 1 } ternocl_dtype;

/* Workspaces.  Every entry that takes a device scratch (ws, ws_bytes) keeps
 * the same first TERNOCL_WS_HEADER_BYTES of it for its cross-workgroup
 * counters and writes nothing else there; its partial sums, re-packed weights
 * and MoE buffers lie after that header, and every *_ws_bytes() function
 * counts it.  Zero a scratch once (ternocl_workspace_zero) before its first
 * use: every call leaves the counters at zero again, so one scratch can serve
 * any sequence of calls of any entries and shapes, as long as calls that
 * share it do not overlap.  A K split whose counters would not fit the header
 * (more than 16384 column strips) runs unsplit instead. */
#define TERNOCL_WS_HEADER_BYTES ((size_t)64 << 10)

/* Human-readable status and the last HIP error text seen by this thread. */
const char *ternocl_status_string(int status);
const char *ternocl_last_error(void);
/* Library version, e.g. "0.1.0". */
const char *ternocl_version(void);

/* ---- int2 upcvt GEMV / GEMM -------------------------------------------
 * Replaces int2_fp16_upcvt_gemm (decode, int2_fp16_upcvt/int2_fp16_upcvt.cl:196-198)
 * and int2_fp16_upcvt_gemm_mt (prefill, :341-343):
 *   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(B[k,n])))
 * The library picks the kernel: a decode GEMV for M <= 16, an MFMA GEMM above.
 * ws / ws_bytes: optional device scratch (16-byte aligned), kept from the XeTLA
 * plugin's entry (the acc/cnt buffers of its global k-slicing,
 * tools/xetla_epilogue_parity/parity.cpp:26-41); ternocl_int2_gemm_ws_bytes()
 * says how much a shape uses (0: pass NULL).  The prefill GEMM uses it for
 * deterministic split-K on shapes whose 128 x 512 tiles would leave CUs idle
 * (M = 1024, K = 14336, N = 4096: 4 K-slices): fp32 partial tiles per slice,
 * then a reduction that adds the slices in order and applies the epilogue,
 * the same bits on every run.  Without the scratch (NULL or short) those
 * shapes run on 128 x 128 tiles instead.  Shapes that run 192 to 256 tiles
 * of 128 x 256 (more than 256 tiles of 128 x 128: M = 1024, K = 4096,
 * N = 6144) take them with or without the scratch and leave it unused
 * (ternocl_int2_gemm_ws_bytes() still counts a split there: the sizes are
 * upper bounds).  The fp8 x fp4 GEMV splits K over
 * several workgroups per column strip where one workgroup per strip would
 * leave CUs idle or stage too much of A (K = 14336, N = 4096; M >= 3):
 * fp32 slice sums [slices][M][N] and a counter per 16-column strip, the
 * last workgroup of a strip adding the slices in order.  Its counters must
 * read zero before the first call on a scratch (ternocl_workspace_zero once);
 * every call leaves them zero.  Without the scratch the GEMV runs unsplit.
 * Calls that share one scratch must not overlap. */
size_t ternocl_int2_gemm_ws_bytes(int M, int N, int K);
ternocl_status ternocl_int2_fp16_upcvt_gemm(int dtype, const void *A, const uint32_t *B,
                                            const void *S, void *C, const void *Other,
                                            const void *Bias, int M, int N, int K, int postop,
                                            int out_f32, void *ws, size_t ws_bytes, void *stream);

/* Decode-GEMV tile, the reference's -DSGM/-DNSG_N/-DLS/-DU knobs for this
 * hardware.  Every field 0 = automatic. */
typedef struct {
    int engine;          /* 1: VALU GEMV (v_dot2 MACs, M <= 8); 2: bf16/fp16 MFMA GEMV (M <= 16);
                            3: MFMA prefill GEMM (any M, 128 x 128 tiles; the M > 16 engine);
                            4: block-scaled fp8 x fp4 MFMA GEMV (M <= 8, A 16-byte aligned;
                               the automatic choice where it applies);
                            5: its multi-strip form (M <= 8, K per slice <= 8192 and at
                               M > 4 <= 4096, A 16-byte aligned): a workgroup stages the
                               activations once and walks many column strips, loading the next
                               strip's weights during the current one's MFMAs (the automatic
                               choice for N a multiple of 32 above 4096); takes cols_per_lane
                               (1 or 2; 4 at M = 1), groups_per_wave (1, 2 or 4; its waves follow)
                               and k_slices (with the ws above) */
    int waves;           /* waves per workgroup: VALU 1..16 (M = 1) or 1..8, MFMA 1..8 */
    int cols_per_lane;   /* MFMA: adjacent columns per lane, 1, 2 or 4 (16-, 32- or 64-column strips) */
    int groups_per_wave; /* MFMA: 128-row groups per wave per LDS window, 1..16 (power of
                            two, times M rounded up to a power of two <= 16) */
    int col_lanes;       /* VALU: lanes across a strip of 4*col_lanes columns, 4, 8 or 16 */
    int k_slices;        /* fp8 x fp4 GEMV: workgroups per column strip, each over a slice of K,
                            1..16 (at most one per 128-row group; > 1 needs the ws above) */
} ternocl_gemv_tile;

/* Same as ternocl_int2_fp16_upcvt_gemm with an explicit tile (NULL = automatic:
 * the fp8 x fp4 GEMV for M <= 8 (A 16-byte aligned), the bf16/fp16 MFMA GEMV
 * for other M <= 16, the prefill GEMM above).  When M > 16 the engine
 * must be 0 or 3. */
ternocl_status ternocl_int2_fp16_upcvt_gemm_ex(int dtype, const void *A, const uint32_t *B,
                                               const void *S, void *C, const void *Other,
                                               const void *Bias, int M, int N, int K,
                                               int postop, int out_f32, void *ws,
                                               size_t ws_bytes, const ternocl_gemv_tile *tile,
                                               void *stream);
/* Zero-fill device memory with a fill kernel (no hipMemset: graph-capturable). */
ternocl_status ternocl_workspace_zero(void *ws, size_t ws_bytes, void *stream);

/* Bit-exact test hook for the int2 unpack (no reference counterpart as an
 * entry point; it materialises the B operand the reference's dq_word builds,
 * int2_fp16_upcvt.cl:118-150): W[k][n] = +0 / S / S^0x8000 for codes 0 / 1 / 3,
 * W is DT [K, N].  The GEMVs' own in-register decodes are exported for testing
 * too: ternocl_int2_gemv_decode writes, per B word, the 8 packed DT pairs that
 * engine (1 = VALU GEMV, 2 = MFMA GEMV, 3 = prefill GEMM) builds (layout
 * [K/16][N][8] uint32); the prefill GEMM folds the group scale into its
 * fragments, and the hook builds them at unit scale (DT 1.0).  Engine 4 (the
 * fp8 x fp4 GEMV) writes its 2 fp4 dwords per word instead ([K/16][N][2]:
 * nibble n of dword h = row 2n + h as e2m1 v/2). */
ternocl_status ternocl_int2_dequant(int dtype, const uint32_t *B, const void *S, void *W, int K,
                                    int N, void *stream);
ternocl_status ternocl_int2_gemv_decode(int dtype, int engine, const uint32_t *B, uint32_t *D,
                                        int K, int N, void *stream);
/* Measurement hook, no GEMV: the decode GEMV's kernel (engine 4, the plan it
 * takes for this M, N, K) with the decode removed -- no activations, no MFMA;
 * it streams the same B and S bytes with the same grid, cross-wave reduction
 * and stores, writing C[m, n] = a checksum of column n's words.  Its duration
 * is the engine's memory ceiling, measured as the reference measures its own
 * (int2_fp16_upcvt/README.md:135-137: the GEMV with the decode removed).
 * C: fp32 [M, N]; M <= 8, N % 16 == 0, K % 128 == 0. */
ternocl_status ternocl_int2_gemv_stream_probe(int dtype, const uint32_t *B, const void *S, void *C, int M,
                                             int N, int K, void *stream);

/* Measurement hook, no GEMV: a plain streaming read of the first bytes & ~15
 * bytes of src (16-byte aligned), every lane issuing four coalesced 16-byte
 * loads of one 16 KiB block per workgroup before using any; it stores to the
 * one word at sink only if the XOR of all words read equals a fixed constant.
 * Its duration is what one launch reading that many bytes takes: the
 * per-launch ceiling a decode GEMV of the same bytes can approach. */
ternocl_status ternocl_stream_read_probe(const void *src, size_t bytes, void *sink, void *stream);

/* ---- int2 x int8 prefill ---------------------------------------------------
 * Replaces quant_a (int2_via_int2_x_int8_dpas/int2_int8_dpas.cl:105-106):
 *   SA[g, m] = DT(127 / max(absmax_{k in group g} |A[m, k]|, FLT_EPSILON))
 *   Aq[m, k] = sat_int8(round_to_nearest_even(A[m, k] * SA[k / 128, m]))
 * bit-exact with the reference's host quantization
 * (int2_via_int2_x_int8_dpas/main.cpp:82-103).  A: DT [M, K];
 * SA: DT [K/128, ternocl_ldsa(M)] (row pitch (M + 31) & ~31; the pad columns
 * are not written); Aq: int8 [M, K], or NULL to write SA only (the reference
 * built without WRITE_Q, :119).  Constraints: K % 128 == 0, M >= 1. */
int ternocl_ldsa(int M);
ternocl_status ternocl_quant_a(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K,
                               void *stream);

/* Replaces int2_int8_gemv / int2_int8_gemm_mt (int2_int8_dpas.cl:213-215,
 * :316-318) in both quantization modes:
 *   C[m,n] = ct(epi(sum_g float(sum_{k in g} Aq[m,k] * v(B[k,n])) * (SB[g,n] * (1/SA[g,m]))))
 * v = the 2-bit two's-complement value of the code (code 2 reads as -2, as
 * the reference's DPAS and host gold do).  The int32 group dot products are
 * exact; the fp32 rescale follows the host gold's order
 * (int2_via_int2_x_int8_dpas/main.cpp:113-116).  Aq non-NULL: upfront mode
 * (QMODE 0), Aq and SA from ternocl_quant_a, A not read (may be NULL).
 * Aq NULL: in-GEMM mode (QMODE 1, :21-27, :61-99): the DT activations A are
 * quantized tile by tile with SA from ternocl_quant_a; the int8 values equal
 * quant_a's for every finite input, so both modes give identical C.
 * SB: DT [K/128, N]; B, C, Other, Bias, postop and out_f32 as
 * ternocl_int2_fp16_upcvt_gemm.  Any M >= 1; the A operand (M*K elements of
 * Aq or A) and B must each be below 2^31 bytes.  M <= 4 with N % 16 == 0 (Aq
 * 8-byte or A 16-byte aligned) runs the decode GEMV (the reference's
 * int2_int8_gemv): the same exact group dot products and the same fold, with
 * the groups of a column summed in a different order than the tile GEMM. */
ternocl_status ternocl_int2_int8_gemm(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                      const uint32_t *B, const void *SB, void *C,
                                      const void *Other, const void *Bias, int M, int N, int K,
                                      int postop, int out_f32, void *stream);
/* The same call with device scratch (no reference counterpart: the
 * reference's int2_int8_gemm_mt and int2_int8_gemv take none).  Upfront mode
 * (Aq) on shapes whose 128 x 512 tiles would leave CUs idle (M = 1024,
 * K = 14336, N = 4096) runs those tiles over 2, 4 or 8 K slices into fp32
 * partials there, then a reduction adds the slices in order and applies the
 * epilogue (shapes that run 128 x 256 tiles instead, M = 1024 K = 4096
 * N = 6144, leave the scratch unused).  The decode GEMV (M <= 4, both modes) splits long K (>= 8192)
 * over narrow N (< 6144 columns) the same way, a counter per 16-column strip
 * electing the workgroup that adds the slices in order.  Either way the same
 * bits on every run.  ws: ternocl_int2_int8_gemm_ws_bytes(M, N, K) bytes (0:
 * none used), 16-byte aligned, zeroed once before its first use (the GEMV's
 * counters return to zero by themselves; calls that share ws must not
 * overlap); NULL or short: the call above. */
size_t ternocl_int2_int8_gemm_ws_bytes(int M, int N, int K);
ternocl_status ternocl_int2_int8_gemm_ws(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                         const uint32_t *B, const void *SB, void *C, const void *Other,
                                         const void *Bias, int M, int N, int K, int postop, int out_f32, void *ws,
                                         size_t ws_bytes, void *stream);

/* Bit-exact test hook of the s8 x s2 GEMM's B decode: D[word][i] (4 dwords per
 * B word, [K/16][N][4] uint32), byte b of dword i = int8 value of row 4b + i
 * of the word (the k order the GEMM uses for both operands). */
ternocl_status ternocl_int2_s8_decode(const uint32_t *B, uint32_t *D, int K, int N, void *stream);

/* ---- BITCOS (presence bitmap + compacted signs) GEMV --------------------
 * Replaces bitcos_fp16_upcvt_gemv / _gemm_mt (bitcos_fp16_upcvt/bitcos_fp16_upcvt.cl:179-181,
 * :303-305):  C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(k,n))).
 * B: the BITCOS buffer of common/bitcos.hpp, uint32 words
 *   bitmap [K/32][N] | offsets [N] | per-column sign streams | 4 pad words
 * (bit c of bitmap word (kp, n) = row 32kp+c of column n is non-zero; a sign
 * bit of 1 = -1, in k order per column).  SR: slice ranks [ls-1][N] for ls K
 * slices (common/bitcos.hpp:81-94; ternocl_bitcos_slice_ranks computes them
 * on the device), may be NULL when ls == 1.  The kernel splits K into exactly
 * ls slices.  Constraints: N % 16 == 0, K % 128 == 0, 1 <= ls <= 16,
 * K % (64 * ls) == 0.  M <= 4 per pass (larger M runs ceil(M/4) passes over
 * the weights). */
ternocl_status ternocl_bitcos_fp16_upcvt_gemm(int dtype, const void *A, const uint32_t *B,
                                              const void *S, const uint32_t *SR, int ls, void *C,
                                              const void *Other, const void *Bias, int M, int N,
                                              int K, int postop, int out_f32, void *stream);
/* The same call with device scratch (no reference counterpart: the
 * reference's GEMV runs one workgroup per 64-column strip, as the entry
 * above does).  Where the strips would load the CUs unevenly (N = 21504:
 * 336 strips on 256 CUs) a strip's ls slices are spread over several
 * workgroups, which store fp32 sums [slices][4][N] and a counter per strip
 * there; the last workgroup of a strip adds the sums in order (the same bits
 * on every run).  ws: ternocl_bitcos_gemv_ws_bytes(N, ls) bytes, 16-byte
 * aligned, zeroed once before its first use (ternocl_workspace_zero); every
 * call leaves the counters at zero.  NULL or short: the unsplit launch.
 * Calls that share a workspace must not overlap. */
size_t ternocl_bitcos_gemv_ws_bytes(int N, int ls);
ternocl_status ternocl_bitcos_fp16_upcvt_gemm_ws(int dtype, const void *A, const uint32_t *B,
                                                 const void *S, const uint32_t *SR, int ls, void *C,
                                                 const void *Other, const void *Bias, int M, int N,
                                                 int K, int postop, int out_f32, void *ws, size_t ws_bytes,
                                                 void *stream);
/* The decode step's sign flip + Hadamard transform and BITCOS GEMV in one
 * launch (no reference counterpart: the reference runs hadamard_fwht,
 * hadamard/hadamard_fwht.cl:62-115, then bitcos_fp16_upcvt_gemv): the same C,
 * bit for bit, as ternocl_hadamard_fwht(x, signs, y, M, K, HB, use_signs)
 * followed by ternocl_bitcos_fp16_upcvt_gemm_ws(y, ...), without writing y.
 * Each workgroup transforms the HB-blocks its K range reads, one wave per
 * block, in the transform's own operation order.  x: DT [M, K], 16-byte
 * aligned; signs: int8 [K], 8-byte aligned, read when use_signs; HB 256 or
 * 512 with K % HB 0 or a power of two >= 8 (that tail transformed as one
 * block, as ternocl_hadamard_fwht does).  B, S, SR, ls, ws and the rest as
 * ternocl_bitcos_fp16_upcvt_gemm_ws. */
ternocl_status ternocl_bitcos_fwht_gemm_ws(int dtype, const void *x, const int8_t *signs, int HB, int use_signs,
                                          const uint32_t *B, const void *S, const uint32_t *SR, int ls, void *C,
                                          const void *Other, const void *Bias, int M, int N, int K, int postop,
                                          int out_f32, void *ws, size_t ws_bytes, void *stream);
/* ---- BITCOS M-tiled prefill ---------------------------------------------
 * Replaces bitcos_fp16_upcvt_gemm_mt (bitcos_fp16_upcvt/bitcos_fp16_upcvt.cl:303-305):
 * the same C as ternocl_bitcos_fp16_upcvt_gemm (within the float tolerance) for
 * any M, with the weights streamed once instead of once per 4 rows.
 * ws = NULL (the reference's call): the int2 prefill GEMM engine's tiles
 * decode the BITCOS weights themselves, each lane following its column's
 * sign stream down K (SR unused).  With ws (ternocl_bitcos_gemm_mt_ws_bytes:
 * the workspace header, then K * N / 4 bytes): one pass re-packs the weights
 * into the int2 format after the header, then the int2 engine runs on them
 * with S as is (the re-pack splits K into ls slices).  SR / ls as for
 * ternocl_bitcos_fp16_upcvt_gemm; the same constraints. */
size_t ternocl_bitcos_gemm_mt_ws_bytes(int K, int N);
ternocl_status ternocl_bitcos_fp16_upcvt_gemm_mt(int dtype, const void *A, const uint32_t *B,
                                                 const void *S, const uint32_t *SR, int ls, void *C,
                                                 const void *Other, const void *Bias, int M, int N,
                                                 int K, int postop, int out_f32, void *ws,
                                                 size_t ws_bytes, void *stream);
/* The re-pack alone (bit-exact hook): W2 uint32 [K/16][N], row j of word (kp, n)
 * in bits 2j, 2j+1 = code 0 / 1 / 3 for 0 / +1 / -1 (the int2 format of
 * ternocl_int2_fp16_upcvt_gemm). */
ternocl_status ternocl_bitcos_to_int2(const uint32_t *B, const uint32_t *SR, int ls, uint32_t *W2, int K,
                                      int N, void *stream);
/* Slice ranks of a BITCOS buffer for ls slices: SR[(s-1)*N + n] = non-zeros of
 * column n in bitmap words kp < s * ceil(K/ls) / 32 (common/bitcos.hpp:81-94). */
ternocl_status ternocl_bitcos_slice_ranks(const uint32_t *B, uint32_t *SR, int K, int N, int ls,
                                          void *stream);
/* A slice count for ternocl_bitcos_fp16_upcvt_gemm at this shape: among the
 * ls <= 16 with K % (64 * ls) == 0 that keep >= 6 sixty-four-row chunks per
 * slice, the one whose slices spread best over the CUs with the _ws entry's
 * split (on a tie: slices of at most 8 sixty-four-row chunks, the most such
 * chunks, else the larger ls; K = 5376: 12 at N = 21504 and at N = 16384). */
int ternocl_bitcos_pick_ls(int M, int N, int K);
/* Bit-exact test hook of the BITCOS decode: W[k][n] = 0 / S / S ^ 0x8000 for
 * code 0 / +1 / -1 (the B operand the reference builds, bitcos_fp16_upcvt.cl:153-175),
 * W DT [K, N]. */
ternocl_status ternocl_bitcos_dequant(int dtype, const uint32_t *B, const void *S, void *W, int K,
                                      int N, void *stream);

/* ---- host packers (CPU; no GPU call) -----------------------------------------
 * Produce the kernels' weight formats from dense ternary weights W: int8
 * [K, N] row-major, values -1, 0, +1 (any other value: TERNOCL_ERR_INVALID_ARG).
 * ternocl_int2_pack: B uint32 [K/16][N], word (kp, n) bits 2j..2j+1 = code of
 *   row 16 kp + j, codes 0 / 1 / 3 for 0 / +1 / -1 (int2_fp16_upcvt.cl:6-19;
 *   the reference generates packed codes directly, int2_fp16_upcvt/main.cpp:238-242).
 *   K % 16 == 0.  ternocl_int2_unpack is the reverse (code 2 reads as -2).
 * ternocl_bitcos_pack: the BITCOS buffer of common/bitcos.hpp:1-8 (bitmap
 *   [K/32][N] | offsets [N] | sign streams | 4 pad words), the layout
 *   bitcos_random (common/bitcos.hpp:31-78) builds; ternocl_bitcos_pack_words
 *   gives its length in uint32 words (0 for invalid W or shape).  K % 32 == 0.
 *   ternocl_bitcos_unpack decodes a buffer back to W (bitcos_decode_col,
 *   common/bitcos.hpp:97-106, for every column).
 * ternocl_bitcos_slice_ranks_host: the slice ranks SR [ls-1][N] of
 *   common/bitcos.hpp:81-94 on the host (ternocl_bitcos_slice_ranks computes
 *   the same on the GPU). */
ternocl_status ternocl_int2_pack(const int8_t *W, uint32_t *B, int K, int N);
ternocl_status ternocl_int2_unpack(const uint32_t *B, int8_t *W, int K, int N);
size_t ternocl_bitcos_pack_words(const int8_t *W, int K, int N);
ternocl_status ternocl_bitcos_pack(const int8_t *W, int K, int N, uint32_t *buf, size_t words);
ternocl_status ternocl_bitcos_unpack(const uint32_t *buf, size_t words, int K, int N, int8_t *W);
ternocl_status ternocl_bitcos_slice_ranks_host(const uint32_t *buf, int K, int N, int ls, uint32_t *SR);

/* ---- Hadamard input transform -------------------------------------------
 * Replaces hadamard_fwht(x, signs, y, K, use_signs) (hadamard/hadamard_fwht.cl:62-64)
 * with -DHB as an argument and the row count explicit:
 *   y = DT(SCALE * H_HB(s .* x)) per HB-wide block along K of x DT [rows, K],
 * fp32 butterflies in the reference's stage order (bit-identical), SCALE =
 * 1/sqrt(HB).  signs: int8 [K] (+1 / -1 per in-row position), read when
 * use_signs != 0.  HB: a power of two in [256, 4096].  K % HB may be non-zero
 * when it is a power of two: that tail is transformed as one block of its own
 * size (the reference leaves it unwritten). */
ternocl_status ternocl_hadamard_fwht(int dtype, const void *x, const int8_t *signs, void *y,
                                     int rows, int K, int HB, int use_signs, void *stream);

/* ---- int2 MoE prefill ----------------------------------------------------
 * Replaces the kernels of int2_moe/int2_moe_prefill.cl and the layer sequence
 * of int2_moe/prefill.cpp:268-279.  Assignments g = t * topk + j (token t,
 * slot j); ids int [G] expert of each assignment; RW DT [G] its gate weight.
 * Expert weights: B_all uint32 [E][K/16][N], S_all DT [E][K/128][N].
 *
 * Route (int2_moe_prefill.cl:29-61): meta int [2E+2] = row offsets [0..E] of
 * each expert in the expert-sorted order, then row-tile offsets [E+1..2E+1]
 * (tiles of ternocl_moe_tile_rows() rows); perm int [G] sorted row -> g;
 * inv int [G] = perm^-1.  Rows of an expert are in assignment order (stable,
 * deterministic).  An id outside [0, E) drops its assignment (inv = -1); the
 * rows past the kept ones, perm[meta[E] .. G), are set to -1.
 * 1 <= E <= 512. */
int ternocl_moe_tile_rows(void);
ternocl_status ternocl_int2_moe_route(const int *ids, int *meta, int *perm, int *inv, int G, int E,
                                      void *stream);
/* Gather (int2_moe_prefill.cl:63-70): Xs[p] = X[perm[p] / topk], rows of K DT,
 * for p < G; a row whose perm[p] is negative (a dropped assignment, as the
 * route leaves it) is written as zeros.  Every non-negative perm[p] must be
 * below T * topk for the T rows of X. */
ternocl_status ternocl_int2_moe_gather(int dtype, const void *X, const int *perm, void *Xs, int G,
                                       int K, int topk, void *stream);
/* Grouped GEMM (int2_moe_prefill.cl:72-141): for every sorted row p of expert e,
 *   C[p, n] = ct(epi(sum_g S_e[g,n] * sum_{k in g} A(p)[k] * code_e(k, n)))
 * A(p) = A_all[perm[p] / topk] when perm is non-NULL (the gather fused into
 * the GEMM's A loads), else A_all[p].  C and Other are [G, N] in sorted order;
 * postop 0, 1, 2 or 4 (no bias), out_f32 as ternocl_int2_fp16_upcvt_gemm. */
ternocl_status ternocl_int2_moe_gemm(int dtype, const int *meta, const void *A_all, const int *perm,
                                     int topk, const uint32_t *B_all, const void *S_all, void *C_all,
                                     const void *Other_all, int E, int G, int N, int K, int postop,
                                     int out_f32, void *stream);
/* Combine (int2_moe_prefill.cl:143-156): O[t, n] = DT(sum_{j < topk} RW[g] * Y[inv[g], n]),
 * j in order, fp32; Y fp32 [G, N] (sorted rows), O DT [T, N]. */
ternocl_status ternocl_int2_moe_combine(int dtype, const float *Y, const int *inv, const void *RW,
                                        void *O, int T, int topk, int N, void *stream);
/* One whole MoE layer: route, up = X x B_up (POSTOP 0), Hs = silu(X x B_gate) * up
 * (POSTOP 1), Y = Hs x B_down (fp32), combine.  X DT [T, H]; gate / up
 * weights [E][H/16][I] / [E][H/128][I]; down [E][I/16][H] / [E][I/128][H];
 * O DT [T, H].  ws: device scratch of ternocl_int2_moe_prefill_ws_bytes()
 * bytes (meta, the row-tile list, perm, inv, Hs, Y; the up and gate
 * projections run as one launch whose result equals the two-step sequence bit
 * for bit, and two experts' tails of at most 64 rows may share a row tile). */
size_t ternocl_int2_moe_prefill_ws_bytes(int T, int E, int topk, int H, int I);
ternocl_status ternocl_int2_moe_prefill(int dtype, const void *X, const int *ids, const void *RW,
                                        int T, int E, int topk, int H, int I, const uint32_t *Bg,
                                        const void *Sg, const uint32_t *Bu, const void *Su,
                                        const uint32_t *Bd, const void *Sd, void *O, void *ws,
                                        size_t ws_bytes, void *stream);

/* Replaces the int8 MoE prefill (int2_moe/int2_moe_prefill_int8.cl:1-191, the
 * sequence of int2_moe/prefill.cpp:243-279 run with --int8 0): route, quant_a
 * of the T token rows (ternocl_quant_a semantics, the reference's quant_x),
 * up = s8 x s2 per expert segment (POSTOP 0) and h = silu(gate) * up (POSTOP
 * 1, Other = up) in one pass that gathers the int8 rows through the route's
 * perm (its gather_q, inside the GEMM; up stays in registers, the bits of the
 * two launches), quant_a of h, down (fp32), combine; the
 * int8 values are the reference's QMODE 0 ones, which its QMODE 1
 * reproduces.  Arguments as ternocl_int2_moe_prefill; ws >=
 * ternocl_int2_moe_prefill_int8_ws_bytes(T, E, topk, H, I) bytes, 256-byte
 * aligned.  The expert-sorted rows (T topk H 4 bytes) and each expert's packed
 * weights must be below 2^31 bytes.  The
 * reference's pass rule for this layer is rel < 5e-2 (prefill.cpp:318). */
size_t ternocl_int2_moe_prefill_int8_ws_bytes(int T, int E, int topk, int H, int I);
ternocl_status ternocl_int2_moe_prefill_int8(int dtype, const void *X, const int *ids, const void *RW,
                                             int T, int E, int topk, int H, int I, const uint32_t *Bg,
                                             const void *Sg, const uint32_t *Bu, const void *Su,
                                             const uint32_t *Bd, const void *Sd, void *O, void *ws,
                                             size_t ws_bytes, void *stream);

/* ---- int2 MoE decode layer ------------------------------------------------
 * Replaces int2_moe_gate_up + int2_moe_down + int2_moe_reduce
 * (int2_moe/int2_moe.cl:61-133, the sequence of int2_moe/main.cpp:226-261): for
 * every assignment g = t * topk + j with expert e = ids[g],
 *   Hs[g] = DT(silu(X[t] . Bg[e]) * (X[t] . Bu[e]))   (fp32 products, one rounding)
 *   O[t]  = DT(sum_j RW[g] * (Hs[g] . Bd[e]))          (fp32, j order)
 * The weight GEMVs run on the fp8 x fp4 decode engine, one launch for gate and up,
 * one for down.  Same tensors as ternocl_int2_moe_prefill (X DT [T, H], ids int32
 * [T, topk], RW DT [T, topk], experts stacked); an id outside [0, E) contributes
 * nothing.  ws: ternocl_int2_moe_decode_ws_bytes() bytes, 256-byte aligned;
 * T * topk < 32768, H and I multiples of 128, X 16-byte aligned. */
size_t ternocl_int2_moe_decode_ws_bytes(int T, int topk, int H, int I);
ternocl_status ternocl_int2_moe_decode(int dtype, const void *X, const int *ids, const void *RW, int T,
                                       int E, int topk, int H, int I, const uint32_t *Bg, const void *Sg,
                                       const uint32_t *Bu, const void *Su, const uint32_t *Bd,
                                       const void *Sd, void *O, void *ws, size_t ws_bytes, void *stream);

/* The same MoE decode layer without a workspace argument: it allocates nothing
 * (no hipMalloc, no allocating library call), for callers that cannot
 * allocate -- code under HIP graph capture, tight serving loops, harnesses
 * that forbid allocation.  No counterpart in the reference.  Its scratch is a
 * fixed array of TERNOCL_NOALLOC_SCRATCH_BYTES per device, held until the
 * process ends; the first call on a device looks up that array's device
 * address (hipGetSymbolAddress, no allocation).  Shapes whose
 * ternocl_int2_moe_decode_ws_bytes() exceed it return TERNOCL_ERR_WORKSPACE.
 * Every call on one device shares that array: calls that overlap on one
 * device (two streams, two threads) race and must be serialised by the
 * caller.  Same results as ternocl_int2_moe_decode, bit for bit. */
#define TERNOCL_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
ternocl_status ternocl_int2_moe_decode_noalloc(int dtype, const void *X, const int *ids, const void *RW,
                                               int T, int E, int topk, int H, int I, const uint32_t *Bg,
                                               const void *Sg, const uint32_t *Bu, const void *Su,
                                               const uint32_t *Bd, const void *Sd, void *O, void *stream);

#ifdef __cplusplus
}
#endif
#endif
