// int2_gemv_f4.hip -- decode GEMV for packed 2-bit ternary weights on the
// gfx950 block-scaled fp8 x fp4 matrix cores (engine 4, the default for
// M <= 8).  Replaces int2_fp16_upcvt_gemm
// (int2_fp16_upcvt/int2_fp16_upcvt.cl:193-290):
//
//   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(B[k,n])))
//
// A decode GEMV streams the weights once; what bounds it after the memory is
// the VALU work done per weight while the stream arrives.  This engine keeps
// that work small on both operands:
//
// * Weights become fp4 (e2m1) MFMA operands with three bit operations per 16
//   weights: a code's two bits (b1 b0) land on bits 3 and 2 of a nibble, the
//   e2m1 sign and upper exponent bit, so codes 0, 1, 3 read as +0, +2.0, -2.0
//   (the unused code 2 as -0), i.e. exactly 2v: a word's even rows are
//   (w << 2) & 0xCCCCCCCC, its odd rows w & 0xCCCCCCCC.
// * Activations become fp8 (e4m3) "pieces" that sum to the activation:
//   piece p = rne_e4m3(r_p / s_p), r_0 = a, r_{p+1} = r_p - piece_p * s_p, with
//   a power-of-two scale s_p per 32-activation block that puts the block's
//   largest |r_p| in [1, 2); the last piece uses the previous scale / 16,
//   enough for every residual (at most half an ulp of a 4-bit value below 2,
//   |r / s_prev| <= 1/16).  The scales are the MFMA's E8M0 block scales.  Each
//   piece of each activation row is its own MFMA row, so one
//   v_mfma_scale_f32_16x16x128_f8f6f4 computes sum piece * 2v for all pieces
//   and rows of a 128-row scale group over 16 columns.
// * Exactness.  The products are exact, but the MFMA adds the products of a
//   32-block with about 12 bits below the block's largest product (measured
//   on gfx950: next to a product of 128, products with bits below 2^-5 lose
//   them).  With the block's largest value in [1, 2), a piece holds 4-bit
//   values down to 2^-6 and e4m3 subnormals (multiples of 2^-9) below, and
//   values under 2^-10 round to 0 and stay whole in the residual: a piece
//   row's block spans at most 11 bits (products below 4 with bits down to
//   2^-8) and adds exactly.  bf16 takes 3 pieces, fp16 4 (rows 4m..4m+3 of
//   the MFMA); an activation within about 2^10 of its block's largest is
//   represented exactly, smaller ones to about 2^-16 of that largest value.
// * Per group and column the VALU then does one FMA per piece row
//   (acc += d * S[g,n]); the factor 1/2 is applied once at the end.
//
// Operand layout of the 16x16x128 MFMA (lane l, r = l % 16, q = l / 16),
// measured on gfx950: A (8 dwords of fp8) byte s of lane (r, q) is k = 16q + s
// for s < 16 and 64 + 16q + (s - 16) otherwise; B (4 dwords of fp4) nibble s
// of lane (c, q) is k = 32q + s; the E8M0 scale of A rows r, k in
// [32b, 32b + 32) comes from lane r + 16b; D element i of lane (c, q) is row
// 4q + i, column c.  So lane (c, q) takes words 2q and 2q + 1 of each group
// (its B dwords: even rows of word 2q, odd rows of 2q, even of 2q + 1, odd of
// 2q + 1), and the activations are staged in that k order.
//
// Work split (as the bf16 MFMA engine): a workgroup owns a strip of 16 * CPL
// columns over all of K; waves take contiguous runs of GPW groups per LDS
// window; each wave stages its own groups' pieces (no workgroup barrier
// before its MACs); wave partials are reduced through LDS in wave order
// (deterministic bit for bit).
//
// K slices (with the caller's workspace): KS workgroups share a strip, each
// over a contiguous 1/KS of the groups, so each stages only its slice of the
// activations -- the per-workgroup cost that grows with M * K.  Each writes
// its fp32 sums to the workspace; the workgroup that finishes last (a counter
// per strip) adds the KS slices in slice order and applies the epilogue, so
// the result does not depend on the order the workgroups run in.
#include "common.hpp"

#include <algorithm>
#include <climits>
#include <cmath>

namespace tcl {
namespace {

typedef int v8i_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef short s16x2_t __attribute__((ext_vector_type(2)));

// Pieces per activation (bf16 3, fp16 4) in MFMA rows 4m .. 4m + P - 1: an
// activation row's pieces sit in one lane of the MFMA result (rows 4q..4q+3).
__host__ __device__ constexpr int f4_pieces(bool bf16) { return bf16 ? 3 : 4; }
constexpr int kF4RowStride = 4;
// Rows per launch: 4 per MFMA row set of 16; M 5..8 take two row sets, two
// MFMAs per group and column on the same decoded weights (the int8 modes: 4).
constexpr int kF4MaxM = 32 / kF4RowStride;
constexpr int kF4MaxMI8 = 16 / kF4RowStride;
__host__ __device__ constexpr int f4_rsets(int mr) { return mr > 4 ? 2 : 1; }

// One weight word (rows 0..15 of a column) -> fp4 dwords: d0 nibble n = row 2n,
// d1 nibble n = row 2n + 1; nibble = (b1 << 3) | (b0 << 2) of the row's code.
__device__ __forceinline__ void f4_decode(uint32_t w, uint32_t &d0, uint32_t &d1) {
    d0 = (w << 2) & 0xCCCCCCCCu;
    d1 = w & 0xCCCCCCCCu;
}

// The s8 x s2 contract's decode (the int8 modes): code 2 reads as -2, the
// nibble 1110 (e2m1 -4.0 = 2 * -2); codes 0, 1, 3 as in f4_decode.  Bit 2r+1
// of t is set where row r holds code 2 (b1 = 1, b0 = 0).
__device__ __forceinline__ void f4_decode_s2(uint32_t w, uint32_t &d0, uint32_t &d1) {
    f4_decode(w, d0, d1);
    const uint32_t t = w & ~(w << 1);
    const uint32_t me = t & 0x22222222u, mo = t & 0x88888888u;  // even rows, odd rows
    d0 |= me | (me << 1);
    d1 |= (mo >> 1) | (mo >> 2);
}

// E8M0 exponent (biased, 1..254) of the scale that maps a block whose
// largest magnitude has fp32 biased exponent e into [1, 2): 2^(e - 127).
__device__ __forceinline__ uint32_t f4_scale_exp(uint32_t maxbits) {
    const int e = (int)(maxbits >> 23);
    return (uint32_t)(e < 1 ? 1 : (e > 254 ? 254 : e));
}

// max over the 4 lanes of a quad (lanes 4b .. 4b + 3: one 32-activation block)
__device__ __forceinline__ uint32_t quad_max(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
    return v;
}

// Four fp32 values (rows i0, i1, i2, i3 of a block) -> four e4m3 bytes of x / s.
__device__ __forceinline__ uint32_t f8x4(float a, float b, float c, float d, float s) {
    s16x2_t r = {0, 0};
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, a, b, s, false);
    r = __builtin_amdgcn_cvt_scalef32_pk_fp8_f32(r, c, d, s, true);
    uint32_t u;
    __builtin_memcpy(&u, &r, 4);
    return u;
}
// ... and back: the four values times s.
__device__ __forceinline__ void f8x4_back(uint32_t u, float s, float o[4]) {
    const f32x2_t lo = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)u, s, false);
    const f32x2_t hi = __builtin_amdgcn_cvt_scalef32_pk_f32_fp8((int)u, s, true);
    o[0] = lo[0]; o[1] = lo[1]; o[2] = hi[0]; o[3] = hi[1];
}

// Byte offset, inside a piece row's 128 bytes, of the 4 even-row bytes of
// the activations 8u .. 8u + 7 of a group (the odd-row bytes follow 8 bytes
// later).  In MFMA k order a 16-activation block b16 keeps its even rows at
// k = 16 b16 + 0..7 and its odd rows at 16 b16 + 8..15; k = 16 b16 + s' sits in
// byte 32 b16 + s' (b16 < 4) or 32 (b16 - 4) + 16 + s' (b16 >= 4).
__device__ __forceinline__ int f4_byte_off(int u) {
    const int b16 = u >> 1, half = u & 1;
    return (b16 < 4 ? 32 * b16 : 32 * (b16 - 4) + 16) + 4 * half;
}

// LDS of one window of one wave: data [GPW][RR][128] bytes, then scales
// [GPW][RR][4] bytes (RR = MFMA rows in use), rounded up to 16 bytes.
__host__ __device__ constexpr int f4_window_bytes(int rr, int gpw) { return (gpw * rr * 132 + 15) & ~15; }

// Activation staging of one window: tasks (m, gl, u) = 8 activations
// A[m, 128 g + 8u .. + 7] of row m < MR, window group gl < GPW, u < 16; task
// idx = (m * GPW + gl) * 16 + u; lane takes idx = lane + 64 t.  A quad of
// lanes holds one 32-activation block (u = 4b .. 4b + 3).
// QM (the int8 modes of the s8 x s2 GEMV): 0 = DT activations; 1 = int8 Aq
// (8 bytes per task); 2 = DT activations quantized here with SA[g, m] exactly
// as quant_a does (q = sat(rne(a * sa)), NaN -> 0).  An int8 value takes 2
// pieces, exactly: |q| <= 127 puts the block scale at <= 2^6, piece 0 keeps q's
// top 4 bits, and the residual is an integer of magnitude <= 2^(e_q - 4) <= 4,
// a multiple of s/16 that e4m3 holds.
// QM 3 (the MoE decode's down GEMV): A is fp32, gate rows, with the up rows
// ldsa floats further; the activation is h = DT(gate * sigmoid(gate) * up),
// the reference's rounding point (int2_moe/int2_moe.cl:95).
// QM 4 (a measurement, not a GEMV): the kernel with the decode removed -- no
// activations, no pieces, no MFMA; it streams the same weight and scale bytes
// with the same grid, reduction and stores (acc += float(w0 ^ w1) * s), the
// memory ceiling of the engine's structure.
template <int MR, int GPW, bool BF16, int QM = 0> struct F4Stage {
    static constexpr bool I8 = QM == 1 || QM == 2;
    static constexpr int P = I8 ? 2 : f4_pieces(BF16), RS = kF4RowStride, RR = RS * MR;
    static constexpr int T = MR * GPW * 16, TPL = (T + 63) / 64;
    uint4 raw[QM == 3 ? 1 : TPL];
    float4 gu[QM == 3 ? TPL : 1][4];  // QM 3: gate 8, up 8
    uint32_t sar[I8 ? TPL : 1];
    // Unconditional loads (row and group clamped into range): a load under a
    // branch is waited for at the branch's end.
    __device__ __forceinline__ void load(const uint16_t *__restrict__ A, int M, int K, int groups, int g0,
                                         int lane, const uint16_t *__restrict__ SA = nullptr, int ldsa = 0) {
#pragma unroll
        for (int t = 0; t < TPL; ++t) {
            const int idx = lane + 64 * t, u = idx & 15, mg = idx >> 4;
            const int m = mg / GPW, gl = mg % GPW;
            const int mc = m < M ? m : M - 1, g = g0 + gl < groups ? g0 + gl : groups - 1;
            if constexpr (QM == 3) {
                const float *ga = (const float *)A + (size_t)mc * K + (size_t)g * kGS + 8 * u;
                gu[t][0] = *(const float4 *)ga;
                gu[t][1] = *(const float4 *)(ga + 4);
                gu[t][2] = *(const float4 *)(ga + ldsa);
                gu[t][3] = *(const float4 *)(ga + ldsa + 4);
            } else if constexpr (QM == 1) {
                const uint2 v = *(const uint2 *)((const int8_t *)A + (size_t)mc * K + (size_t)g * kGS + 8 * u);
                raw[t] = make_uint4(v.x, v.y, 0u, 0u);
            } else {
                raw[t] = *(const uint4 *)(A + (size_t)mc * K + (size_t)g * kGS + 8 * u);
            }
            if constexpr (I8) sar[t] = SA[(size_t)g * ldsa + mc];
        }
    }
    __device__ __forceinline__ void store(uint8_t *data, int lane) const {
#pragma unroll
        for (int t = 0; t < TPL; ++t) {
            const int idx = lane + 64 * t, u = idx & 15, mg = idx >> 4;
            const int m = mg / GPW, gl = mg % GPW;
            const bool live = idx < T;
            const uint32_t w[4] = {raw[QM == 3 ? 0 : t].x, raw[QM == 3 ? 0 : t].y, raw[QM == 3 ? 0 : t].z,
                                   raw[QM == 3 ? 0 : t].w};
            float f[8];
            if constexpr (QM == 3) {
                const float ga[8] = {gu[t][0].x, gu[t][0].y, gu[t][0].z, gu[t][0].w,
                                     gu[t][1].x, gu[t][1].y, gu[t][1].z, gu[t][1].w};
                const float ua[8] = {gu[t][2].x, gu[t][2].y, gu[t][2].z, gu[t][2].w,
                                     gu[t][3].x, gu[t][3].y, gu[t][3].z, gu[t][3].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = dt2f<BF16>(f2dt<BF16>(ga[i] * sigmoid_ref(ga[i]) * ua[i]));
            } else if constexpr (QM == 1) {
#pragma unroll
                for (int i = 0; i < 8; ++i) f[i] = (float)(int8_t)(w[i >> 2] >> (8 * (i & 3)));
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    f[2 * i] = dt2f<BF16>(w[i] & 0xffffu);
                    f[2 * i + 1] = dt2f<BF16>(w[i] >> 16);
                }
            }
            if constexpr (QM == 2) {
                const float sa = dt2f<BF16>(sar[t]);  // quant_a's scale, as the quantization uses it
#pragma unroll
                for (int i = 0; i < 8; ++i) {  // the product is exact; |a * sa| <= 127.06
                    const float pq = f[i] * sa;
                    f[i] = pq == pq ? fminf(fmaxf(__builtin_rintf(pq), -128.0f), 127.0f) : 0.0f;
                }
            }
            float r[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) r[i] = f[i];
            const int row0 = (gl * RR + RS * m) * 128 + f4_byte_off(u);
            const int srow0 = GPW * RR * 128 + (gl * RR + RS * m) * 4 + (u >> 2);
            if constexpr (I8) {
                // 1 / SA[g, m] for the fold, in the scale slot of piece row
                // RS m + 2, which the two int8 pieces leave unused
                const float sa = dt2f<BF16>(sar[t]);
                if (live && u == 0)
                    *(float *)(data + GPW * RR * 128 + (gl * RR + RS * m + 2) * 4) = sa != 0.0f ? 1.0f / sa : 0.0f;
            }
            uint32_t se = 0;
#pragma unroll
            for (int p = 0; p < P; ++p) {
                // piece p's block scale: 2^(e - 127) for the block's largest
                // |r_p|; the last piece takes the previous scale / 16, which
                // bounds its residuals (|r| <= s_prev / 16) without a reduction
                if (p + 1 < P) {
                    float mx = 0.0f;
#pragma unroll
                    for (int i = 0; i < 8; ++i) mx = fmaxf(mx, fabsf(r[i]));
                    se = f4_scale_exp(quad_max(__float_as_uint(mx)));
                } else {
                    se = se > 5 ? se - 4 : 1;
                }
                const float s = __uint_as_float(se << 23);
                const float *x = r;
                const uint32_t ev = f8x4(x[0], x[2], x[4], x[6], s);
                const uint32_t od = f8x4(x[1], x[3], x[5], x[7], s);
                if (live) {
                    *(uint32_t *)(data + row0 + p * 128) = ev;
                    *(uint32_t *)(data + row0 + p * 128 + 8) = od;
                    if ((u & 3) == 0) data[srow0 + p * 4] = (uint8_t)se;
                }
                if (p + 1 < P) {  // residual for the next piece
                    float be[4], bo[4];
                    f8x4_back(ev, s, be);
                    f8x4_back(od, s, bo);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        r[2 * i] -= be[i];
                        r[2 * i + 1] -= bo[i];
                    }
                }
            }
        }
    }
};

// Weight words and scales are read once per launch: non-temporal loads (NT),
// so that the weight stream does not evict from L2 what the launch and the
// next one re-read (activations, epilogue operands, slice sums).  Measured
// against plain loads (graph-timed, >2 GiB rotated): the C2 step 2214-2252 ->
// 2281-2323 GB/s, K = 4096 N = 151680 33.1-34.4 -> 32.4-32.6 us, K = 5120 N =
// 34816 13.7 -> 12.8 us; the same bits.  The grouped (MoE decode) GEMVs, a few
// MB per launch and latency-bound, keep plain loads: the decode layer took
// 12.15 us with them non-temporal against 11.65 us (same box, three runs).
typedef uint32_t f4_u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t f4_u32x4 __attribute__((ext_vector_type(4)));

template <bool NT, class T> __device__ __forceinline__ T f4_ld(const T *p) {
    if constexpr (NT) return __builtin_nontemporal_load(p);
    else return *p;
}

template <int CPL, bool NT> struct F4Words;
template <bool NT> struct F4Words<1, NT> {
    uint32_t v[1];
    __device__ void load(const uint32_t *p) { v[0] = f4_ld<NT>(p); }
};
template <bool NT> struct F4Words<2, NT> {
    uint32_t v[2];
    __device__ void load(const uint32_t *p) {
        const f4_u32x2 t = f4_ld<NT>((const f4_u32x2 *)p);
        v[0] = t.x; v[1] = t.y;
    }
};
template <bool NT> struct F4Words<4, NT> {
    uint32_t v[4];
    __device__ void load(const uint32_t *p) {
        const f4_u32x4 t = f4_ld<NT>((const f4_u32x4 *)p);
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
};

// This wave's weight words (words 2q and 2q + 1 of each group) and raw scale
// bits of one window; loads unconditional (group clamped; groups past K are
// never consumed).
template <int CPL, int GPW, bool NT = true> struct F4Slab {
    F4Words<CPL, NT> w[GPW][2];
    uint32_t sc[GPW][(CPL + 1) / 2];
    __device__ __forceinline__ void load(const uint32_t *__restrict__ B, const uint16_t *__restrict__ S,
                                         int N, int groups, int g0w, int q, int n0) {
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = g0w + gi < groups ? g0w + gi : groups - 1;

#pragma unroll
            for (int t = 0; t < 2; ++t) w[gi][t].load(B + ((size_t)g * 8 + 2 * q + t) * N + n0);
            if constexpr (CPL == 4) {
                const f4_u32x2 t = f4_ld<NT>((const f4_u32x2 *)(S + (size_t)g * N + n0));
                sc[gi][0] = t.x;
                sc[gi][1] = t.y;
            } else if constexpr (CPL == 2) {
                sc[gi][0] = f4_ld<NT>((const uint32_t *)(S + (size_t)g * N + n0));
            } else {
                sc[gi][0] = f4_ld<NT>(S + (size_t)g * N + n0);
            }
        }
    }
    __device__ __forceinline__ uint32_t scale(int gi, int j) const {
        return CPL == 1 ? sc[gi][0] : ((j & 1) ? sc[gi][j >> 1] >> 16 : sc[gi][j >> 1] & 0xffffu);
    }
};

// Epilogue operands of the outputs a lane of wave 0 stores: row m = q,
// columns n0 + j.  Buffer loads with no branch: the other waves (and an
// operand the post-op does not use) pass an offset past the buffer's end,
// which returns 0 without a memory access, so the loads can be issued early
// and waited for only at the epilogue.
template <int MR, int CPL, bool BF16> struct F4EpiIn {
    static constexpr int OPL = f4_rsets(MR);  // outputs per lane: rows m = q + 4h, h < OPL
    // raw bits, converted only in the epilogue (a conversion here would make
    // the compiler wait for these loads, which follow every weight load)
    uint32_t o[OPL][CPL], b[CPL];
    __device__ __forceinline__ void load(const uint16_t *__restrict__ Other, const void *__restrict__ Bias,
                                         int postop, int out_f32, int M, int N, int q, int n0, bool mine) {
        const bool uo = postop_needs_other(postop), ub = postop_needs_bias(postop);
        const uint32_t ob = uo ? (uint32_t)((size_t)M * N * 2) : 0u;
        const uint32_t bb = ub ? (uint32_t)((size_t)N * (out_f32 ? 4 : 2)) : 0u;
        const __amdgpu_buffer_rsrc_t ro = buf_rsrc(uo ? Other : nullptr, ob);
        const __amdgpu_buffer_rsrc_t rb = buf_rsrc(ub ? Bias : nullptr, bb);
        const uint32_t off = 0x7ffffff0u;
        const int bsz = out_f32 ? 4 : 2;
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
#pragma unroll
            for (int h = 0; h < OPL; ++h) {
                const int m = q + 4 * h < M ? q + 4 * h : M - 1;
                const uint32_t oo = mine ? (uint32_t)(((size_t)m * N + n0 + j) * 2) : off;
                o[h][j] = __builtin_amdgcn_raw_buffer_load_b16(ro, oo, 0, 0);
            }
            const uint32_t bo = mine ? (uint32_t)((n0 + j) * bsz) : off;
            b[j] = out_f32 ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rb, bo, 0, 0)
                           : (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rb, bo, 0, 0);
        }
    }
    __device__ __forceinline__ float other(int h, int j) const { return dt2f<BF16>(o[h][j]); }
    __device__ __forceinline__ float bias(int j, int out_f32) const {
        return out_f32 ? __uint_as_float(b[j]) : dt2f<BF16>(b[j]);
    }
};

// Workgroup barrier between a window's activation loads and its weight loads
// (no data wait): every wave's activation requests enter the memory pipeline
// ahead of the weight stream.  The returned zero passes through an asm so the
// weight loads stay below the barrier.
__device__ __forceinline__ int f4_loads_after_barrier() {
    __builtin_amdgcn_s_barrier();
    int zero = 0;
    asm volatile("" : "+s"(zero));
    return zero;
}

// Waves per workgroup at most: 16 for one row and 16-column strips (the
// long-K shapes, whose activation staging is the bulk of the VALU work), else 8.
__host__ __device__ constexpr int f4_max_waves(int mr, int cpl) { return mr == 1 && cpl == 1 ? 16 : 8; }

// Grouped mode (the MoE decode GEMVs, int2_moe/int2_moe.cl:61-174): row v =
// blockIdx.y of the launch is pair g = v mod G of weight set v / G (set 1 =
// B2 / S2) with expert e = ids[g] of the stacked experts [E][K/16][N] /
// [E][K/128][N], activation row g / adiv of A (rows of K), and writes fp32 row
// v of C.  A pair whose expert id lies outside [0, E) writes zeros.
// DS (the decode layer's down launch with its weighted sum, the reference's
// int2_moe_down_sum, int2_moe/int2_moe.cl:133-174): workgroup (strip,
// token t), wave j = slot j: its own GEMV over all of K for pair g = t topk + j
// (expert ids[g], activation row g of the QM 3 staging); wave 0 then writes
// O[t] = DT(sum_j RW[g] * y_j) in slot order (fp32 products and sums, no
// contraction, as k_moe_combine).  A slot whose id lies outside [0, E)
// streams expert 0 and contributes y = 0.
struct F4Group {
    const int *ids;
    int G, E, adiv;
    const uint32_t *B2;
    const uint16_t *S2;
    int topk;
    const uint16_t *RW;
    uint16_t *O;
};

// QM != 0: the s8 x s2 GEMV (int2_int8_dpas.cl:213-215): S is SB, SA [K/128]
// [ldsa] the activation scales, A int8 (QM 1) or DT quantized while staged (QM
// 2); per group and column acc += float(dot) * (SB * (1 / SA)), the int32 dot
// exact (piece rows 4m, 4m + 1 sum to 2 dot).
// ksn > 1 (the plain GEMV, DT or int8, grid.y = ksn): K slice blockIdx.y; part fp32
// [ksn][M][N] slice sums, cnt one zero-initialised counter per strip (left at
// zero again).
template <int MR, int CPL, int GPW, bool BF16, bool GRP = false, int QM = 0, bool DS = false, bool MW = false>
__global__ void __launch_bounds__(64 * f4_max_waves(MR, CPL))
k_int2_gemv_f4(const uint16_t *__restrict__ A, const uint32_t *__restrict__ B,
               const uint16_t *__restrict__ S, void *__restrict__ C,
               const uint16_t *__restrict__ Other, const void *__restrict__ Bias, int M, int N,
               int K, int postop, int out_f32, int swz, F4Group grp = F4Group{},
               const uint16_t *__restrict__ SA = nullptr, int ldsa = 0, int ksn = 1, float *part = nullptr,
               uint32_t *cnt = nullptr) {
    constexpr bool I8 = QM == 1 || QM == 2, NODEC = QM == 4;
    constexpr int RS = kF4RowStride, RR = RS * MR, P = I8 ? 2 : f4_pieces(BF16);
    constexpr int RSETS = f4_rsets(MR), RR1 = RR < 16 ? RR : 16;  // MFMA row sets, rows per set
    static_assert(RR <= 32 && (RSETS == 1 || QM == 0 || NODEC), "two row sets: the DT mode only");
    extern __shared__ uint8_t lds8[];
    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    int groups = K / kGS;
    int ks = 0;
    constexpr bool SPLIT = (QM == 0 || QM == 1 || QM == 2) && !GRP && !DS;
    if constexpr (SPLIT) {
        if (ksn > 1) {  // slice ks: groups [ks gps, ks gps + gps) (the host keeps every slice non-empty)
            ks = blockIdx.y;
            const int gps = (groups + ksn - 1) / ksn, g_lo = ks * gps;
            groups = min(gps, groups - g_lo);
            if constexpr (QM == 1) A = (const uint16_t *)((const int8_t *)A + (size_t)g_lo * kGS);  // int8 rows
            else A += (size_t)g_lo * kGS;
            if constexpr (I8) SA += (size_t)g_lo * ldsa;
            B += (size_t)g_lo * 8 * N;
            S += (size_t)g_lo * N;
        }
    }
    const int gw = DS ? GPW : W * GPW;   // groups per window (DS: each wave covers all of K)
    const int g0w = DS ? 0 : wave * GPW;  // this wave's first group of a window
    const int windows = (groups + gw - 1) / gw;
    int strip = blockIdx.x;
    if (swz) {  // strips 2j, 2j+1 (sharing 128-byte lines) on the same XCD
        const int qq = blockIdx.x >> 3, x = blockIdx.x & 7;
        strip = (((qq >> 1) << 3) + x) * 2 + (qq & 1);
    }
    const int n0 = strip * 16 * CPL + CPL * c;
    bool dead = false;  // DS: this wave's slot has no expert
    if constexpr (DS) {
        const int g = blockIdx.y * grp.topk + wave;
        int e = grp.ids[g];
        dead = e < 0 || e >= grp.E;
        e = dead ? 0 : e;
        A = (const uint16_t *)((const float *)A + (size_t)g * K);
        B += (size_t)e * (K / 16) * N;
        S += (size_t)e * (K / kGS) * N;
    } else if constexpr (GRP) {  // (uniform per workgroup: no wave returns alone)
        const int v = blockIdx.y, set = v >= grp.G ? 1 : 0, g = v - set * grp.G;
        const int e = grp.ids[g];
        float *crow = (float *)C + (size_t)v * N;
        if (e < 0 || e >= grp.E) {
            if (wave == 0 && q == 0)
#pragma unroll
                for (int j = 0; j < CPL; ++j) crow[n0 + j] = 0.0f;
            return;
        }
        if constexpr (QM == 3)
            A = (const uint16_t *)((const float *)A + (size_t)g * K);
        else
            A += (size_t)(g / grp.adiv) * K;
        B = (set ? grp.B2 : B) + (size_t)e * (K / 16) * N;
        S = (set ? grp.S2 : S) + (size_t)e * (K / kGS) * N;
        C = crow;
    }
    constexpr int WB = f4_window_bytes(RR, GPW);
    const int nbuf = windows > 1 ? 2 : 1;
    uint8_t *wlds = lds8 + (size_t)wave * nbuf * WB;
    const int rho = c & (RR1 - 1);  // A row (piece row) this lane feeds in each row set; rows >= RR are don't-care

    F4Stage<MR, GPW, BF16, QM> st;
    if constexpr (!NODEC) st.load(A, M, K, groups, g0w, lane, SA, ldsa);
    int after = f4_loads_after_barrier();
    F4Slab<CPL, GPW, !GRP> cur;
    cur.load(B + after, S + after, N, groups, g0w, q, n0);
    F4EpiIn<MR, CPL, BF16> ein;  // behind the weights: waited for only at the epilogue
    ein.load(Other, Bias, postop, out_f32, M, N, q, n0, wave == 0);
    if constexpr (!NODEC) st.store(wlds, lane);

    constexpr int ROWS = I8 ? 1 : P;  // accumulators per column: the pieces of row m = q, or their sum
    float acc[RSETS][CPL][ROWS];  // row set t: rows m = q + 4t
#pragma unroll
    for (int t = 0; t < RSETS; ++t)
#pragma unroll
        for (int j = 0; j < CPL; ++j)
#pragma unroll
            for (int i = 0; i < ROWS; ++i) acc[t][j][i] = 0.0f;

    // One window: its MFMAs and group FMAs; PRE: first the next window's loads,
    // unconditional -- loads under a branch are waited for at the branch's
    // end, which would serialise them with this window's work.
    auto window = [&](int win, auto PRE_, F4Slab<CPL, GPW, !GRP> &cu, F4Slab<CPL, GPW, !GRP> &nx) __attribute__((always_inline)) {
        constexpr bool PRE = decltype(PRE_)::value;
        asm volatile("" ::: "memory");  // staging writes precede the reads (in-order LDS per wave)
        const uint8_t *buf = wlds + (size_t)(win & 1) * WB;
        if constexpr (PRE) {
            if constexpr (!NODEC) st.load(A, M, K, groups, (win + 1) * gw + g0w, lane, SA, ldsa);
            after = f4_loads_after_barrier();
            nx.load(B + after, S + after, N, groups, (win + 1) * gw + g0w, q, n0);
        }
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = win * gw + g0w + gi;
            if (g >= groups) break;  // uniform across the wave
            if constexpr (NODEC) {
#pragma unroll
                for (int j = 0; j < CPL; ++j)
                    acc[0][j][0] += (float)(cu.w[gi][0].v[j] ^ cu.w[gi][1].v[j]) * dt2f<BF16>(cu.scale(gi, j));
                continue;
            }
            v8i_t av[RSETS];
            int sa[RSETS];
#pragma unroll
            for (int t = 0; t < RSETS; ++t) {
                const int pr = gi * RR + 16 * t + rho;
                const uint8_t *row = buf + pr * 128 + 32 * q;
                const uint4 a0 = *(const uint4 *)row, a1 = *(const uint4 *)(row + 16);
                sa[t] = buf[GPW * RR * 128 + pr * 4 + q];
                av[t] = v8i_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
            }
            float inv = 0.0f;  // int8 modes: 1 / SA[g, m] of row m = q (clamped into the rows staged)
            if constexpr (I8)
                inv = *(const float *)(buf + GPW * RR * 128 + (gi * RR + RS * (q < MR ? q : MR - 1) + 2) * 4);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                uint32_t d0, d1, e0, e1;
                if constexpr (I8) {
                    f4_decode_s2(cu.w[gi][0].v[j], d0, d1);
                    f4_decode_s2(cu.w[gi][1].v[j], e0, e1);
                } else {
                    f4_decode(cu.w[gi][0].v[j], d0, d1);
                    f4_decode(cu.w[gi][1].v[j], e0, e1);
                }
                const v8i_t bv = {(int)d0, (int)d1, (int)e0, (int)e1, 0, 0, 0, 0};
                const float s = dt2f<BF16>(cu.scale(gi, j));
#pragma unroll
                for (int t = 0; t < RSETS; ++t) {
                    const f32x4_t d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        av[t], bv, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0 /*A e4m3*/, 4 /*B e2m1*/, 0, sa[t], 0, 127);
                    if constexpr (I8) {
                        const float dot = (d[0] + d[1]) * 0.5f;  // the group's int32 dot product
                        acc[t][j][0] += dot * (s * inv);
                    } else {
#pragma unroll
                        for (int i = 0; i < ROWS; ++i) acc[t][j][i] = d[i] * s + acc[t][j][i];
                    }
                }
            }
        }
        if constexpr (PRE) {
            asm volatile("" ::: "memory");
            uint8_t *nb = wlds + (size_t)((win + 1) & 1) * WB;
            if constexpr (!NODEC) st.store(nb, lane);
        }
    };
    if constexpr (!MW) {
        // one window (the host's choice for one), or the group modes: a next
        // window loaded under a branch and copied into place
        for (int win = 0; win < windows; ++win) {
            F4Slab<CPL, GPW, !GRP> nxt;
            if (win + 1 < windows) {
                window(win, std::true_type{}, cur, nxt);
                cur = nxt;
            } else {
                window(win, std::false_type{}, cur, nxt);
            }
        }
    } else {
        F4Slab<CPL, GPW, !GRP> cur2;
        // two register sets used in turn (ping-pong): a copy of the next
        // window's registers into the current ones would wait for their
        // loads; the last window loads nothing (uniform tests, no loads inside)
        for (int win = 0;; win += 2) {
            window(win, std::true_type{}, cur, cur2);
            if (win + 2 == windows) {
                window(win + 1, std::false_type{}, cur2, cur);
                break;
            }
            window(win + 1, std::true_type{}, cur2, cur);
            if (win + 3 == windows) {
                window(win + 2, std::false_type{}, cur, cur2);
                break;
            }
        }
    }

    // ---- pieces -> outputs (x 1/2: the fp4 operand held 2v), then waves ----
    // lane q holds, in row set h, rows 4q .. 4q + P - 1 of the set: the pieces
    // of output row m = q + 4h
    constexpr int OPL = F4EpiIn<MR, CPL, BF16>::OPL, QV = MR < 4 ? MR : 4;
    float out[CPL][OPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j)
#pragma unroll
        for (int h = 0; h < OPL; ++h) {
            if constexpr (I8) {
                out[j][h] = acc[h][j][0];
            } else {
                float t = acc[h][j][0];
#pragma unroll
                for (int i = 1; i < P; ++i) t += acc[h][j][i];
                out[j][h] = t * 0.5f;
            }
        }
    const bool live = q < QV;
    if constexpr (DS) {  // y_j of every slot, then wave 0's weighted sum in slot order
        float *red = (float *)(lds8 + (size_t)nbuf * W * WB);  // [W][CPL][16]
        if (live)
#pragma unroll
            for (int j = 0; j < CPL; ++j) red[(wave * CPL + j) * 16 + c] = dead ? 0.0f : out[j][0];
        __syncthreads();
        if (wave != 0 || !live) return;
        const int t = blockIdx.y;
        float sum[CPL];
#pragma unroll
        for (int j = 0; j < CPL; ++j) sum[j] = 0.0f;
        for (int w2 = 0; w2 < W; ++w2) {
            const float rw = dt2f<BF16>(grp.RW[t * grp.topk + w2]);
#pragma unroll
            for (int j = 0; j < CPL; ++j) sum[j] = __fadd_rn(sum[j], __fmul_rn(rw, red[(w2 * CPL + j) * 16 + c]));
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) grp.O[(size_t)t * N + n0 + j] = (uint16_t)f2dt<BF16>(sum[j]);
        return;
    }
    if (W > 1) {
        float *red = (float *)(lds8 + (size_t)nbuf * W * WB);  // [W-1][CPL][QV*16][OPL]
        constexpr int JS = QV * 16 * OPL;
        if (wave != 0 && live) {
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int h = 0; h < OPL; ++h) red[((wave - 1) * CPL + j) * JS + (q * 16 + c) * OPL + h] = out[j][h];
        }
        __syncthreads();
        if (wave != 0 || !live) return;
        for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int h = 0; h < OPL; ++h) out[j][h] += red[((w2 - 1) * CPL + j) * JS + (q * 16 + c) * OPL + h];
    }
    if (!live) return;
    if constexpr (SPLIT) {
        if (ksn > 1) {
            // This slice's sums, then the strip's counter; the last of the ksn
            // workgroups adds the slices in order.  No fences, by design (the
            // orderings rest on how gfx950 executes scoped accesses):
            // * release side: the sums are agent-scope stores (global_store
            //   sc1, written through to the point of coherence of all XCDs),
            //   and s_waitcnt(0) waits for their completion before the
            //   counter's atomic issues -- what an agent-scope release would
            //   order, without its L2 write-back (buffer_wbl2) in every
            //   workgroup;
            // * acquire side: the elected workgroup reads the sums with
            //   agent-scope loads (global_load sc1, which read the point of
            //   coherence, not a stale L1 or L2 line), issued only after the
            //   counter's result has been tested.  An agent-scope acquire
            //   fence here (buffer_inv sc1) measured 7.2 -> 7.75 us per launch
            //   at K = 14336, N = 4096: it drops the XCD's L2 lines the
            //   strip's other workgroups still read.
            // The split tests run each shape repeatedly and require the same
            // bits every time; recheck them after a toolchain update.
#pragma unroll
            for (int h = 0; h < OPL; ++h) {
                const int m = q + 4 * h;
                if (m < M)
#pragma unroll
                    for (int j = 0; j < CPL; ++j)
                        __hip_atomic_store(part + ((size_t)ks * M + m) * N + n0 + j, out[j][h], __ATOMIC_RELAXED,
                                           __HIP_MEMORY_SCOPE_AGENT);
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            __builtin_amdgcn_s_waitcnt(0);
            const uint32_t prev = split_arrive(cnt + strip, ksn, lane);
            if (prev != (uint32_t)(ksn - 1)) return;
            // four slices' loads in flight at a time (rows and slices past the
            // end clamped, loaded and not added), then added in slice order
            for (int s0 = 0; s0 < ksn; s0 += 4) {
                float v[4][OPL][CPL];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    const int s2 = s0 + u < ksn ? s0 + u : ksn - 1;
#pragma unroll
                    for (int h = 0; h < OPL; ++h) {
                        const int m = q + 4 * h < M ? q + 4 * h : M - 1;
#pragma unroll
                        for (int j = 0; j < CPL; ++j)
                            v[u][h][j] = __hip_atomic_load(part + ((size_t)s2 * M + m) * N + n0 + j,
                                                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                    }
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    if (s0 + u >= ksn) break;
#pragma unroll
                    for (int h = 0; h < OPL; ++h)
#pragma unroll
                        for (int j = 0; j < CPL; ++j) out[j][h] = s0 + u == 0 ? v[u][h][j] : out[j][h] + v[u][h][j];
                }
            }
        }
    }
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
        constexpr int PO = decltype(P_)::value;
        constexpr bool F32 = decltype(F_)::value;
#pragma unroll
        for (int h = 0; h < OPL; ++h) {
            const int m = q + 4 * h;
            if (m >= M) break;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float r = epi_apply_c<PO>(out[j][h], ein.other(h, j), ein.bias(j, F32));
                const size_t oi = (size_t)m * N + n0 + j;
                if constexpr (F32) ((float *)C)[oi] = r;
                else ((uint16_t *)C)[oi] = (uint16_t)f2dt<BF16>(r);
            }
        }
    });
}

// ---- multi-strip decode GEMV (engine 5: M <= 4, all of K in one window) ----
// The kernel above stages the activation pieces in every workgroup, i.e. once
// per 16- or 32-column strip: at N = 151680 that is 4740 times the same
// vector, and the staging's VALU work, not HBM, bounds the launch.  Here a
// workgroup stages them once and keeps each wave's A fragments (its GPW
// groups, all of K across the W waves) in registers, then walks the strips
// s = blockIdx.x, + gridDim.x, ... of 16 columns: the next strip's weight
// words, scales and epilogue operands are loaded while the current strip's
// MFMAs run, the wave partials meet in LDS (two buffers, one barrier per
// strip) and wave it % W adds them in wave order and stores the strip.  The
// per-column arithmetic (pieces, MFMA, per-group FMA in group order, wave
// order) is the kernel above's with the same waves and groups per wave: the
// same bits.  MR rows (1, 2, 4 or 8 >= M): piece rows 4m .. 4m + 3 of the
// MFMA; up to 4 rows one MFMA per group and 16 columns, 8 rows two (row sets t
// = 0, 1: rows m = 4t + q); lane q carries output rows q + 4t (rows from M on
// are computed on the last row's data and not stored).  MR 8: at most 8 waves
// (the registers of two row sets), and the wave partials reuse the staging
// windows once the fragments are in registers.  QM 1 / 2 (MR <= 4): the s8 x
// s2 GEMV's int8 modes (the kernel above's QM 1 / 2: A int8, or DT quantized
// while staged; SA [K/128][ldsa]), each group's 1 / SA[g, q] held in
// registers beside its fragments.  KS (ksn > 1, grid.y = ksn): K slice
// blockIdx.y for every strip the workgroup walks; each strip's reducer stores
// the slice's sums (part fp32 [ksn][M][N]) and arrives at the strip's counter,
// and the last of the ksn adds the slices in order -- the kernel above's
// handoff.  (A variant of its own: the handoff's registers would make the
// unsplit kernel spill.)
template <int MR, int GPW, int CPL, bool BF16, int QM = 0, bool KS = false>
__global__ void __launch_bounds__(MR > 4 ? 64 * 8 : 64 * 16)
k_int2_gemv_f4ms(const uint16_t *__restrict__ A, const uint32_t *__restrict__ B,
                 const uint16_t *__restrict__ S, void *__restrict__ C, const uint16_t *__restrict__ Other,
                 const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32,
                 const uint16_t *__restrict__ SA = nullptr, int ldsa = 0, int ksn = 1, float *part = nullptr,
                 uint32_t *cnt = nullptr) {
    static_assert(MR == 1 || MR == 2 || MR == 4 || MR == 8, "1, 2, 4 or 8 rows");
    static_assert(QM == 0 || ((QM == 1 || QM == 2) && MR <= 4), "DT, or int8 activations up to 4 rows");
    static_assert(!KS || QM == 0, "K slices: DT activations");
    constexpr bool I8 = QM != 0;
    constexpr int RS = kF4RowStride, RR = RS * MR, P = I8 ? 2 : f4_pieces(BF16);
    constexpr int RSETS = f4_rsets(MR), RR1 = RR < 16 ? RR : 16, QV = MR < 4 ? MR : 4;
    constexpr int WB = f4_window_bytes(RR, GPW);
    extern __shared__ uint8_t lds8[];
    const int W = blockDim.x >> 6;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    int groups = K / kGS;
    const int g0w = wave * GPW;  // (the host keeps a slice's groups <= W GPW)
    const int ks = KS ? (int)blockIdx.y : 0;
    if constexpr (KS) {  // slice ks: groups [ks gps, ks gps + gps) (the host keeps every slice non-empty)
        const int gps = (groups + ksn - 1) / ksn, g_lo = ks * gps;
        groups = min(gps, groups - g_lo);
        A += (size_t)g_lo * kGS;
        B += (size_t)g_lo * 8 * N;
        S += (size_t)g_lo * N;
    }
    const int strips = N / (16 * CPL);
    int s = blockIdx.x;
    if (s >= strips) return;  // (whole workgroup)
    uint8_t *wlds = lds8 + (size_t)wave * WB;
    float *red = (float *)(lds8 + (MR > 4 ? (size_t)0 : (size_t)W * WB));  // [2][W][CPL][MR][16]

    F4Stage<MR, GPW, BF16, QM> st;
    st.load(A, M, K, groups, g0w, lane, SA, ldsa);
    int after = f4_loads_after_barrier();
    F4Slab<CPL, GPW> cur;
    cur.load(B + after, S + after, N, groups, g0w, q, s * 16 * CPL + CPL * c);
    F4EpiIn<MR, CPL, BF16> ein;
    ein.load(Other, Bias, postop, out_f32, M, N, q, s * 16 * CPL + CPL * c, wave == 0);
    st.store(wlds, lane);
    asm volatile("" ::: "memory");  // this wave's staging writes precede its reads (in-order LDS per wave)
    const int rho = c & (RR1 - 1);
    v8i_t av[RSETS][GPW];
    int sa[RSETS][GPW];
    float inv[GPW];  // int8 modes: 1 / SA[g, m] of row m = q (clamped into the rows staged)
#pragma unroll
    for (int gi = 0; gi < GPW; ++gi) {
#pragma unroll
        for (int t = 0; t < RSETS; ++t) {
            const int pr = gi * RR + 16 * t + rho;
            const uint8_t *row = wlds + pr * 128 + 32 * q;
            const uint4 a0 = *(const uint4 *)row, a1 = *(const uint4 *)(row + 16);
            sa[t][gi] = wlds[GPW * RR * 128 + pr * 4 + q];
            av[t][gi] = v8i_t{(int)a0.x, (int)a0.y, (int)a0.z, (int)a0.w, (int)a1.x, (int)a1.y, (int)a1.z, (int)a1.w};
        }
        inv[gi] = I8 ? *(const float *)(wlds + GPW * RR * 128 + (gi * RR + RS * (q < MR ? q : MR - 1) + 2) * 4)
                     : 0.0f;
    }
    if constexpr (MR > 4) __syncthreads();  // every wave's fragments read: the windows become the partials
    // Strips in pairs with two register sets (ping-pong): a copy of the next
    // strip's registers into the current ones would wait for their loads.
    F4Slab<CPL, GPW> cur2;
    F4EpiIn<MR, CPL, BF16> ein2;
    int it = 0;
    // PRE: the next strip's loads first, unconditional (loads under a branch
    // are waited for at the branch's end, which would serialise them with this
    // strip's work); the last strip of the workgroup loads nothing.
    auto strip = [&](F4Slab<CPL, GPW> &cu, F4EpiIn<MR, CPL, BF16> &ec, F4Slab<CPL, GPW> &nx,
                     F4EpiIn<MR, CPL, BF16> &en, auto PRE_) __attribute__((always_inline)) {
        const int sn = s + (int)gridDim.x;
        if constexpr (decltype(PRE_)::value) {
            nx.load(B, S, N, groups, g0w, q, sn * 16 * CPL + CPL * c);
            en.load(Other, Bias, postop, out_f32, M, N, q, sn * 16 * CPL + CPL * c, wave == (it + 1) % W);
        }
        float acc[RSETS][CPL][P];
#pragma unroll
        for (int t = 0; t < RSETS; ++t)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int i = 0; i < P; ++i) acc[t][j][i] = 0.0f;
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            if (g0w + gi >= groups) break;  // uniform across the wave
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                uint32_t d0, d1, e0, e1;
                if constexpr (I8) {
                    f4_decode_s2(cu.w[gi][0].v[j], d0, d1);
                    f4_decode_s2(cu.w[gi][1].v[j], e0, e1);
                } else {
                    f4_decode(cu.w[gi][0].v[j], d0, d1);
                    f4_decode(cu.w[gi][1].v[j], e0, e1);
                }
                const v8i_t bv = {(int)d0, (int)d1, (int)e0, (int)e1, 0, 0, 0, 0};
                const float sc = dt2f<BF16>(cu.scale(gi, j));
#pragma unroll
                for (int t = 0; t < RSETS; ++t) {
                    const f32x4_t d = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                        av[t][gi], bv, f32x4_t{0.f, 0.f, 0.f, 0.f}, 0 /*A e4m3*/, 4 /*B e2m1*/, 0, sa[t][gi], 0, 127);
                    if constexpr (I8) {
                        const float dot = (d[0] + d[1]) * 0.5f;  // the group's int32 dot product
                        acc[t][j][0] += dot * (sc * inv[gi]);
                    } else {
#pragma unroll
                        for (int i = 0; i < P; ++i) acc[t][j][i] = d[i] * sc + acc[t][j][i];
                    }
                }
            }
        }
        float *rb = red + (size_t)(it & 1) * W * CPL * MR * 16;
        if (q < QV) {  // lane q: the pieces of rows q + 4t
#pragma unroll
            for (int t = 0; t < RSETS; ++t)
#pragma unroll
                for (int j = 0; j < CPL; ++j) {
                    float out = acc[t][j][0];
                    if constexpr (!I8) {
#pragma unroll
                        for (int i = 1; i < P; ++i) out += acc[t][j][i];
                        out *= 0.5f;  // the fp4 operand held 2v
                    }
                    rb[((wave * CPL + j) * MR + q + 4 * t) * 16 + c] = out;
                }
        }
        __syncthreads();
        if constexpr (!KS) {
            if (wave == it % W && q < QV) {  // (wave-uniform) this strip's reducer, lane q rows q + 4t
#pragma unroll
                for (int t = 0; t < RSETS; ++t) {
                    const int m = q + 4 * t;
                    float sum[CPL];
#pragma unroll
                    for (int j = 0; j < CPL; ++j) sum[j] = rb[(j * MR + m) * 16 + c];
                    for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
                        for (int j = 0; j < CPL; ++j) sum[j] += rb[((w2 * CPL + j) * MR + m) * 16 + c];
                    const size_t o0 = (size_t)m * N + s * 16 * CPL + CPL * c;
                    if (m < M)
                        epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
                            constexpr int PO = decltype(P_)::value;
                            constexpr bool F32 = decltype(F_)::value;
#pragma unroll
                            for (int j = 0; j < CPL; ++j) {
                                const float r = epi_apply_c<PO>(sum[j], ec.other(t, j), ec.bias(j, F32));
                                if constexpr (F32) ((float *)C)[o0 + j] = r;
                                else ((uint16_t *)C)[o0 + j] = (uint16_t)f2dt<BF16>(r);
                            }
                        });
                }
            }
        } else if (wave == it % W && q < QV) {  // (wave-uniform) the reducer, then the K-slice handoff
            const int n0 = s * 16 * CPL + CPL * c;
            float sum[RSETS][CPL];
#pragma unroll
            for (int t = 0; t < RSETS; ++t) {
                const int m = q + 4 * t;
#pragma unroll
                for (int j = 0; j < CPL; ++j) sum[t][j] = rb[(j * MR + m) * 16 + c];
                for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
                    for (int j = 0; j < CPL; ++j) sum[t][j] += rb[((w2 * CPL + j) * MR + m) * 16 + c];
            }
            bool last;  // the K-slice handoff of the kernel above, for strip s
            {
#pragma unroll
                for (int t = 0; t < RSETS; ++t) {
                    const int m = q + 4 * t;
                    if (m < M)
#pragma unroll
                        for (int j = 0; j < CPL; ++j)
                            __hip_atomic_store(part + ((size_t)ks * M + m) * N + n0 + j, sum[t][j], __ATOMIC_RELAXED,
                                               __HIP_MEMORY_SCOPE_AGENT);
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __builtin_amdgcn_s_waitcnt(0);
                last = split_arrive(cnt + s, ksn, lane) == (uint32_t)(ksn - 1);
                if (last) {
                    for (int s0 = 0; s0 < ksn; s0 += 4) {
                        float v[4][RSETS][CPL];
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            const int s2 = s0 + u < ksn ? s0 + u : ksn - 1;
#pragma unroll
                            for (int t = 0; t < RSETS; ++t) {
                                const int m = q + 4 * t < M ? q + 4 * t : M - 1;
#pragma unroll
                                for (int j = 0; j < CPL; ++j)
                                    v[u][t][j] = __hip_atomic_load(part + ((size_t)s2 * M + m) * N + n0 + j,
                                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                            }
                        }
#pragma unroll
                        for (int u = 0; u < 4; ++u) {
                            if (s0 + u >= ksn) break;
#pragma unroll
                            for (int t = 0; t < RSETS; ++t)
#pragma unroll
                                for (int j = 0; j < CPL; ++j)
                                    sum[t][j] = s0 + u == 0 ? v[u][t][j] : sum[t][j] + v[u][t][j];
                        }
                    }
                }
            }
            if (last)
#pragma unroll
                for (int t = 0; t < RSETS; ++t) {
                    const int m = q + 4 * t;
                    const size_t o0 = (size_t)m * N + n0;
                    if (m < M)
                        epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
                            constexpr int PO = decltype(P_)::value;
                            constexpr bool F32 = decltype(F_)::value;
#pragma unroll
                            for (int j = 0; j < CPL; ++j) {
                                const float r = epi_apply_c<PO>(sum[t][j], ec.other(t, j), ec.bias(j, F32));
                                if constexpr (F32) ((float *)C)[o0 + j] = r;
                                else ((uint16_t *)C)[o0 + j] = (uint16_t)f2dt<BF16>(r);
                            }
                        });
                }
        }
        ++it;
        s = sn;
    };
    const int G = (int)gridDim.x;
    for (;;) {  // (uniform tests)
        if (s + G >= strips) {
            strip(cur, ein, cur2, ein2, std::false_type{});
            break;
        }
        strip(cur, ein, cur2, ein2, std::true_type{});
        if (s + G >= strips) {
            strip(cur2, ein2, cur, ein, std::false_type{});
            break;
        }
        strip(cur2, ein2, cur, ein, std::true_type{});
    }
}

struct F4Plan {
    int cpl, waves, gpw, mr;
    size_t lds;
    int windows = 1;           // LDS windows per workgroup (its K slice / (waves x gpw))
    int ks = 1;                // K slices (workgroups per strip)
    float *part = nullptr;     // ks > 1: slice sums fp32 [ks][M][N] ...
    uint32_t *cnt = nullptr;   // ... and a counter per strip (workspace)
};

constexpr size_t kF4MaxLds = 96 * 1024;
// The automatic plan of a GEMV takes the multi-strip kernel from this many
// 32-column strips on, i.e. past the 128 that put one per-strip workgroup of
// 16 columns on each CU (graph-timed against the one-strip kernel, fp16: K = N
// = 4096, 128 strips, 4.12 against 3.97 us; N = 4224 (132 strips): K = 4096
// M = 1 / 4 / 8 4.17 / 5.87 / 9.45 against 5.46 / 8.40 / 11.54 us, K = 8192
// 5.64 / 8.50 against 8.19 / 12.03, K = 2048 3.62 / 4.25 against 4.46 /
// 4.99; K = 6144 N = 5120 5.16 against 6.85 us; K = 5120 N = 248320 72.0
// against 100.8 us).
constexpr int kF4msMinStrips = 129;
constexpr int kF4msCpl = 2;  // its columns per lane (4: too many registers, measured slower)
constexpr size_t kF4msMaxLds = 160 * 1024;  // a workgroup's LDS on gfx950

int f4_mr(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : 8; }

size_t f4_lds(int MR, int waves, int gpw, int cpl, int groups) {
    const int rr = kF4RowStride * MR;
    const int gw = waves * gpw, windows = (groups + gw - 1) / gw;
    const size_t stage = (size_t)(windows > 1 ? 2 : 1) * waves * f4_window_bytes(rr, gpw);
    return stage + (size_t)(waves - 1) * cpl * MR * 16 * 4;
}

// Automatic tile: 2 columns per lane (32-column strips) when that still gives
// >= 384 workgroups, else 1; then waves x groups-per-wave (<= 4) covering a
// K slice (ks slices) with the fewest idle group slots, then the fewest windows.
F4Plan f4_plan(bool bf16, int M, int N, int K, int waves, int cpl, int gpw, int ks = 1) {
    const int MR = f4_mr(M), groups = (K / kGS + ks - 1) / ks;
    F4Plan p;
    p.mr = MR;
    p.ks = ks;
    p.cpl = cpl > 0 ? cpl : ((N % 32 == 0 && N / 32 >= 384) ? 2 : 1);
    int bw = 8, bg = 1;
    long best = LONG_MIN;
    for (int g : {1, 2, 4, 8, 16}) {
        if (gpw > 0 && g != gpw) continue;
        if (MR * g > 16) continue;      // staging registers: MR * GPW / 4 tasks per lane
        if (p.cpl * g > 16) continue;   // weight registers: 2 * CPL * GPW words per lane
        // more than 8 waves only pays for long K (measured: K = 14336 gains,
        // K = 4096 loses)
        const int wmax = (waves > 0 || groups > 64) ? f4_max_waves(MR, p.cpl) : 8;
        for (int w = 1; w <= wmax; ++w) {
            if (waves > 0 && w != waves) continue;
            if (f4_lds(MR, w, g, p.cpl, groups) > kF4MaxLds) continue;
            const int gw = w * g, windows = (groups + gw - 1) / gw;
            const int idle = windows * gw - groups;
            // fewest idle group slots, then fewest windows, then more waves;
            // automatic tiles keep <= 4 groups per wave (measured best)
            if (gpw == 0 && g > 4) continue;
            const long score = -(long)idle * 100000 - (long)windows * 100 + w;
            if (score > best) { best = score; bw = w; bg = g; }
        }
    }
    p.waves = bw;
    p.gpw = bg;
    p.lds = f4_lds(MR, bw, bg, p.cpl, groups);
    p.windows = (groups + bw * bg - 1) / (bw * bg);
    return p;
}

template <int MR, int CPL, int GPW, bool BF16, int QMODE = 0>
hipError_t f4_launch_t(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    if constexpr (kF4RowStride * MR > 32) {
        return hipErrorInvalidValue;
    } else {
        const int strips = N / (16 * CPL);
        const int swz = (CPL == 1 && strips % 16 == 0) ? 1 : 0;
        // (several windows: the form that keeps the next window's loads in flight)
        if (p.windows > 1)
            hipLaunchKernelGGL((k_int2_gemv_f4<MR, CPL, GPW, BF16, false, QMODE, false, true>), dim3(strips, p.ks),
                               dim3(64 * p.waves), p.lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C,
                               (const uint16_t *)Other, Bias, M, N, K, postop, out_f32, swz, F4Group{}, nullptr, 0,
                               p.ks, p.part, p.cnt);
        else
            hipLaunchKernelGGL((k_int2_gemv_f4<MR, CPL, GPW, BF16, false, QMODE>), dim3(strips, p.ks),
                               dim3(64 * p.waves), p.lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C,
                               (const uint16_t *)Other, Bias, M, N, K, postop, out_f32, swz, F4Group{}, nullptr, 0,
                               p.ks, p.part, p.cnt);
        return hipGetLastError();
    }
}

template <int MR, int CPL, bool BF16, int QMODE = 0>
hipError_t f4_launch_g(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    switch (p.gpw) {
    case 1: return f4_launch_t<MR, CPL, 1, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return f4_launch_t<MR, CPL, 2, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 4:  // (groups per wave x rows <= 16: the host checks)
        if constexpr (MR <= 4) return f4_launch_t<MR, CPL, 4, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        return hipErrorInvalidValue;
    case 8:
        if constexpr (MR <= 2 && CPL <= 2) return f4_launch_t<MR, CPL, 8, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        return hipErrorInvalidValue;
    default:
        if constexpr (MR == 1 && CPL == 1) return f4_launch_t<MR, CPL, 16, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        return hipErrorInvalidValue;
    }
}

template <int MR, bool BF16, int QMODE = 0>
hipError_t f4_launch_c(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    if (p.cpl == 4) return f4_launch_g<MR, 4, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    if (p.cpl == 2) return f4_launch_g<MR, 2, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return f4_launch_g<MR, 1, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
}

template <bool BF16, int QMODE = 0>
hipError_t f4_launch(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C,
                     const void *Other, const void *Bias, int M, int N, int K, int postop,
                     int out_f32, hipStream_t st) {
    switch (p.mr) {
    case 1: return f4_launch_c<1, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return f4_launch_c<2, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 4: return f4_launch_c<4, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    default: return f4_launch_c<8, BF16, QMODE>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
}

// QM 3: the down GEMV of the decode layer (A = fp32 gate rows, up rows
// up_off floats further).  DS: one workgroup per (strip, token), a wave per slot.
template <int CPL, int GPW, bool BF16, int QM, bool DS>
hipError_t f4_group_launch_t(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C,
                             int rows, int N, int K, const F4Group &grp, int up_off, hipStream_t st) {
    const int strips = N / (16 * CPL);
    hipLaunchKernelGGL((k_int2_gemv_f4<1, CPL, GPW, BF16, true, QM, DS>), dim3(strips, rows), dim3(64 * p.waves),
                       p.lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C, nullptr, nullptr, 1, N, K, 0, 1,
                       0, grp, nullptr, up_off);
    return hipGetLastError();
}

template <bool BF16, int QM, bool DS>
hipError_t f4_group_launch(const F4Plan &p, const void *A, const uint32_t *B, const void *S, void *C, int rows,
                           int N, int K, const F4Group &grp, int up_off, hipStream_t st) {
    if (!DS && p.cpl == 2) {
        switch (p.gpw) {
        case 1: return f4_group_launch_t<2, 1, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
        case 2: return f4_group_launch_t<2, 2, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
        default: return f4_group_launch_t<2, 4, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
        }
    }
    switch (p.gpw) {
    case 1: return f4_group_launch_t<1, 1, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
    case 2: return f4_group_launch_t<1, 2, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
    default: return f4_group_launch_t<1, 4, BF16, QM, DS>(p, A, B, S, C, rows, N, K, grp, up_off, st);
    }
}

// The s8 x s2 GEMV launches: QM 1 (A = Aq, int8) or 2 (A = DT, quantized
// while staged); tiles of <= 2 columns per lane and <= 4 groups per wave.
template <int MR, int CPL, int GPW, bool BF16, int QM>
hipError_t f4q_launch_t(const F4Plan &p, const void *A, const void *SA, int ldsa, const uint32_t *B,
                        const void *S, void *C, const void *Other, const void *Bias, int M, int N, int K,
                        int postop, int out_f32, hipStream_t st) {
    const int strips = N / (16 * CPL);
    const int swz = (CPL == 1 && strips % 16 == 0) ? 1 : 0;
    if (p.windows > 1)
        hipLaunchKernelGGL((k_int2_gemv_f4<MR, CPL, GPW, BF16, false, QM, false, true>), dim3(strips, p.ks),
                           dim3(64 * p.waves), p.lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C,
                           (const uint16_t *)Other, Bias, M, N, K, postop, out_f32, swz, F4Group{}, (const uint16_t *)SA,
                           ldsa, p.ks, p.part, p.cnt);
    else
        hipLaunchKernelGGL((k_int2_gemv_f4<MR, CPL, GPW, BF16, false, QM>), dim3(strips, p.ks), dim3(64 * p.waves),
                           p.lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M,
                           N, K, postop, out_f32, swz, F4Group{}, (const uint16_t *)SA, ldsa, p.ks, p.part, p.cnt);
    return hipGetLastError();
}

template <int MR, bool BF16, int QM>
hipError_t f4q_launch_m(const F4Plan &p, const void *A, const void *SA, int ldsa, const uint32_t *B,
                        const void *S, void *C, const void *Other, const void *Bias, int M, int N, int K,
                        int postop, int out_f32, hipStream_t st) {
#define TCL_F4Q(CPL, GPW) \
    return f4q_launch_t<MR, CPL, GPW, BF16, QM>(p, A, SA, ldsa, B, S, C, Other, Bias, M, N, K, postop, out_f32, st)
    switch (p.cpl * 10 + p.gpw) {
    case 11: TCL_F4Q(1, 1);
    case 12: TCL_F4Q(1, 2);
    case 14: TCL_F4Q(1, 4);
    case 21: TCL_F4Q(2, 1);
    case 22: TCL_F4Q(2, 2);
    case 24: TCL_F4Q(2, 4);
    default: return hipErrorInvalidValue;
    }
#undef TCL_F4Q
}

template <bool BF16, int QM>
hipError_t f4q_launch(const F4Plan &p, const void *A, const void *SA, int ldsa, const uint32_t *B, const void *S,
                      void *C, const void *Other, const void *Bias, int M, int N, int K, int postop, int out_f32,
                      hipStream_t st) {
    switch (p.mr) {
    case 1: return f4q_launch_m<1, BF16, QM>(p, A, SA, ldsa, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return f4q_launch_m<2, BF16, QM>(p, A, SA, ldsa, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    default: return f4q_launch_m<4, BF16, QM>(p, A, SA, ldsa, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
}

// The s8 x s2 GEMV's tile: the automatic one for ks K slices (<= 2 columns
// per lane, <= 4 groups per wave; 16 waves only with 1 column per lane and
// M = 1, which the kernel's launch bounds allow).
F4Plan f4q_plan(int M, int N, int K, int cpl = 0, int ks = 1) {
    F4Plan p = f4_plan(false, M, N, K, 0, cpl, 0, ks);
    if (p.cpl > 2 || p.gpw > 4)
        p = f4_plan(false, M, N, K, p.waves, p.cpl > 2 ? 2 : p.cpl, p.gpw > 4 ? 4 : p.gpw, ks);
    return p;
}

// Decode hook: the two fp4 dwords the kernel builds from each word,
// D[word][0] = rows 0, 2, .., 14, D[word][1] = rows 1, 3, .., 15 (e2m1 2v).
__global__ void k_int2_f4_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D, size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    uint32_t d0, d1;
    f4_decode(B[i], d0, d1);
    D[2 * i] = d0;
    D[2 * i + 1] = d1;
}

}  // namespace

// Whether the fp8 x fp4 engine takes a call: M <= 8, A 16-byte aligned (it
// reads A with 16-byte loads), and byte offsets into C, Other and Bias below
// 2^31 (its buffer loads use 32-bit offsets).
bool int2_gemv_f4_supports(int M, int N, const void *A) {
    return M >= 1 && M <= kF4MaxM && ((uintptr_t)A & 15) == 0 && (size_t)M * N * 4 < 0x7ff00000u;
}

// Workspace of a K split: one counter per column strip (at most N / 16 of
// them) in the workspace header, then the slice sums fp32 [ks][M][N] after it.
// A split whose counters would not fit the header is not taken.
bool f4_cnt_fit(int N) { return (size_t)(N / 16) * 4 <= kWsHeader; }
size_t f4_split_ws(int M, int N, int ks) { return ks > 1 ? kWsHeader + (size_t)ks * M * N * 4 : 0; }

// Slices that leave none empty: ceil(G / ceil(G / ks)).
int f4_slices(int groups, int ks) {
    const int gps = (groups + ks - 1) / ks;
    return (groups + gps - 1) / gps;
}

// Automatic K split (when the caller gives the workspace), from graph-timed
// sweeps of M = 1..8 over K = 4096..16384 and N = 1024..14336: a split pays
// only where the unsplit plan has fewer than 384 strips (one workgroup each)
// and K is long: >= 104 groups at M = 1, >= 64 at M = 2..4, >= 16 at M = 5..8
// (the staging grows with M).  About 28 groups per slice, at least 4 slices
// from 64 groups on; 16-column-wide MFMA operands shared by 4 columns per
// lane at M >= 5 (2 below).  N = 4096: K = 14336, M = 1 8.4 -> 7.6 us, M = 4
// 14.2 -> 10.4, M = 8 23.2 -> 12.2; K = 8192, M = 4 9.2 -> 7.5; K = 4096, M = 8
// 8.6 -> 7.1.  (M = 1, K = 8192..12288 loses: 5.8 -> 6.4 us at K = 8192.)
void f4_auto_split(int M, int N, int K, int cpl_req, int &cpl, int &ks) {
    const int groups = K / kGS, MR = f4_mr(M);
    const int cpl_u = cpl_req > 0 ? cpl_req : ((N % 32 == 0 && N / 32 >= 384) ? 2 : 1);
    cpl = cpl_u;
    ks = 1;
    const int gmin = MR >= 8 ? 16 : MR >= 2 ? 64 : 104;
    if (N / (16 * cpl_u) >= 384 || groups < gmin || !f4_cnt_fit(N)) return;
    const int c = cpl_req > 0 ? cpl_req : (MR >= 8 && groups >= 64 && N % 64 == 0 ? 4 : (N % 32 == 0 ? 2 : 1));
    int k = groups >= 64 ? 4 : 2;  // the power of two nearest groups / 28 (log scale), 2 .. 16
    while (k < 16 && (double)groups / 28.0 > k * 1.4142) k *= 2;
    cpl = c;
    ks = f4_slices(groups, k);
    // Slices that do not split into waves of whole groups (K = 17408: 136
    // groups / 4 = 34 = 2 x 17, planned as one group on each of 2 waves for 17
    // windows, one 16-byte load per lane in flight) take instead the slice
    // count, from 2 to 16, whose plan needs the fewest windows, the nearest to
    // k on a tie (K = 17408: 5 slices of 28 groups, 7 waves x 4 groups).
    const F4Plan p0 = f4_plan(false, M, N, K, 0, c, 0, ks);
    if (p0.waves * p0.gpw < 4) {
        int best_w = p0.windows;
        double best_d = 0.0;
        for (int kk = 2; kk <= 16; ++kk) {
            const int s = f4_slices(groups, kk);
            const F4Plan p = f4_plan(false, M, N, K, 0, c, 0, s);
            const double d = std::fabs(std::log((double)s / k));
            if (p.windows < best_w || (p.windows == best_w && d < best_d)) {
                best_w = p.windows;
                best_d = d;
                ks = s;
            }
        }
    }
}

// The multi-strip GEMV's plan for K and mr rows: groups per wave (1, 2 or 4)
// and waves (<= 16; 8 rows: <= 8) holding all of K in one window; 0 waves: K
// too long (> 64 groups; 8 rows: > 32).
void f4ms_plan(int K, int &gpw, int &waves, int mr = 1) {
    const int groups = K / kGS;
    if (mr > 4) gpw = groups > 16 ? 4 : groups > 8 ? 2 : 1;
    else gpw = groups >= 32 ? 4 : groups >= 16 ? 2 : 1;
    waves = (groups + gpw - 1) / gpw;
    if (waves > (mr > 4 ? 8 : 16)) waves = 0;
}
// Staging windows, then the double-buffered wave partials (8 rows: the
// partials in the windows' place).
size_t f4ms_lds(int mr, int gpw, int waves, int cpl) {
    const size_t win = (size_t)waves * f4_window_bytes(kF4RowStride * mr, gpw);
    const size_t red = (size_t)2 * waves * cpl * mr * 16 * 4;
    return mr > 4 ? std::max(win, red) : win + red;
}

// cpl: columns per lane (1, 2 or 4; 0 = automatic), strips of 16 cpl columns.
// Grid, from graph-timed sweeps (fp16, >2 GiB rotated): workgroups of up to 8
// waves (K <= 4096) run two per CU, min(strips, 512) of them; larger ones one
// per CU, the strips spread evenly (every workgroup ceil or floor of the
// mean): against 512 of them, K = 5120 N = 248320 70.9 -> 64.5 us, K = 7168
// N = 28672 16.5 -> 14.7, K = 8192 N = 14336 11.4 -> 9.9, K = 3072 N = 32768
// 10.0 -> 8.9; 8-wave workgroups lose that way (K = 4096 N = 151680 33.9 ->
// 36.3, K = 2048 N = 65536 10.5 -> 12.8).  8 rows: one per CU too (their
// staging windows take most of a CU's LDS).  2 to 4 rows with at most 512
// strips: one per CU as well -- a strip's staging and MFMA work grows with
// the rows, and the CUs that would hold two workgroups set the launch's
// length (same box, bf16, bias + residual, K = 4096 N = 14336, M = 2 / 3 / 4:
// 6.61 / 8.08 / 7.88 -> 6.34 / 6.90 / 7.00 us; N = 6144 level); with more
// strips two per CU stay ahead (K = 2048 N = 65536, M = 2: 10.2 against 13.6).
int f4ms_grid(int strips, int waves, int mr = 1) {
    if (waves <= 8 && mr <= 4 && (mr == 1 || strips > 512)) return std::min(strips, 512);
    const int per = (strips + 255) / 256;
    return (strips + per - 1) / per;
}

// ks > 1: K slices of the workspace's split (f4_split_ws bytes; K per slice
// within one window); gpw_req: groups per wave (0: f4ms_plan's).  Walkers per
// slice: a grid of about 512 workgroups (256 above 8 waves or 4 rows).
ternocl_status int2_gemv_f4ms_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K, int postop,
                                  int out_f32, int cpl, int gpw_req, int ks_req, void *ws, size_t ws_bytes,
                                  hipStream_t st) {
    const int mr = f4_mr(M), groups = K / kGS;
    const int ksn = ks_req > 1 ? f4_slices(groups, ks_req) : 1, gps = (groups + ksn - 1) / ksn;
    int gpw, waves;
    f4ms_plan(gps * kGS, gpw, waves, mr);
    if (gpw_req > 0) {
        gpw = gpw_req;
        waves = (gps + gpw - 1) / gpw;
        if (gpw != 1 && gpw != 2 && gpw != 4) waves = 0;
        if (waves > (mr > 4 ? 8 : 16)) waves = 0;
    }
    if (cpl == 0) cpl = N % (16 * kF4msCpl) == 0 ? kF4msCpl : N % 32 == 0 ? 2 : 1;
    if (M < 1 || M > 8 || waves == 0 || (cpl != 1 && cpl != 2 && cpl != 4) || (cpl == 4 && mr > 1) ||
        N % (16 * cpl) || f4ms_lds(mr, gpw, waves, cpl) > kF4msMaxLds) {
        set_error("the multi-strip GEMV (engine 5) takes M <= 8, K per slice <= 8192 (M > 4: <= 4096), "
                  "groups_per_wave 1, 2 or 4 with at most 16 waves, cols_per_lane 1 or 2 (4 at M = 1) and "
                  "N % (16 * cols_per_lane) == 0");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (ksn > 1 && (cpl != 2 || gpw == 1)) {
        set_error("the multi-strip GEMV over k_slices > 1 takes cols_per_lane 2 and groups_per_wave 2 or 4");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (ksn > 1 && !(f4_cnt_fit(N) && ws && ((uintptr_t)ws & 15) == 0 && ws_bytes >= f4_split_ws(M, N, ksn))) {
        set_error("k_slices > 1 needs a 16-byte aligned workspace of ternocl_int2_gemm_ws_bytes() bytes for "
                  "that split (and at most 16384 column strips)");
        return TERNOCL_ERR_WORKSPACE;
    }
    const int strips = N / (16 * cpl);
    const int walkers = ksn > 1 ? std::min(strips, std::max(1, (waves > 8 || mr > 4 ? 256 : 512) / ksn))
                                : f4ms_grid(strips, waves, mr);
    const dim3 grid(walkers, ksn), block(64 * waves);
    const size_t lds = f4ms_lds(mr, gpw, waves, cpl);
    const uint16_t *a = (const uint16_t *)A, *s = (const uint16_t *)S, *o = (const uint16_t *)Other;
    float *part = ksn > 1 ? (float *)((uint8_t *)ws + kWsHeader) : nullptr;
    uint32_t *cnt = ksn > 1 ? (uint32_t *)ws : nullptr;
#define TCL_F4MS(R, G, CP, BF)                                                                                 \
    hipLaunchKernelGGL((k_int2_gemv_f4ms<R, G, CP, BF>), grid, block, lds, st, a, B, s, C, o, Bias, M, N, K,  \
                       postop, out_f32)
#define TCL_F4MS_KS(R, G, BF)                                                                                  \
    hipLaunchKernelGGL((k_int2_gemv_f4ms<R, G, 2, BF, 0, true>), grid, block, lds, st, a, B, s, C, o, Bias, M, \
                       N, K, postop, out_f32, nullptr, 0, ksn, part, cnt)
#define TCL_F4MS_G(R, CP, BF)                \
    do {                                     \
        if (gpw == 4) TCL_F4MS(R, 4, CP, BF);     \
        else if (gpw == 2) TCL_F4MS(R, 2, CP, BF); \
        else TCL_F4MS(R, 1, CP, BF);         \
    } while (0)
#define TCL_F4MS_KR(BF)                                             \
    do {                                                            \
        if (mr == 1) {                                              \
            if (gpw == 4) TCL_F4MS_KS(1, 4, BF);                    \
            else TCL_F4MS_KS(1, 2, BF);                             \
        } else if (mr == 2) {                                       \
            if (gpw == 4) TCL_F4MS_KS(2, 4, BF);                    \
            else TCL_F4MS_KS(2, 2, BF);                             \
        } else if (mr == 4) {                                       \
            if (gpw == 4) TCL_F4MS_KS(4, 4, BF);                    \
            else TCL_F4MS_KS(4, 2, BF);                             \
        } else {                                                    \
            if (gpw == 4) TCL_F4MS_KS(8, 4, BF);                    \
            else TCL_F4MS_KS(8, 2, BF);                             \
        }                                                           \
    } while (0)
#define TCL_F4MS_R(BF)                                                    \
    do {                                                                  \
        if (mr == 1) {                                                    \
            if (cpl == 4) TCL_F4MS_G(1, 4, BF);                           \
            else if (cpl == 2) TCL_F4MS_G(1, 2, BF);                      \
            else TCL_F4MS_G(1, 1, BF);                                    \
        } else if (mr == 2) {                                             \
            if (cpl == 2) TCL_F4MS_G(2, 2, BF);                           \
            else TCL_F4MS_G(2, 1, BF);                                    \
        } else if (mr == 4) {                                             \
            if (cpl == 2) TCL_F4MS_G(4, 2, BF);                           \
            else TCL_F4MS_G(4, 1, BF);                                    \
        } else {                                                          \
            if (cpl == 2) TCL_F4MS_G(8, 2, BF);                           \
            else TCL_F4MS_G(8, 1, BF);                                    \
        }                                                                 \
    } while (0)
    if (ksn > 1) {
        if (dtype == TERNOCL_BF16) TCL_F4MS_KR(true);
        else TCL_F4MS_KR(false);
    } else if (dtype == TERNOCL_BF16) {
        TCL_F4MS_R(true);
    } else {
        TCL_F4MS_R(false);
    }
#undef TCL_F4MS_KR
#undef TCL_F4MS_R
#undef TCL_F4MS_G
#undef TCL_F4MS_KS
#undef TCL_F4MS
    return launch_status(hipGetLastError());
}

// Whether the automatic choice for a GEMV of M <= 4 rows is the multi-strip
// kernel: many strips per CU (the staging it saves grows with them) and all
// of K in one window.  Graph-timed against the per-strip engine's automatic
// plan (fp16, >2 GiB rotated), M = 2 / 4: K = 4096 N = 151680 47.0 / 57.2 ->
// 32.3 / 32.4 us, K = 5120 N = 248320 110.7 / 226.2 -> 65.5 / 65.1, K = 5120
// N = 34816 19.3 / 37.3 -> 13.2 / 14.7, K = 4096 N = 14336 (bf16, bias +
// residual) 6.82 / 8.14 -> 6.46 / 7.63, K = 4096 N = 6144 6.19 / 8.16 -> 4.96 /
// 5.98; below 160 strips the per-strip engine's K split wins (K = 8192 N =
// 4096: 6.33 / 7.18 against 6.69 / 8.42).  5..8 rows (K <= 4096, one
// workgroup per CU), the same rule; M = 5 / 8 against the per-strip engine:
// K = 4096 N = 151680 101.6 -> 49.7 us (M = 8), N = 24576 19.3 / 18.9 -> 14.5 /
// 14.6, N = 14336 11.2 / 11.4 -> 11.1 / 11.1, N = 6144 11.6 -> 9.5, K = 3072
// N = 32768 19.7 / 19.1 -> 15.3 / 15.4; N = 4096 (128 strips) 7.2 against 9.3.
bool int2_gemv_f4ms_auto(int M, int N, int K) {
    const int mr = f4_mr(M);
    int gpw, waves;
    f4ms_plan(K, gpw, waves, mr);
    const int strips = N % (16 * kF4msCpl) == 0 ? N / (16 * kF4msCpl) : 0;
    return M >= 1 && M <= 8 && waves > 0 && strips >= kF4msMinStrips &&
           f4ms_lds(mr, gpw, waves, kF4msCpl) <= kF4msMaxLds;
}

// Workspace bytes of the automatic plan (0: no K split; the multi-strip
// kernel takes none).
size_t int2_gemv_f4_ws_need(int M, int N, int K) {
    if (M < 1 || M > kF4MaxM || N < 16 || N % 16 || K < kGS || K % kGS) return 0;
    if (int2_gemv_f4ms_auto(M, N, K)) return 0;
    int cpl, ks;
    f4_auto_split(M, N, K, 0, cpl, ks);
    return f4_split_ws(M, N, ks);
}

ternocl_status int2_gemv_f4_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                const void *Other, const void *Bias, int M, int N, int K, int postop,
                                int out_f32, int waves, int cpl, int gpw, int ks, void *ws, size_t ws_bytes,
                                hipStream_t st) {
    const bool bf16 = dtype == TERNOCL_BF16;
    if (M > kF4MaxM) {
        set_error("the fp8 x fp4 GEMV takes M <= 8");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if ((size_t)M * N * 4 >= 0x7ff00000u) {
        set_error("the fp8 x fp4 GEMV takes M * N * 4 < 2^31 bytes of output");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (cpl != 0 && cpl != 1 && cpl != 2 && cpl != 4) {
        set_error("cols_per_lane must be 0 (automatic), 1, 2 or 4");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (gpw != 0 && gpw != 1 && gpw != 2 && gpw != 4 && gpw != 8 && gpw != 16) {
        set_error("groups_per_wave must be 0 (automatic), 1, 2, 4, 8 or 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (gpw * f4_mr(M) > 16 || gpw * (cpl ? cpl : 1) > 16) {
        set_error("groups_per_wave * (M rounded up to a power of two) and groups_per_wave * "
                  "cols_per_lane must be <= 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (waves < 0 || waves > 16) {
        set_error("waves must be 0 (automatic) .. 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (((uintptr_t)A & 15) != 0) {
        set_error("the fp8 x fp4 GEMV reads A with 16-byte loads: A must be 16-byte aligned");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (ks < 0 || ks > 16) {
        set_error("k_slices must be 0 (automatic) .. 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const bool ws_ok = ws && ((uintptr_t)ws & 15) == 0;
    int pc = cpl, pk = ks > 0 ? f4_slices(K / kGS, ks) : 1;
    if (ks == 0) {  // automatic: split where the workspace holds it, else one slice
        f4_auto_split(M, N, K, cpl, pc, pk);
        if (pk > 1 && !(ws_ok && ws_bytes >= f4_split_ws(M, N, pk))) {
            pk = 1;
            pc = cpl;
        }
    } else if (pk > 1 && !f4_cnt_fit(N)) {
        set_error("k_slices > 1 takes at most 16384 column strips (the workspace header's counters)");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    } else if (pk > 1 && !(ws_ok && ws_bytes >= f4_split_ws(M, N, pk))) {
        set_error("k_slices > 1 needs a 16-byte aligned workspace of ternocl_int2_gemm_ws_bytes() bytes "
                  "for that split");
        return TERNOCL_ERR_WORKSPACE;
    }
    F4Plan p = f4_plan(bf16, M, N, K, waves, pc, gpw, pk);
    if (pk > 1) {
        p.cnt = (uint32_t *)ws;
        p.part = (float *)((uint8_t *)ws + kWsHeader);
    }
    if (p.waves > f4_max_waves(p.mr, p.cpl)) {
        set_error("more than 8 waves per workgroup only for M = 1 with 16-column strips (cols_per_lane 1)");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (N % (16 * p.cpl)) {
        set_error("N must be a multiple of 16 * cols_per_lane");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (p.lds > kF4MaxLds) {
        set_error("GEMV tile needs more than 96 KiB of LDS: use fewer waves or groups per wave");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const hipError_t e = bf16 ? f4_launch<true>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st)
                              : f4_launch<false>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return launch_status(e);
}

// The decode-removed variant (QM 4) with the plan int2_gemv_f4_run would use
// for the same shape: the memory ceiling of the engine (a measurement).
ternocl_status int2_gemv_stream_probe_run(int dtype, const uint32_t *B, const void *S, void *C, int M, int N,
                                          int K, hipStream_t st) {
    const bool bf16 = dtype == TERNOCL_BF16;
    if (M < 1 || M > kF4MaxM || (size_t)M * N * 4 >= 0x7ff00000u) {
        set_error("the decode-removed GEMV takes M <= 8 and M * N * 4 < 2^31 bytes of output");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    const F4Plan p = f4_plan(bf16, M, N, K, 0, 0, 0);
    if (N % (16 * p.cpl) || p.lds > kF4MaxLds) {
        set_error("N must be a multiple of 16 * cols_per_lane");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    // (C fp32: postop 0, out_f32 1)
    const hipError_t e = bf16 ? f4_launch<true, 4>(p, nullptr, B, S, C, nullptr, nullptr, M, N, K, 0, 1, st)
                              : f4_launch<false, 4>(p, nullptr, B, S, C, nullptr, nullptr, M, N, K, 0, 1, st);
    return launch_status(e);
}

// Whether the s8 x s2 GEMV takes a call: M <= 4; N a multiple of 16 (32 when
// the tile takes 2 columns per lane); Aq 8-byte or A 16-byte aligned; C,
// Other and Bias byte offsets below 2^31.
bool int2_int8_gemv_supports(int M, int N, int K, const void *A, const int8_t *Aq) {
    if (M < 1 || M > kF4MaxMI8 || N % 16 || (size_t)M * N * 4 >= 0x7ff00000u) return false;
    if (Aq ? ((uintptr_t)Aq & 7) != 0 : ((uintptr_t)A & 15) != 0) return false;
    const F4Plan p = f4q_plan(M, N, K);
    return N % (16 * p.cpl) == 0 && p.lds <= kF4MaxLds;
}

// The automatic K split of the s8 x s2 GEMV: the DT GEMV's rule (M <= 4
// keeps it to <= 2 columns per lane); 1 where it does not split.
static int f4q_auto_split(int M, int N, int K, int &cpl) {
    int ks;
    f4_auto_split(M, N, K, 0, cpl, ks);
    if (ks > 1 && (cpl > 2 || N % (16 * cpl))) {
        cpl = 0;
        ks = 1;
    }
    if (ks == 1) cpl = 0;
    return ks;
}

size_t int2_int8_gemv_ws_need(int M, int N, int K) {
    if (M < 1 || M > kF4MaxMI8 || N < 16 || N % 16 || K < kGS || K % kGS) return 0;
    if (int2_gemv_f4ms_auto(M, N, K)) return 0;  // the multi-strip kernel takes none
    int cpl;
    return f4_split_ws(M, N, f4q_auto_split(M, N, K, cpl));
}

// ws (16-byte aligned, int2_int8_gemv_ws_need bytes, zeroed once before its
// first use): the automatic K split; NULL or short: one slice.
// The multi-strip kernel in an int8 mode (QM 1: A = Aq int8, 2: A = DT
// quantized while staged), 32-column strips; the host has checked
// int2_gemv_f4ms_auto(M, N, K).
template <int QM, bool BF16>
static hipError_t f4ms_q_launch(const void *A, const void *SA, int ldsa, const uint32_t *B, const void *S, void *C,
                                const void *Other, const void *Bias, int M, int N, int K, int postop, int out_f32,
                                hipStream_t st) {
    int gpw, waves;
    f4ms_plan(K, gpw, waves);
    const int mr = M <= 1 ? 1 : M <= 2 ? 2 : 4, strips = N / 32;
    // (the rows count in the grid rule here too: M = 2 / 3 / 4 at K = 4096
    // N = 14336, 7.24 / 8.1 / 8.15 -> 7.06 / 7.46 / 7.47 us)
    const dim3 grid(f4ms_grid(strips, waves, mr)), block(64 * waves);
    const size_t lds = f4ms_lds(mr, gpw, waves, 2);
    auto go = [&](auto R_, auto G_) {
        hipLaunchKernelGGL((k_int2_gemv_f4ms<decltype(R_)::value, decltype(G_)::value, 2, BF16, QM>), grid, block,
                           lds, st, (const uint16_t *)A, B, (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M,
                           N, K, postop, out_f32, (const uint16_t *)SA, ldsa);
    };
    auto rows = [&](auto G_) {
        if (mr == 1) go(std::integral_constant<int, 1>{}, G_);
        else if (mr == 2) go(std::integral_constant<int, 2>{}, G_);
        else go(std::integral_constant<int, 4>{}, G_);
    };
    if (gpw == 4) rows(std::integral_constant<int, 4>{});
    else if (gpw == 2) rows(std::integral_constant<int, 2>{});
    else rows(std::integral_constant<int, 1>{});
    return hipGetLastError();
}

ternocl_status int2_int8_gemv_run(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                  const uint32_t *B, const void *SB, void *C, const void *Other,
                                  const void *Bias, int M, int N, int K, int postop, int out_f32,
                                  hipStream_t st, void *ws, size_t ws_bytes) {
    if (!int2_int8_gemv_supports(M, N, K, A, Aq)) {
        set_error("the s8 x s2 GEMV takes M <= 4, N % 16 == 0 and aligned activations");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (int2_gemv_f4ms_auto(M, N, K)) {  // many strips: the multi-strip kernel, as the int2 GEMV
        const int ldsa = (M + 31) & ~31;
        const bool bf = dtype == TERNOCL_BF16;
        hipError_t e;
        if (Aq)
            e = bf ? f4ms_q_launch<1, true>(Aq, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
                   : f4ms_q_launch<1, false>(Aq, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st);
        else
            e = bf ? f4ms_q_launch<2, true>(A, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
                   : f4ms_q_launch<2, false>(A, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st);
        return launch_status(e);
    }
    int cpl = 0, ks = f4q_auto_split(M, N, K, cpl);
    if (ks > 1 && !(ws && ((uintptr_t)ws & 15) == 0 && ws_bytes >= f4_split_ws(M, N, ks))) {
        ks = 1;
        cpl = 0;
    }
    F4Plan p = f4q_plan(M, N, K, cpl, ks);
    if (ks > 1 && p.lds <= kF4MaxLds) {
        p.cnt = (uint32_t *)ws;
        p.part = (float *)((uint8_t *)ws + kWsHeader);
    } else if (ks > 1) {
        p = f4q_plan(M, N, K);
    }
    const int ldsa = (M + 31) & ~31;
    const bool bf16 = dtype == TERNOCL_BF16;
    hipError_t e;
    if (Aq)
        e = bf16 ? f4q_launch<true, 1>(p, Aq, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
                 : f4q_launch<false, 1>(p, Aq, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st);
    else
        e = bf16 ? f4q_launch<true, 2>(p, A, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
                 : f4q_launch<false, 2>(p, A, SA, ldsa, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st);
    return launch_status(e);
}

// The grouped GEMVs of the MoE decode: C fp32 [rows][N], rows = G (one weight
// set) or 2G (B / S for pairs 0..G-1, B2 / S2 for G..2G-1); A rows of K, row
// g / adiv for pair g; experts ids[g] of [E][K/16][N] weights.  Tiles: the
// M = 1 tile with 2 columns per lane where N % 32 == 0 (else 1) and 4 groups
// per wave where K / 128 is a multiple of 4 (else the automatic count, at most
// 4).  The launch has a workgroup per strip and row: the wider strips halve
// the workgroups each row's activations are staged in, and 4 groups per wave
// halve a workgroup's waves.  The MoE decode layer at T = 1, E = 128, top-8,
// H = 2048, I = 768 (same box, the same bits): 1 column per lane 11.54 us,
// 2 columns 10.66 us; then at 2 columns, (waves x groups per wave) 8 x 2
// 10.67, 4 x 4 10.13, 4 x 2 10.46, 2 x 4 10.84, 8 x 1 11.36 us.
static F4Plan f4_group_plan(int N, int K) {
    F4Plan p = f4_plan(false, 1, N, K, 0, N % 32 == 0 ? 2 : 0, (K / kGS) % 4 == 0 ? 4 : 0);
    if (p.cpl > 2 || p.gpw > 4 || p.waves > 8) p = f4_plan(false, 1, N, K, 8, p.cpl > 2 ? 2 : p.cpl, p.gpw > 4 ? 4 : p.gpw);
    return p;
}

// The down launch with the weighted sum (DS): topk waves (<= 16), one column
// per lane, each wave's groups in windows of up to 4.
static F4Plan f4_down_sum_plan(int K, int topk) {
    const int groups = K / kGS;
    F4Plan p;
    p.mr = 1;
    p.cpl = 1;
    p.waves = topk;
    p.gpw = groups >= 3 ? 4 : groups;
    const int windows = (groups + p.gpw - 1) / p.gpw;
    p.lds = (size_t)(windows > 1 ? 2 : 1) * topk * f4_window_bytes(kF4RowStride, p.gpw) + (size_t)topk * 16 * 4;
    return p;
}

// The decode layer's grouped GEMVs (fp32 weights of the MoE experts [E][K/16][N]):
// mode 0, gate/up: C [2G][N] = rows of X (row g / topk for pair g) times gate
//   (rows < G) or up (B2 / S2, rows >= G) of expert ids[g];
// mode 1, down: C [G][N] = h times down, h = DT(silu(gate) * up) staged from
//   the fp32 rows A = mode 0's C;
// mode 2, down with the weighted sum (topk <= 16): O [T][N] directly.
ternocl_status int2_gemv_f4_group_run(int dtype, const void *A, const int *ids, int G, int E, int topk,
                                      const uint32_t *B, const void *S, const uint32_t *B2, const void *S2,
                                      float *C, int N, int K, const void *RW, void *O, int mode,
                                      hipStream_t st) {
    const bool bf16 = dtype == TERNOCL_BF16;
    const F4Plan p = mode == 2 ? f4_down_sum_plan(K, topk) : f4_group_plan(N, K);
    if (N % (16 * p.cpl) || p.lds > kF4MaxLds || (mode == 2 && (topk < 1 || topk > 16))) {
        set_error("grouped GEMV: N must be a multiple of 16, the tile must fit in LDS, topk <= 16 for the fused sum");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    const F4Group grp{ids, G, E, mode == 0 ? topk : 1, B2, (const uint16_t *)S2, topk, (const uint16_t *)RW,
                      (uint16_t *)O};
    const int up_off = G * K;  // modes 1, 2: floats from a gate row to its up row
    hipError_t e;
    if (mode == 0)
        e = bf16 ? f4_group_launch<true, 0, false>(p, A, B, S, C, 2 * G, N, K, grp, 0, st)
                 : f4_group_launch<false, 0, false>(p, A, B, S, C, 2 * G, N, K, grp, 0, st);
    else if (mode == 1)
        e = bf16 ? f4_group_launch<true, 3, false>(p, A, B, S, C, G, N, K, grp, up_off, st)
                 : f4_group_launch<false, 3, false>(p, A, B, S, C, G, N, K, grp, up_off, st);
    else
        e = bf16 ? f4_group_launch<true, 3, true>(p, A, B, S, C, G / topk, N, K, grp, up_off, st)
                 : f4_group_launch<false, 3, true>(p, A, B, S, C, G / topk, N, K, grp, up_off, st);
    return launch_status(e);
}

ternocl_status int2_f4_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st) {
    const size_t words = (size_t)(K / 16) * N;
    const unsigned blocks = (unsigned)((words + 255) / 256);
    hipLaunchKernelGGL(k_int2_f4_decode, dim3(blocks), dim3(256), 0, st, B, D, words);
    return check_launch();
}

}  // namespace tcl
