// bitcos.hip -- BITCOS (presence bitmap + compacted signs) ternary GEMV on
// gfx950, replacing bitcos_fp16_upcvt_gemv (bitcos_fp16_upcvt/bitcos_fp16_upcvt.cl:177-277),
// plus the slice-rank precompute (common/bitcos.hpp:81-94) and a bit-exact
// decode hook.
//
//   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(k,n))),  code in {-1, 0, +1}
//
// B is one uint32 buffer: bitmap [K/32][N] (bit c of word (kp, n) = row
// 32kp+c of column n is non-zero) | offsets [N] (first sign word of column n) |
// per-column sign streams (one bit per non-zero in k order, 1 = -1) | pad.
// SR [ls-1][N]: non-zeros of column n above each slice start s*K/ls.
//
// Work split: lane = output column (64 columns per wave, every bitmap load is
// 256 contiguous bytes), wave s of a workgroup = K slice s (it enters the
// column's sign stream at SR[s-1]); the slices reduce through LDS in slice
// order (deterministic).  With a workspace the ls slices of a strip may be
// spread over ksw workgroups (grid.y), so that the launch fills the CUs evenly
// (N = 21504: 336 strips of 14 waves leave 80 CUs with twice the work); each
// writes its sums to the workspace and the last of a strip's workgroups (a
// device-scope counter) adds them in order and applies the epilogue.  Per
// 64-row chunk a lane loads the column's two bitmap words and three sign words
// (the chunk consumes at most 64 sign bits from the column's rank onwards), in
// blocks of up to 8 chunks: a block's bitmap words one block ahead, then its
// ranks, then all of its sign words at once (their addresses need the ranks).
// Decode per 32-row word: the word's sign window is funnel-shifted out of the
// three sign words (v_alignbit); each 4-row nibble m and the next four window
// bits s index a 256-entry LDS table of four DT codes +1 / -1 / 0 (a 4-bit
// pdep), and the window advances by popcount(m) (v_bfe at a running offset,
// v_bcnt with accumulate).  MACs: v_dot2_f32_{f16,bf16} of the code pairs with
// activation pairs that are uniform across the wave (scalar loads), one fp32
// partial per 128-row group, then acc += partial * S as the reference's host
// gold (bitcos_fp16_upcvt/main.cpp:64-86).
#include "common.hpp"

#include <algorithm>


namespace tcl {
namespace {

constexpr int kBcMaxLs = 16;  // slices (waves) per workgroup

template <bool BF16> __host__ __device__ constexpr uint32_t bc_pos() { return BF16 ? 0x3F80u : 0x3C00u; }
template <bool BF16> __host__ __device__ constexpr uint32_t bc_neg() { return BF16 ? 0xBF80u : 0xBC00u; }

// Table entry (m, s): row i of the nibble is 0 if bit i of m is clear, else
// -1 if sign bit popcount(m & ((1 << i) - 1)) of s is set, else +1
// (bitcos_fp16_upcvt.cl:108-124).  .x = rows 0, 1; .y = rows 2, 3.
template <bool BF16>
__device__ __forceinline__ uint2 bc_lut_entry(int idx) {
    const uint32_t m = (uint32_t)idx >> 4, s = (uint32_t)idx & 15u;
    uint32_t c[4], r = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t p = (m >> i) & 1u;
        c[i] = p ? (((s >> r) & 1u) ? bc_neg<BF16>() : bc_pos<BF16>()) : 0u;
        r += p;
    }
    return make_uint2(c[0] | (c[1] << 16), c[2] | (c[3] << 16));
}

template <bool BF16>
__device__ __forceinline__ void bc_build_lut(uint2 *lut) {
    for (int i = threadIdx.x; i < 256; i += blockDim.x) lut[i] = bc_lut_entry<BF16>(i);
    __syncthreads();
}

// 32-bit sign window at stream bit r from three consecutive words q[0..2]
// starting at word base (r / 32 - base is 0 or 1).
__device__ __forceinline__ uint32_t bc_window(const uint32_t q[3], uint32_t base, uint32_t r) {
    const bool up = (r >> 5) != base;
    const uint32_t lo = up ? q[1] : q[0], hi = up ? q[2] : q[1];
    return __builtin_amdgcn_alignbit(hi, lo, r & 31u);
}

// The 8 nibble lookups of one bitmap word with window sw.
__device__ __forceinline__ void bc_decode_word(const uint2 *lut, uint32_t bm, uint32_t sw, uint2 e[8]) {
    uint32_t p = 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t m4 = (bm >> (4 * i)) & 15u;
        const uint32_t s4 = (sw >> p) & 15u;
        p = __builtin_popcount(m4) + p;
        e[i] = lut[(m4 << 4) | s4];
    }
}

// The sign flip and Hadamard transform fused in front of the GEMV (the decode
// step's hadamard_fwht + bitcos_fp16_upcvt_gemv, hadamard_fwht.cl:62-115):
// each workgroup transforms the HB-blocks (HB <= 512: one wave per block) that
// cover its K range, for its rows, into LDS as DT values -- y = DT(SCALE *
// H(s .* x)) with k_fwht_r's operations in its order (hadamard.hip), so the
// GEMV reads the bits a separate transform would have written.
struct BcFwht {
    const int8_t *signs;  // int8 [K] (+1 / -1), read when use_signs
    int HB, use_signs;
    float scale_full, scale_tail;
};

// One block of n elements (a power of two, 8 <= n <= 512) of row x in one
// wave: lane l holds elements 8 l .. 8 l + 7 (lanes past n / 8 idle), strides 1,
// 2, 4 in registers and 8 .. n / 2 across lanes, as k_fwht_r; the DT results
// go to d[8 l .. 8 l + 7].
template <bool BF16>
__device__ __forceinline__ void bc_fwht_block(const uint16_t *__restrict__ x, const int8_t *__restrict__ sg,
                                              int n, int use_signs, float sc, uint16_t *d, int lane) {
    const int e0 = 8 * lane;
    const bool live = e0 < n;
    const int ec = live ? e0 : 0;
    float v[8];
    const uint4 raw = *(const uint4 *)(x + ec);
    const uint2 sv = use_signs ? *(const uint2 *)(sg + ec) : make_uint2(0u, 0u);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        float f = dt2f<BF16>((w[i >> 1] >> (16 * (i & 1))) & 0xffffu);
        if (use_signs) f *= (float)(int8_t)(((i < 4 ? sv.x : sv.y) >> (8 * (i & 3))) & 0xffu);
        v[i] = f;
    }
#pragma unroll
    for (int h = 1; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if ((j & h) == 0) {
                const float a = v[j], c = v[j + h];
                v[j] = a + c;
                v[j + h] = a - c;
            }
    for (int h = 8; h < n; h <<= 1) {  // partner lane ^ h / 8 holds elements i ^ h
        const int m = h >> 3;
        const bool up = (lane & m) != 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float p = __shfl_xor(v[j], m);
            v[j] = up ? p - v[j] : v[j] + p;  // (a + c, a - c) with a the lower element
        }
    }
    if (!live) return;
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        o[i] = (uint32_t)f2dt<BF16>(v[2 * i] * sc) | ((uint32_t)f2dt<BF16>(v[2 * i + 1] * sc) << 16);
    *(uint4 *)(d + e0) = make_uint4(o[0], o[1], o[2], o[3]);
}

// ksw > 1: workgroup (strip, blockIdx.y) runs slices blockIdx.y * wps ..
// + wps - 1 (wps = waves per workgroup); wsum fp32 [ksw][MR][N] sums, cnt one
// zero-initialised counter per strip (left at zero again).
// FW: A holds the untransformed activations x; the workgroup transforms its
// K range of rows m0 .. m0 + MR - 1 first (fw), into the dynamic LDS xs.
template <int MR, bool BF16, int BC, bool FW = false>
__global__ void __launch_bounds__(64 * kBcMaxLs)
k_bitcos_gemv(const uint16_t *__restrict__ A, const uint32_t *__restrict__ Bc,
              const uint16_t *__restrict__ S, const uint32_t *__restrict__ SR, void *__restrict__ C,
              const uint16_t *__restrict__ Other, const void *__restrict__ Bias, int M, int m0, int N,
              int K, int ls, int postop, int out_f32, int ksw = 1, float *wsum = nullptr, uint32_t *cnt = nullptr,
              BcFwht fw = BcFwht{}) {
    __shared__ uint2 lut[256];
    __shared__ float red[kBcMaxLs - 1][MR][64];
    extern __shared__ __attribute__((aligned(16))) uint32_t xs[];  // FW: [MR][xlen] DT pairs of the blocks

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 64 + lane;
    const int nc = n < N ? n : N - 1;
    const size_t bw = (size_t)(K >> 5) * N;
    const uint32_t *__restrict__ sg = Bc + bw + N + Bc[bw + nc];
    const int wps = blockDim.x >> 6, ks = ksw > 1 ? (int)blockIdx.y : 0;
    const int sl = __builtin_amdgcn_readfirstlane(ks * wps + wave);  // this wave's K slice
    const int slice = K / ls;
    const int k0 = sl * slice;
    const int chunks = slice >> 6;  // 64-row chunks (K % (64 * ls) == 0)
    uint32_t R = sl ? SR[(size_t)(sl - 1) * N + nc] : 0u;

    // activation rows m0 .. m0 + MR - 1 as packed pairs (rows past M repeat M - 1)
    const uint32_t *__restrict__ ar[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) ar[r] = (const uint32_t *)(A + (size_t)min(m0 + r, M - 1) * K);
    // Blocks of BC 64-row chunks.  A block's bitmap words are loaded one block
    // ahead (the first block's with the slice rank and the stream offset);
    // the block's ranks then follow from them at once, and all of its sign
    // and scale loads go out together before its decode, so a slice of at
    // most BC chunks waits on two memory round trips (bitmaps, then signs)
    // rather than one per few chunks.  All loads are unconditional (a load
    // under a branch is waited for at once, and with it -- vmcnt counts in
    // order -- every load issued before it).  Bitmap words of chunks past
    // the slice read as 0, so the rank stops there and their sign loads
    // repeat the last window (inside the stream and its pad words).
    auto bm_load = [&](int c, uint32_t b[2]) {
        const int cc = c < chunks ? c : chunks - 1;
        const size_t kp = (size_t)((k0 >> 5) + 2 * cc);
        const uint32_t x = Bc[kp * N + nc], y = Bc[(kp + 1) * N + nc];
        b[0] = c < chunks ? x : 0u;
        b[1] = c < chunks ? y : 0u;
    };
    const int groups = K / kGS;
    auto s_load = [&](int c) {
        const int g = min((k0 + 64 * c) >> 7, groups - 1);
        return (uint32_t)S[(size_t)g * N + nc];
    };

    float acc[MR], part[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) acc[r] = part[r] = 0.0f;

    uint32_t bm[BC][2];  // (issued before the transform below: they do not depend on it)
#pragma unroll
    for (int i = 0; i < BC; ++i) bm_load(i, bm[i]);
    // FW: the blocks b_lo .. b_hi cover this workgroup's rows [kw0, kw0 + wps slice)
    // of K; row r's transformed block b sits at xs + r xlen + (b - b_lo) HB / 2
    int xofs = 0, xlen = 0;
    if constexpr (FW) {
        const int kw0 = ks * wps * slice, b_lo = kw0 / fw.HB, b_hi = (kw0 + wps * slice - 1) / fw.HB;
        xlen = (b_hi - b_lo + 1) * fw.HB / 2;
        xofs = b_lo * fw.HB / 2;
        for (int b = b_lo + wave; b <= b_hi; b += wps) {  // (uniform per wave)
            const int kb = b * fw.HB, nb = min(fw.HB, K - kb);
            const float sc = nb == fw.HB ? fw.scale_full : fw.scale_tail;
#pragma unroll
            for (int r = 0; r < MR; ++r)
                bc_fwht_block<BF16>(A + (size_t)min(m0 + r, M - 1) * K + kb, fw.signs + kb, nb, fw.use_signs, sc,
                                    (uint16_t *)(xs + r * xlen) + (kb - b_lo * fw.HB), lane);
        }
    }
    bc_build_lut<BF16>(lut);  // (its barrier also publishes the transformed blocks)
    // activation pair idx of row r (FW: from the LDS blocks, a broadcast read)
    auto act = [&](int r, int idx) __attribute__((always_inline)) -> uint32_t {
        if constexpr (FW) return xs[r * xlen + idx - xofs];
        else return ar[r][idx];
    };

    for (int b0 = 0; b0 < chunks; b0 += BC) {
        uint32_t rs[BC], q[BC][3], sc[BC], nb[BC][2];
#pragma unroll
        for (int i = 0; i < BC; ++i) rs[i] = i ? rs[i - 1] + __builtin_popcount(bm[i - 1][0]) + __builtin_popcount(bm[i - 1][1]) : R;
        R = rs[BC - 1] + __builtin_popcount(bm[BC - 1][0]) + __builtin_popcount(bm[BC - 1][1]);
#pragma unroll
        for (int i = 0; i < BC; ++i) {
            const uint32_t w = rs[i] >> 5;
            q[i][0] = sg[w];
            q[i][1] = sg[w + 1];
            q[i][2] = sg[w + 2];
        }
#pragma unroll
        for (int i = 0; i < BC; ++i) sc[i] = s_load(b0 + i);
#pragma unroll
        for (int i = 0; i < BC; ++i) bm_load(b0 + BC + i, nb[i]);
        // Pin the block's sign and scale words here: without a use at this
        // point the compiler sinks each chunk's loads past the early exit
        // below into that chunk's decode, one memory round trip per chunk.
        // (The wait this implies covers these loads only: the bitmap loads
        // just issued stay in flight.)
#pragma unroll
        for (int i = 0; i < BC; ++i) asm volatile("" : "+v"(q[i][0]), "+v"(q[i][1]), "+v"(q[i][2]), "+v"(sc[i]));
#pragma unroll
        for (int u = 0; u < BC; ++u) {
            const int c = b0 + u;
            if (c >= chunks) break;  // uniform
            const uint32_t b0w = bm[u][0], b1w = bm[u][1];
            const uint32_t r0 = rs[u], r1 = __builtin_popcount(b0w) + r0;
            const int k = k0 + 64 * c;
            const uint32_t base = r0 >> 5;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                uint2 e[8];
                bc_decode_word(lut, h ? b1w : b0w, bc_window(q[u], base, h ? r1 : r0), e);
                const int kd = (k + 32 * h) >> 1;  // first activation pair of the word
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    float pr = part[r];
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        pr = dot2<BF16>(e[i].x, act(r, kd + 2 * i), pr);
                        pr = dot2<BF16>(e[i].y, act(r, kd + 2 * i + 1), pr);
                    }
                    part[r] = pr;
                }
            }
            // group end (or slice end mid-group): apply the group's scale
            if (((k + 64) & (kGS - 1)) == 0 || c + 1 == chunks) {
                const float s = dt2f<BF16>(sc[u]);
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    acc[r] += part[r] * s;
                    part[r] = 0.0f;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < BC; ++i) {
            bm[i][0] = nb[i][0];
            bm[i][1] = nb[i][1];
        }
    }

    // reduce the workgroup's slices in slice order
    if (wps > 1) {
        if (wave > 0)
#pragma unroll
            for (int r = 0; r < MR; ++r) red[wave - 1][r][lane] = acc[r];
        __syncthreads();
        if (wave > 0) return;
        for (int j = 0; j < wps - 1; ++j)
#pragma unroll
            for (int r = 0; r < MR; ++r) acc[r] += red[j][r][lane];
    }
    if (ksw > 1) {
        // this workgroup's sums, then the strip's counter; the last of the ksw
        // workgroups adds them in order: agent-scope stores completed
        // (s_waitcnt) before the counter's atomic, agent-scope loads after its
        // result is tested, no fences -- the int2 GEMV's K-split handoff and
        // its reasoning (int2_gemv_f4.hip)
        if (n < N)
#pragma unroll
            for (int r = 0; r < MR; ++r)
                __hip_atomic_store(wsum + ((size_t)ks * MR + r) * N + n, acc[r], __ATOMIC_RELAXED,
                                   __HIP_MEMORY_SCOPE_AGENT);
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
        __builtin_amdgcn_s_waitcnt(0);
        const uint32_t prev = split_arrive(cnt + blockIdx.x, ksw, lane);
        if (prev != (uint32_t)(ksw - 1)) return;
        // 16 / MR workgroups' sums in flight at a time (past ksw clamped, loaded
        // and not added), added in order
        constexpr int U = 16 / MR;
        for (int u0 = 0; u0 < ksw; u0 += U) {
            float v[U][MR];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                const int s2 = u0 + u < ksw ? u0 + u : ksw - 1;
#pragma unroll
                for (int r = 0; r < MR; ++r)
                    v[u][r] = __hip_atomic_load(wsum + ((size_t)s2 * MR + r) * N + nc, __ATOMIC_RELAXED,
                                                __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (u0 + u >= ksw) break;
#pragma unroll
                for (int r = 0; r < MR; ++r) acc[r] = u0 + u == 0 ? v[u][r] : acc[r] + v[u][r];
            }
        }
    }
    if (n >= N) return;
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
#pragma unroll
        for (int r = 0; r < MR; ++r)
            if (m0 + r < M)
                epi_store1_c<BF16, decltype(P_)::value, decltype(F_)::value>(C, Other, Bias, N, m0 + r, n, acc[r]);
    });
}

// SR[(s-1)*N + n] = non-zeros of column n in bitmap words kp < s * ceil(K/ls) / 32
__global__ void k_bitcos_slice_ranks(const uint32_t *__restrict__ Bc, uint32_t *__restrict__ SR, int N,
                                     int K, int ls) {
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const int slice_k = (K + ls - 1) / ls;
    uint32_t s = 0;
    int kp = 0;
    for (int sl = 1; sl < ls; ++sl) {
        for (; kp < sl * slice_k / 32; ++kp) s += __builtin_popcount(Bc[(size_t)kp * N + n]);
        SR[(size_t)(sl - 1) * N + n] = s;
    }
}

// Test hook: W[k][n] = 0 / S / S ^ 0x8000 for code 0 / +1 / -1, through the
// GEMV's decode (sign windows, nibble table) -- one thread per column.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_bitcos_dequant(const uint32_t *__restrict__ Bc, const uint16_t *__restrict__ S, uint16_t *__restrict__ W,
                 int N, int K) {
    __shared__ uint2 lut[256];
    bc_build_lut<BF16>(lut);
    const int n = blockIdx.x * blockDim.x + threadIdx.x;
    if (n >= N) return;
    const size_t bw = (size_t)(K >> 5) * N;
    const uint32_t *sg = Bc + bw + N + Bc[bw + n];
    uint32_t R = 0;
    for (int kp = 0; kp < K / 32; ++kp) {
        const uint32_t bm = Bc[(size_t)kp * N + n];
        const uint32_t q[3] = {sg[R >> 5], sg[(R >> 5) + 1], sg[(R >> 5) + 2]};
        uint2 e[8];
        bc_decode_word(lut, bm, bc_window(q, R >> 5, R), e);
        R += __builtin_popcount(bm);
        const uint32_t s = S[(size_t)(kp >> 2) * N + n];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const uint32_t cw[4] = {e[i].x & 0xffffu, e[i].x >> 16, e[i].y & 0xffffu, e[i].y >> 16};
#pragma unroll
            for (int j = 0; j < 4; ++j)
                W[(size_t)(32 * kp + 4 * i + j) * N + n] = (uint16_t)(cw[j] ? (s ^ (cw[j] & 0x8000u)) : 0u);
        }
    }
}

// Re-pack for the M-tiled path: the BITCOS weights as int2 words (row j of
// word (kp, n) in bits 2j, 2j + 1; codes 0 / 1 / 3 = 0 / +1 / -1), so the int2
// prefill GEMM engine runs on them.  Lane = column, wave = K slice (entering
// the column's sign stream at SR[s-1], as the GEMV); per block of up to 8
// bitmap words, all bitmap loads go out together, then -- the ranks known --
// all sign-word loads, then the decode: two dependent memory round trips per
// block.  The 256-byte table maps (nibble of presence bits, next four sign
// bits) to the nibble's four 2-bit codes.
__global__ void __launch_bounds__(64 * kBcMaxLs)
k_bitcos_to_int2(const uint32_t *__restrict__ Bc, const uint32_t *__restrict__ SR, uint32_t *__restrict__ W2,
                 int N, int K, int ls) {
    __shared__ uint8_t lut[256];
    for (int i = threadIdx.x; i < 256; i += blockDim.x) {
        const uint32_t m = (uint32_t)i >> 4, sgn = (uint32_t)i & 15u;
        uint32_t r = 0, out = 0;
        for (int j = 0; j < 4; ++j)
            if ((m >> j) & 1u) {
                out |= (1u | (((sgn >> r) & 1u) << 1)) << (2 * j);
                ++r;
            }
        lut[i] = (uint8_t)out;
    }
    __syncthreads();
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const int n = blockIdx.x * 64 + lane;
    const int nc = n < N ? n : N - 1;
    const size_t bw = (size_t)(K >> 5) * N;
    const uint32_t *__restrict__ sg = Bc + bw + N + Bc[bw + nc];
    const int words = K >> 5, per = words / ls, w0 = wave * per;
    uint32_t R = wave ? SR[(size_t)(wave - 1) * N + nc] : 0u;
    for (int b = 0; b < per; b += 8) {
        uint32_t bm[8], r[8], lo[8], hi[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int kp = w0 + b + j < words ? w0 + b + j : words - 1;
            const uint32_t x = Bc[(size_t)kp * N + nc];
            bm[j] = b + j < per ? x : 0u;  // words past the slice: no rows, no signs
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            r[j] = R;
            R += __builtin_popcount(bm[j]);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // inside the stream or its pad words
            lo[j] = sg[r[j] >> 5];
            hi[j] = sg[(r[j] >> 5) + 1];
        }
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            if (b + j >= per) break;  // uniform
            const uint32_t sw = __builtin_amdgcn_alignbit(hi[j], lo[j], r[j] & 31u);
            uint32_t out[2] = {0u, 0u}, p = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t m4 = (bm[j] >> (4 * i)) & 15u;
                const uint32_t s4 = (sw >> p) & 15u;
                p = __builtin_popcount(m4) + p;
                out[i >> 2] |= (uint32_t)lut[(m4 << 4) | s4] << (8 * (i & 3));
            }
            if (n < N) {
                const size_t kp2 = 2 * (size_t)(w0 + b + j);
                W2[kp2 * N + n] = out[0];
                W2[(kp2 + 1) * N + n] = out[1];
            }
        }
    }
}

// Chunks per block: the slice's own count up to 8 (from 2, 4, 6, 8), else 6
// where that divides it, else 8.
int bc_block(int chunks) {
    if (chunks <= 8) return chunks <= 2 ? 2 : chunks <= 4 ? 4 : chunks <= 6 ? 6 : 8;
    return chunks % 6 == 0 ? 6 : 8;
}

// LDS of the fused transform: MR rows of the blocks a workgroup's K range
// (ls / ksw slices) can touch.
size_t bc_fw_lds(int MR, int K, int ls, int ksw, int HB) {
    const int range = K / ls * (ls / ksw);
    return (size_t)MR * ((range + HB - 1) / HB + 1) * HB * 2;
}

template <int MR, bool BF16, int BC>
void bc_launch_b(const void *A, const uint32_t *Bc, const void *S, const uint32_t *SR, void *C,
                 const void *Other, const void *Bias, int M, int m0, int N, int K, int ls, int postop,
                 int out_f32, int ksw, float *part, uint32_t *cnt, hipStream_t st, const BcFwht *fw) {
    if (fw)
        hipLaunchKernelGGL((k_bitcos_gemv<MR, BF16, BC, true>), dim3((N + 63) / 64, ksw), dim3(64 * (ls / ksw)),
                           bc_fw_lds(MR, K, ls, ksw, fw->HB), st, (const uint16_t *)A, Bc, (const uint16_t *)S, SR,
                           C, (const uint16_t *)Other, Bias, M, m0, N, K, ls, postop, out_f32, ksw, part, cnt, *fw);
    else
        hipLaunchKernelGGL((k_bitcos_gemv<MR, BF16, BC>), dim3((N + 63) / 64, ksw), dim3(64 * (ls / ksw)), 0, st,
                           (const uint16_t *)A, Bc, (const uint16_t *)S, SR, C, (const uint16_t *)Other, Bias,
                           M, m0, N, K, ls, postop, out_f32, ksw, part, cnt);
}

template <int MR, bool BF16>
void bc_launch(const void *A, const uint32_t *Bc, const void *S, const uint32_t *SR, void *C,
               const void *Other, const void *Bias, int M, int m0, int N, int K, int ls, int postop,
               int out_f32, int ksw, float *part, uint32_t *cnt, hipStream_t st, const BcFwht *fw) {
#define TCL_BC_B(BC) \
    bc_launch_b<MR, BF16, BC>(A, Bc, S, SR, C, Other, Bias, M, m0, N, K, ls, postop, out_f32, ksw, part, cnt, st, fw)
    switch (bc_block(K / ls / 64)) {
    case 2: TCL_BC_B(2); break;
    case 4: TCL_BC_B(4); break;
    case 6: TCL_BC_B(6); break;
    default:
        if constexpr (MR == 4) TCL_BC_B(4);  // (8 chunks of 4 rows need more than 128 VGPRs)
        else TCL_BC_B(8);
        break;
    }
#undef TCL_BC_B
}

// Launches of up to maxr (1, 2 or 4) rows each.
template <bool BF16>
void bc_launch_rows(const void *A, const uint32_t *Bc, const void *S, const uint32_t *SR, void *C,
                    const void *Other, const void *Bias, int M, int N, int K, int ls, int postop,
                    int out_f32, int ksw, float *part, uint32_t *cnt, hipStream_t st, const BcFwht *fw = nullptr,
                    int maxr = 4) {
    for (int m0 = 0; m0 < M; m0 += maxr) {
        const int rows = std::min(M - m0, maxr);
        if (rows == 1) bc_launch<1, BF16>(A, Bc, S, SR, C, Other, Bias, M, m0, N, K, ls, postop, out_f32, ksw, part, cnt, st, fw);
        else if (rows == 2) bc_launch<2, BF16>(A, Bc, S, SR, C, Other, Bias, M, m0, N, K, ls, postop, out_f32, ksw, part, cnt, st, fw);
        else bc_launch<4, BF16>(A, Bc, S, SR, C, Other, Bias, M, m0, N, K, ls, postop, out_f32, ksw, part, cnt, st, fw);
    }
}

// Relative cost of a launch with k workgroups per 64-column strip (each over
// K / k rows), dealt evenly over the 256 CUs: the busiest CU's workgroups,
// each costing its share of K plus a fixed part (the table build, the
// slice-sum exchange) worth 2.55% of a whole K.  Fitted to graph-timed runs
// at K = 5376, z = .5, N = 21504 (336 strips): ls = 12 with k = 1, 2, 3, 4, 6
// 20.6 / 19.3 / 16.9 / 19.1 / 18.2 us, ls = 14 with k = 1, 2, 7 20.9 / 17.7 /
// 19.4 us.
double bc_cost(int N, int k) {
    const long strips = (N + 63) / 64;
    return (double)((strips * k + 255) / 256) * (1.0 / k + 0.0255);
}

// Workgroups per strip for ls slices: the divisor of ls of least cost.
int bc_pick_ksw(int N, int ls) {
    int best = 1;
    for (int k = 2; k <= ls; ++k)
        if (ls % k == 0 && bc_cost(N, k) < bc_cost(N, best)) best = k;
    return best;
}

// Workspace of a split launch: a counter per 64-column strip (256-byte
// block), then the sums fp32 [ksw][4][N].
// counters (one per 64-column strip) in the workspace header, sums after it
bool bc_cnt_fit(int N) { return (size_t)((N + 63) / 64) * 4 <= kWsHeader; }
size_t bc_split_ws(int N, int ksw) { return ksw > 1 ? kWsHeader + (size_t)ksw * 4 * N * 4 : 0; }

}  // namespace

int bitcos_max_ls() { return kBcMaxLs; }

// The slice count whose best split (bc_pick_ksw) costs least, among ls <= 16
// with K % (64 * ls) == 0 and >= 6 sixty-four-row chunks per slice.  On a tie:
// a slice of at most 8 chunks (one block of loads: two round trips), the most
// chunks among those, else the larger ls.  K = 5376: N = 21504 takes 12 (3
// workgroups of 4 waves per strip: 14.5 us, against 17.5 at 14 split in 2);
// N = 16384 takes 12 (one workgroup per strip, 7 chunks per slice: 11.9 us,
// against 12.4 at 14 and 13.1 at 7).
int bitcos_pick_ls(int N, int K) {
    int best = 0;
    double best_cost = 0.0;
    auto tie_prefers = [K](int a, int b) {  // ls a over ls b at equal cost
        const int ca = K / (64 * a), cb = K / (64 * b);
        if ((ca <= 8) != (cb <= 8)) return ca <= 8;
        return ca <= 8 ? ca > cb : a > b;
    };
    for (int ls = 1; ls <= kBcMaxLs; ++ls) {
        if (K % (64 * ls) || K / (64 * ls) < 6) continue;
        const double c = bc_cost(N, bc_pick_ksw(N, ls));
        if (best == 0 || c < best_cost || (c == best_cost && tie_prefers(ls, best))) {
            best = ls;
            best_cost = c;
        }
    }
    return best ? best : 1;
}

// Workspace bytes for the split launch of this shape (0: none helps).
size_t bitcos_gemv_ws_need(int N, int ls) { return bc_split_ws(N, bc_pick_ksw(N, ls)); }

// ws (16-byte aligned, counters zeroed before the first call, as
// bitcos_gemv_ws_need): the split launch; without it one workgroup per strip.
ternocl_status bitcos_gemv_run(int dtype, const void *A, const uint32_t *Bc, const void *S,
                               const uint32_t *SR, int ls, void *C, const void *Other, const void *Bias,
                               int M, int N, int K, int postop, int out_f32, hipStream_t st, void *ws,
                               size_t ws_bytes) {
    int ksw = bc_pick_ksw(N, ls);
    if (ksw > 1 && !(ws && ((uintptr_t)ws & 15) == 0 && ws_bytes >= bc_split_ws(N, ksw) && bc_cnt_fit(N))) ksw = 1;
    uint32_t *cnt = ksw > 1 ? (uint32_t *)ws : nullptr;
    float *part = ksw > 1 ? (float *)((uint8_t *)ws + kWsHeader) : nullptr;
    if (dtype == TERNOCL_BF16)
        bc_launch_rows<true>(A, Bc, S, SR, C, Other, Bias, M, N, K, ls, postop, out_f32, ksw, part, cnt, st);
    else
        bc_launch_rows<false>(A, Bc, S, SR, C, Other, Bias, M, N, K, ls, postop, out_f32, ksw, part, cnt, st);
    return check_launch();
}

// The sign flip + FWHT (HB <= 512; blocks of K: each a power of two >= 8,
// x 16-byte and signs 8-byte aligned: the host checks) fused into the GEMV;
// the same workspace rule as bitcos_gemv_run.
ternocl_status bitcos_fwht_gemv_run(int dtype, const void *x, const int8_t *signs, int HB, int use_signs,
                                    float scale_full, float scale_tail, const uint32_t *Bc, const void *S,
                                    const uint32_t *SR, int ls, void *C, const void *Other, const void *Bias, int M,
                                    int N, int K, int postop, int out_f32, hipStream_t st, void *ws, size_t ws_bytes) {
    int ksw = bc_pick_ksw(N, ls);
    if (ksw > 1 && !(ws && ((uintptr_t)ws & 15) == 0 && ws_bytes >= bc_split_ws(N, ksw) && bc_cnt_fit(N))) ksw = 1;
    // rows per launch: the most (4, 2, 1) whose blocks fit the workgroup's LDS
    // beside the table and the slice sums
    int maxr = 4;
    auto lds_of = [&](int r) { return bc_fw_lds(r, K, ls, ksw, HB) + 256 * 8 + (size_t)(kBcMaxLs - 1) * r * 64 * 4; };
    while (maxr > 1 && lds_of(maxr) > 64 * 1024) maxr >>= 1;
    if (lds_of(maxr) > 64 * 1024) {
        set_error("the fused transform's blocks take more than 64 KiB of LDS at this K / ls");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    uint32_t *cnt = ksw > 1 ? (uint32_t *)ws : nullptr;
    float *part = ksw > 1 ? (float *)((uint8_t *)ws + kWsHeader) : nullptr;
    const BcFwht fw{signs, HB, use_signs, scale_full, scale_tail};
    if (dtype == TERNOCL_BF16)
        bc_launch_rows<true>(x, Bc, S, SR, C, Other, Bias, M, N, K, ls, postop, out_f32, ksw, part, cnt, st, &fw, maxr);
    else
        bc_launch_rows<false>(x, Bc, S, SR, C, Other, Bias, M, N, K, ls, postop, out_f32, ksw, part, cnt, st, &fw, maxr);
    return check_launch();
}

ternocl_status bitcos_to_int2_run(const uint32_t *Bc, const uint32_t *SR, int ls, uint32_t *W2, int N, int K,
                                  hipStream_t st) {
    hipLaunchKernelGGL(k_bitcos_to_int2, dim3((N + 63) / 64), dim3(64 * ls), 0, st, Bc, SR, W2, N, K, ls);
    return check_launch();
}

ternocl_status bitcos_slice_ranks_run(const uint32_t *Bc, uint32_t *SR, int N, int K, int ls,
                                      hipStream_t st) {
    hipLaunchKernelGGL(k_bitcos_slice_ranks, dim3((N + 255) / 256), dim3(256), 0, st, Bc, SR, N, K, ls);
    return check_launch();
}

ternocl_status bitcos_dequant_run(int dtype, const uint32_t *Bc, const void *S, void *W, int N, int K,
                                  hipStream_t st) {
    const dim3 grid((N + 255) / 256), block(256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_bitcos_dequant<true>, grid, block, 0, st, Bc, (const uint16_t *)S,
                           (uint16_t *)W, N, K);
    else
        hipLaunchKernelGGL(k_bitcos_dequant<false>, grid, block, 0, st, Bc, (const uint16_t *)S,
                           (uint16_t *)W, N, K);
    return check_launch();
}

}  // namespace tcl
