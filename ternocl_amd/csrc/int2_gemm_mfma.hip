// int2_gemm_mfma.hip -- prefill GEMM (M > 16) for packed 2-bit ternary weights
// on gfx950: the MI355X replacement of int2_fp16_upcvt_gemm_mt
// (int2_fp16_upcvt/int2_fp16_upcvt.cl:292-395), and the tile engine of the MoE
// prefill (int2_moe/int2_moe_prefill.cl:72-141).
//
//   C[m,n] = ct(epi(sum_k A[m,k] * w(k,n))),  w(k,n) = code(k,n) * S[k/128, n]
//
// Tiling: a workgroup computes a BM x BN tile of C, 128 x 512 (eight waves
// side by side, each 128 x 64) or 128 x 128 (2 x 2 waves of 64 x 64); a wave's
// outputs are 32 x 32 blocks of v_mfma_f32_32x32x16_{f16,bf16} whose fp32
// accumulators stay in registers over all of K.  K advances in LDS stages of
// 64 (four MFMA k-steps of 16).
//   * A (DT, row-major) goes global -> registers -> LDS once per workgroup and
//     stage, each 16-element chunk stored in the order 0,8,1,9,...,7,15, so the
//     MFMA A fragment of lane (row, q) -- pairs (4h+i, 4h+i+8) of one chunk --
//     is one 16-byte LDS read (row pitch 72 elements: conflict-free);
//   * B is never expanded in memory: each wave loads the packed words of its
//     columns (L2-resident across the M tiles) and builds the MFMA B fragment
//     in registers with the group scale folded in, as the reference's
//     dequantising decode does (int2_fp16_upcvt.cl:118-150), so the MFMA chains
//     run over all of K with no per-group rescale:
//       fp16: (w << (14 - 2j)) & 0xC000C000 is exactly +-2.0 / 0 for the rows
//             (j, j+8) of a word; one v_pk_mul_f16 by (s, s) gives +-2s exactly
//             and the accumulators are halved once at the end;
//       bf16: v_perm_b32 through per-column byte tables {0, s, 0, -s} (low and
//             high bytes) indexed by the codes: selector = ((w >> 2j) &
//             0x30003) * 0x101 + 0x04000400, one v_mad_u32_u24;
//   * workgroup -> tile mapping keeps the M tiles of one column strip on one
//     XCD, so a strip's packed weights are fetched into that XCD's L2 once.
#include "common.hpp"

namespace tcl {
// Whether a prefill GEMM below the 128 x 512 tile's 192-tile mark runs 128 x
// 256 tiles: where 128 x 128 tiles would number more than 256 (some CUs would
// hold two) and 128 x 256 tiles fit one per CU.  Used by gemm_plan (the
// measurements are at its comment) and by the s8 x s2 GEMM's planner.
bool gemm_half_tile(int M, int N) {
    auto tiles = [&](int BM, int BN) { return (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN); };
    return tiles(128, 512) < 192 && tiles(128, 128) > 256 && tiles(128, 256) <= 256;
}
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef int i32x4_t __attribute__((ext_vector_type(4)));

constexpr int BK = 64;           // K per LDS stage
constexpr int A_PITCH = BK + 8;  // DT elements per LDS row (16 bytes of padding)
constexpr int kMoeTileRows = 128;  // MoE row tiles (experts hold a few hundred rows each)

typedef float f32x16_t __attribute__((ext_vector_type(16)));

// v_mfma_f32_32x32x16_{f16,bf16}: on gfx950 twice the throughput of the
// 16x16x32 shape (measured: 2.05 vs 1.15 PFLOP/s in a pure MFMA loop).  Lane
// (c, q) = (l % 32, l / 32) holds 8 k values of A row c / B column c, slot s of
// A pairing with slot s of B; result element i is row 8(i/4) + 4q + i%4,
// column c.
template <bool BF16>
__device__ __forceinline__ f32x16_t mfma32(const uint32_t a[4], const uint32_t b[4], f32x16_t c) {
    if constexpr (BF16) {
        bf168_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(x, y, c, 0, 0, 0);
    } else {
        half8_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(x, y, c, 0, 0, 0);
    }
}

// Per-column scale operand of the decode: fp16 (s, s) packed; bf16 the byte
// tables lo = {0, s.lo, 0, s.lo}, hi = {0, s.hi, 0, s.hi ^ 0x80}.
template <bool BF16> struct ScaleOp;
template <> struct ScaleOp<false> {
    uint32_t s2;
    __device__ __forceinline__ void set(uint32_t s) { s2 = s | (s << 16); }
};
template <> struct ScaleOp<true> {
    uint32_t lo, hi;
    // the decode's mask and bits: registers (gemm_tile pins them), so that
    // the mask-and-set is one v_and_or_b32 (a VOP3 takes no literal here)
    uint32_t km = 0x03030303u, ko = 0x04000400u;
    __device__ __forceinline__ void set(uint32_t s) {
        const uint32_t l = s & 0xffu, h = (s >> 8) & 0xffu;
        lo = (l << 8) | (l << 24);
        hi = (h << 8) | ((h ^ 0x80u) << 24);
    }
};

// B fragment of half h of word w with the scale folded in: dword i = rows
// (4h+i, 4h+i+8) of the word as (w(j), w(j+8)); fp16 values are 2x the weight.
__device__ __forceinline__ void frag(uint32_t w, int h, const ScaleOp<false> &sc, uint32_t b[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int j = 4 * h + i;
        const uint32_t t = (w << (14 - 2 * j)) & 0xC000C000u;  // +-2.0 / +-0 per half
        half2_t x, y;
        __builtin_memcpy(&x, &t, 4);
        __builtin_memcpy(&y, &sc.s2, 4);
        const half2_t r = x * y;  // v_pk_mul_f16: exact
        __builtin_memcpy(&b[i], &r, 4);
    }
}
// bf16: the byte selector of dword i is (c, c + 4, c', c' + 4) for the codes c,
// c' of rows j, j + 8: bytes h and h + 2 of the word (rows 4h .. 4h + 3 and
// 4h + 8 .. 4h + 11) are spread to (b, b, b', b') once, then each dword takes
// its 2-bit field of every byte and sets bit 2 of bytes 1 and 3 (three
// operations per dword).
__device__ __forceinline__ void frag(uint32_t w, int h, const ScaleOp<true> &sc, uint32_t b[4]) {
    const uint32_t t = __builtin_amdgcn_perm(w, w, h ? 0x03030101u : 0x02020000u);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t sel = ((t >> (2 * i)) & sc.km) | sc.ko;  // v_and_or_b32
        b[i] = __builtin_amdgcn_perm(sc.hi, sc.lo, sel);
    }
}

// Interleave a 16-element chunk (v[0..3] = elements 0..7, v[4..7] = 8..15) into
// 0,8,1,9,...,7,15.
__device__ __forceinline__ void chunk_interleave(const uint32_t v[8], uint32_t o[8]) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = v[i >> 1], hi = v[4 + (i >> 1)];
        o[i] = __builtin_amdgcn_perm(hi, lo, (i & 1) ? 0x07060302u : 0x05040100u);
    }
}

// Row source of the A tile: a plain row-major [M, K] matrix, or rows gathered
// through an index (the MoE path reads token rows of X through perm).
// Rows from `split` on form a second segment (a tile holding two experts'
// rows): row r >= split is A + (idx2[r - split] / div) * K, or without an
// index A + (base2 + r - split) * K.
struct ARows {
    const uint16_t *A;
    const int *idx;  // nullptr: row r is A + r * K; else A + (idx[r] / div) * K
    int div;
    const int *idx2 = nullptr;
    int base2 = 0, split = 1 << 30;
    // byte offset of row r from A (the A operand stays below 2^31 bytes)
    __device__ __forceinline__ uint32_t rowoff(int r, int K) const {
        if (r >= split) return (uint32_t)(idx2 ? idx2[r - split] / div : base2 + r - split) * (uint32_t)K * 2u;
        return (uint32_t)(idx ? idx[r] / div : r) * (uint32_t)K * 2u;
    }
};

// A row tile of the MoE layer holding two experts' short tails: rows
// [0, kPairSplit) are expert a's (nA of them, C rows from crow0), rows
// [kPairSplit, 2 kPairSplit) expert b's (nB, C rows from crowB), and the waves
// of the second half read expert b's weights (Bb, Sb; DUAL: B2b, S2b).
constexpr int kPairSplit = 64;
struct PairTile {
    const uint32_t *Bb = nullptr;
    const uint16_t *Sb = nullptr;
    const uint32_t *B2b = nullptr;
    const uint16_t *S2b = nullptr;
    int nA = 0, nB = 0, crowB = 0;
};

constexpr int kEpPitch = 36;  // epilogue floats per row: 32 + 4 (16-byte aligned rows)

// Tile shape: WVM x WVN waves, each owning NMB x NCB blocks of 16 x 16 outputs
// (NMB, NCB even: the MFMAs are 32 x 32).
template <int NMB_, int NCB_, int WVM_ = 2, int WVN_ = 2> struct TileCfg {
    static constexpr int NMB = NMB_, NCB = NCB_, WVM = WVM_, WVN = WVN_;
    static constexpr int THREADS = 64 * WVM * WVN;
    static constexpr int BM = 16 * NMB * WVM, BN = 16 * NCB * WVN;
    static constexpr int ACH = BM * 4 / THREADS;  // 16-element A chunks per thread per stage
    static_assert(BM * 4 % THREADS == 0, "A chunks must divide evenly");
    // LDS (DT elements): three A stages while K runs, then the epilogue's
    // per-wave [8 NMB][kEpPitch] fp32 blocks
    static constexpr size_t stage_elems = 3 * (size_t)BM * A_PITCH;
    static constexpr size_t epi_elems = (size_t)(THREADS / 64) * 8 * NMB * kEpPitch * 2;
    static constexpr size_t lds_elems = stage_elems > epi_elems ? stage_elems : epi_elems;
};

// One BM x BN output tile of rows [0, mrows) of ar (mrows <= BM) and columns
// [n0, n0 + BN) (columns >= N masked); C row r is crow0 + r.  The tile runs
// over kseg rows of K (a multiple of 128): A's rows have stride K, and ar, B
// and S start at the segment's first row (split-K: one K-slice).
// DUAL: the MoE gate/up pair in one pass over A -- acc from (B, S) is the up
// projection, acc2 from (B2, S2) the gate; C = DT(silu(gate) * DT(up)), the
// two-launch sequence's result (up rounded to DT, then POSTOP 1) bit for bit.
// BC: B is a BITCOS buffer (bitmap [K/32][N] | offsets [N] | sign streams |
// pad), decoded in the tile into the int2 words the int2 path loads (the
// M-tiled BITCOS GEMM with no re-pack); bclut is the 256-byte table of
// k_bitcos_gemm.  Unsplit only (kseg == K).
// PAIR: a tile of two experts' tails (PairTile; Cfg of two 64-row wave rows).
template <class Cfg, bool BF16, bool DUAL = false, bool SHORT = false, bool BC = false, bool PAIR = false>
__device__ __forceinline__ void gemm_tile(const ARows &ar, uint32_t a_bytes, int mrows,
                                          const uint32_t *__restrict__ B, const uint16_t *__restrict__ S,
                                          void *__restrict__ C, const uint16_t *__restrict__ Other,
                                          const void *__restrict__ Bias, int crow0, int N, int K, int kseg,
                                          int n0, int postop, int out_f32, uint16_t *lds,
                                          const uint32_t *__restrict__ B2 = nullptr,
                                          const uint16_t *__restrict__ S2 = nullptr,
                                          const uint8_t *__restrict__ bclut = nullptr,
                                          const PairTile &pt = PairTile{}) {
    constexpr int NMB = Cfg::NMB, NCB = Cfg::NCB, TH = Cfg::THREADS;
    static_assert(!PAIR || (SHORT && Cfg::BM == 2 * kPairSplit && 16 * NMB == kPairSplit), "pair tiles: two 64-row wave rows");
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = SHORT ? __builtin_amdgcn_readfirstlane(tid >> 6) : tid >> 6;
    const int wm = (wave / Cfg::WVN) * 16 * NMB, wn = (wave % Cfg::WVN) * 16 * NCB;
    const bool hb = PAIR && wm >= kPairSplit;  // (uniform) this wave computes expert b's rows
    if constexpr (PAIR) {
        if (hb) {
            B = pt.Bb;
            S = pt.Sb;
            B2 = pt.B2b;
            S2 = pt.S2b;
        }
    }
    const int stages = kseg / BK;

    // All operand loads are buffer loads with per-lane offsets set up once and
    // issued unconditionally (a load under a branch is waited for at the
    // branch's end); the loads issued past the last stage read in-range memory
    // (A: stage clamped) or return 0 (B, S: past the buffer's end).
    //
    // A staging: chunk id = tid + THREADS u -> row id >> 2, 16-element chunk id & 3.
    // Rows past mrows re-read row mrows - 1: their outputs are never stored.
    const __amdgpu_buffer_rsrc_t rA = buf_rsrc(ar.A, a_bytes);
    uint32_t va[Cfg::ACH];
#pragma unroll
    for (int u = 0; u < Cfg::ACH; ++u) {
        const int id = tid + TH * u, r = id >> 2;
        const int rc = PAIR ? (r < kPairSplit ? min(r, pt.nA - 1) : kPairSplit + min(r - kPairSplit, pt.nB - 1))
                            : (r < mrows ? r : mrows - 1);
        va[u] = ar.rowoff(rc, K) + 32u * (id & 3);
    }
    // two register sets: stage t's A chunks live in av[t & 1] from their load,
    // issued two stages ahead, to their LDS store in the middle of stage t - 1
    uint4 av[2][Cfg::ACH][2];
    auto a_load = [&](int st, int set) __attribute__((always_inline)) {
        const int sc = (st < stages ? st : stages - 1) * BK * 2;  // bytes, uniform
#pragma unroll
        for (int u = 0; u < Cfg::ACH; ++u)
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const i32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rA, va[u] + 16 * e, sc, 0);
                av[set][u][e] = make_uint4((uint32_t)t[0], (uint32_t)t[1], (uint32_t)t[2], (uint32_t)t[3]);
            }
    };
    auto a_store = [&](uint16_t *buf, int set) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < Cfg::ACH; ++u) {
            const int id = tid + TH * u;
            const uint32_t v[8] = {av[set][u][0].x, av[set][u][0].y, av[set][u][0].z, av[set][u][0].w,
                                   av[set][u][1].x, av[set][u][1].y, av[set][u][1].z, av[set][u][1].w};
            uint32_t o[8];
            chunk_interleave(v, o);
            uint4 *d = (uint4 *)(buf + (size_t)(id >> 2) * A_PITCH + 16 * (id & 3));
            d[0] = make_uint4(o[0], o[1], o[2], o[3]);
            d[1] = make_uint4(o[4], o[5], o[6], o[7]);
        }
    };

    // B words of this wave for stage st: 32-column block cb, 16-row k-step ks ->
    // word kp = 4 st + ks of column n0 + wn + 32 cb + c32 (lanes q = 0, 1 read
    // the same word and decode its halves q).  vb advances one stage per load;
    // a 32-column block past N (when N % BN != 0) reads the next row's words --
    // in range, feeding outputs that are not stored -- or, past the last row, 0.
    static_assert(NMB % 2 == 0 && NCB % 2 == 0, "32 x 32 MFMA blocks");
    constexpr int MB2 = NMB / 2, CB2 = NCB / 2;
    const int c32 = lane & 31, q32 = lane >> 5;
    const __amdgpu_buffer_rsrc_t rB = buf_rsrc(B + n0, (uint32_t)(((size_t)(kseg / 16) * N - n0) * 4));
    const __amdgpu_buffer_rsrc_t rS = buf_rsrc(S + n0, (uint32_t)(((size_t)(kseg / kGS) * N - n0) * 2));
    // (DUAL: the gate weights, same shape, same offsets)
    const __amdgpu_buffer_rsrc_t rB2 = buf_rsrc(DUAL ? B2 + n0 : B + n0, (uint32_t)(((size_t)(kseg / 16) * N - n0) * 4));
    const __amdgpu_buffer_rsrc_t rS2 = buf_rsrc(DUAL ? S2 + n0 : S + n0, (uint32_t)(((size_t)(kseg / kGS) * N - n0) * 2));
    uint32_t vb = (uint32_t)((wn + c32) * 4);
    const uint32_t vs0 = (uint32_t)((wn + c32) * 2);
    constexpr int NB = DUAL ? 2 : 1;  // weight matrices
    uint32_t bw[NB][CB2][4], sraw[NB][CB2];
    auto b_load = [&]() {
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int cb = 0; cb < CB2; ++cb)
#pragma unroll
                for (int ks = 0; ks < 4; ++ks)
                    bw[m][cb][ks] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                        m ? rB2 : rB, vb + (uint32_t)(ks * N * 4) + 128 * cb, 0, 0);
        vb += (uint32_t)(16 * N);
    };
    auto s_load = [&](int g) {  // the scales of group g (past the last: 0)
        const uint32_t v = vs0 + (uint32_t)(g * 2 * N);
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int cb = 0; cb < CB2; ++cb)
                sraw[m][cb] = __builtin_amdgcn_raw_buffer_load_b16(m ? rS2 : rS, v + 64 * cb, 0, 0);
    };

    // BC: lane column n (32 cb + c32 of the wave's block), its sign stream and
    // rank (non-zeros above the next stage to decode), the bitmap words of two
    // stages (slot = stage & 1, loaded two stages ahead) and the sign words of
    // the next stage (loaded one stage ahead: their address needs the rank).
    // Loads past the last stage read the last stage's words and the stream's
    // pad words, and are never decoded.
    constexpr int BCC = BC ? CB2 : 1;
    const size_t bcw = (size_t)(K >> 5) * N;  // bitmap words
    const uint32_t *bc_sg[BCC];
    uint32_t bc_r[BCC], bc_bm[2][BCC][2], bc_q[BCC][3];
    int bc_n[BCC];
    auto bc_bm_load = [&](int st, int slot) __attribute__((always_inline)) {
        const size_t kp = (size_t)2 * (st < stages ? st : stages - 1);
#pragma unroll
        for (int cb = 0; cb < BCC; ++cb) {
            bc_bm[slot][cb][0] = B[kp * N + bc_n[cb]];
            bc_bm[slot][cb][1] = B[(kp + 1) * N + bc_n[cb]];
        }
    };
    auto bc_sg_load = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int cb = 0; cb < BCC; ++cb) {
            const uint32_t w = bc_r[cb] >> 5;
            bc_q[cb][0] = bc_sg[cb][w];
            bc_q[cb][1] = bc_sg[cb][w + 1];
            bc_q[cb][2] = bc_sg[cb][w + 2];
        }
    };
    // the stage's 64 rows of column cb as four int2 words (16 rows each); the
    // rank advances.  Lanes l and l + 32 hold the same column: each decodes one
    // 32-row bitmap word (h = q32) and v_permlane32_swap hands each the other's.
    auto bc_decode = [&](int slot, uint32_t out[NB][CB2][4]) __attribute__((always_inline)) {
#pragma unroll
        for (int cb = 0; cb < BCC; ++cb) {
            const uint32_t r0 = bc_r[cb], base = r0 >> 5;
            const uint32_t b0 = bc_bm[slot][cb][0], b1 = bc_bm[slot][cb][1];
            const uint32_t bm = q32 ? b1 : b0;
            const uint32_t r = q32 ? r0 + __builtin_popcount(b0) : r0;
            const bool up = (r >> 5) != base;  // the window starts in the second sign word
            const uint32_t sw = __builtin_amdgcn_alignbit(up ? bc_q[cb][2] : bc_q[cb][1],
                                                          up ? bc_q[cb][1] : bc_q[cb][0], r & 31u);
            uint32_t w[2] = {0u, 0u}, p = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t m4 = (bm >> (4 * i)) & 15u;
                const uint32_t s4 = (sw >> p) & 15u;
                p = __builtin_popcount(m4) + p;
                w[i >> 2] |= (uint32_t)bclut[(m4 << 4) | s4] << (8 * (i & 3));
            }
            // element 0: the words of lanes 0..31 (h = 0) in every lane; element 1: of lanes 32..63
            const auto x0 = __builtin_amdgcn_permlane32_swap(w[0], w[0], false, false);
            const auto x1 = __builtin_amdgcn_permlane32_swap(w[1], w[1], false, false);
            out[0][cb][0] = x0[0];
            out[0][cb][1] = x1[0];
            out[0][cb][2] = x0[1];
            out[0][cb][3] = x1[1];
            bc_r[cb] = r0 + __builtin_popcount(b0) + __builtin_popcount(b1);
        }
    };

    f32x16_t acc[MB2][CB2], acc2[DUAL ? MB2 : 1][DUAL ? CB2 : 1];
#pragma unroll
    for (int mb = 0; mb < MB2; ++mb)
#pragma unroll
        for (int cb = 0; cb < CB2; ++cb) acc[mb][cb] = f32x16_t{};
    if constexpr (DUAL) {
#pragma unroll
        for (int mb = 0; mb < MB2; ++mb)
#pragma unroll
            for (int cb = 0; cb < CB2; ++cb) acc2[mb][cb] = f32x16_t{};
    }

    ScaleOp<BF16> sop[NB][CB2];
    if constexpr (BF16) {  // the decode's constants in registers (opaque to constant folding)
        uint32_t km = 0x03030303u, ko = 0x04000400u;
        asm("" : "+v"(km));
        asm("" : "+s"(ko));
#pragma unroll
        for (int m = 0; m < NB; ++m)
#pragma unroll
            for (int cb = 0; cb < CB2; ++cb) {
                sop[m][cb].km = km;
                sop[m][cb].ko = ko;
            }
    }
    a_load(0, 0);
    if constexpr (BC) {
#pragma unroll
        for (int cb = 0; cb < BCC; ++cb) {
            const int n = n0 + wn + 32 * cb + c32;
            bc_n[cb] = n < N ? n : N - 1;
            bc_sg[cb] = B + bcw + N + B[bcw + bc_n[cb]];
            bc_r[cb] = 0;
        }
        bc_bm_load(0, 0);
        bc_bm_load(1, 1);
        bc_sg_load();
    } else {
        b_load();
    }
    s_load(0);
    a_load(1, 1);
    a_store(lds, 0);
    __syncthreads();
    // A fragments of k-step ks of the stage in LDS buffer buf: row wm + 32 mb + c32,
    // elements 8 q32 .. 8 q32 + 7 of the stage's 16-element chunk ks (stored as
    // pairs (j, j + 8))
    // (the first lmb 32-row blocks: SHORT tiles read only the blocks that hold rows)
    auto a_frags = [&](const uint16_t *buf, int ks, uint32_t af[MB2][4], auto LMB_) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < decltype(LMB_)::value; ++mb) {
            const uint4 v = *(const uint4 *)(buf + (size_t)(wm + 32 * mb + c32) * A_PITCH + 16 * ks + 8 * q32);
            af[mb][0] = v.x; af[mb][1] = v.y; af[mb][2] = v.z; af[mb][3] = v.w;
        }
    };
    uint32_t af0[MB2][4];  // k-step 0 fragments of the coming stage, read a stage early
    // SHORT (tiles that may end early, as an expert's last tile): the 32-row
    // blocks of this wave that hold tile rows.  Its MFMAs and A fragment reads
    // stop there (none: the wave still stages A and meets the barriers); the
    // loop is compiled per count, so no branch sits inside it.  (uniform)
    // A wave is dead when its rows all lie past the tile's end (WVM > 1) or
    // its columns all lie past N (the last column tile of an N that is not a
    // multiple of BN, as the MoE gate/up's I = 1408 on 256-column tiles).
    const int lmb = PAIR ? max(0, min(MB2, ((hb ? pt.nB : pt.nA) + 31) / 32))
                         : SHORT ? max(0, min(MB2, (mrows - wm + 31) / 32)) : MB2;
    constexpr bool kDeadWaves = SHORT;
    const bool dead = (Cfg::WVM > 1 && lmb == 0) || n0 + wn >= N;
    if (kDeadWaves && dead) {
    } else if (lmb == 1 && MB2 > 1) {
        a_frags(lds, 0, af0, std::integral_constant<int, 1>{});
    } else {
        a_frags(lds, 0, af0, std::integral_constant<int, MB2>{});
    }
    // Stage st reads LDS buffer st % 3.  B words and scales are loaded one
    // stage ahead, A two stages ahead (register set st & 1).  Between k-steps 1
    // and 2 a wave stores stage st + 1's A into buffer (st + 1) % 3, reads its
    // k-step 2 fragments, and then meets the stage's one barrier: after it,
    // every wave's store for stage st + 1 is visible, and the buffer the next
    // stage overwrites, (st + 2) % 3, was last read in stage st - 1, before
    // that stage's barrier.  So no wave waits at a barrier for data it needs
    // right after it, and the MFMAs queued before the barrier keep running.
    // K is a multiple of 128: the stage count is even and the loop runs in
    // pairs with the register set fixed at compile time.
    constexpr uint32_t kBuf = (uint32_t)Cfg::BM * A_PITCH;  // DT elements per buffer
    uint32_t cur = 0;  // st % 3
    auto stage = [&](int st, int par, auto LMB_) __attribute__((always_inline)) {
        constexpr int LMB = decltype(LMB_)::value;  // live 32-row blocks (MB2: all)
        const uint16_t *abuf = lds + cur * kBuf;
        const uint32_t nxt = cur == 2 ? 0 : cur + 1;
        uint32_t bwc[NB][CB2][4];
        if constexpr (BC) {
            bc_decode(par, bwc);
        } else {
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int cb = 0; cb < CB2; ++cb)
#pragma unroll
                    for (int ks = 0; ks < 4; ++ks) bwc[m][cb][ks] = bw[m][cb][ks];
        }
        if (par == 0) {  // a new 128-row scale group
#pragma unroll
            for (int m = 0; m < NB; ++m)
#pragma unroll
                for (int cb = 0; cb < CB2; ++cb) sop[m][cb].set(sraw[m][cb]);
        }
        // B and scale loads first: the next stage waits for them, not for the
        // A loads issued after them.  The scales of the group after this one
        // are loaded on the group's second stage.  (sched_barrier: the
        // scheduler would otherwise sink the loads below the MFMAs, next to
        // their consumers.)
        if constexpr (BC) {
            bc_sg_load();              // the next stage's signs (its rank is known now)
            bc_bm_load(st + 2, par);   // the bitmap two stages ahead, into the slot just decoded
        } else {
            b_load();
        }
        s_load((st >> 1) + 1);
        a_load(st + 2, par);
        __builtin_amdgcn_sched_barrier(0);
        uint32_t af[MB2][4];
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
            if (ks == 0) {
#pragma unroll
                for (int mb = 0; mb < LMB; ++mb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) af[mb][i] = af0[mb][i];
            } else if (ks == 2) {
                __builtin_amdgcn_sched_barrier(0);
                a_store(lds + nxt * kBuf, par ^ 1);  // past the last stage: never read
                a_frags(abuf, 2, af, LMB_);
                __syncthreads();
                // the next stage's k-step 0 fragments (its buffer is complete
                // now): its first MFMAs wait for no LDS read
                a_frags(lds + nxt * kBuf, 0, af0, LMB_);
                __builtin_amdgcn_sched_barrier(0);
            } else {
                a_frags(abuf, ks, af, LMB_);
            }
#pragma unroll
            for (int cb = 0; cb < CB2; ++cb) {
                uint32_t bf[4];
                frag(bwc[0][cb][ks], q32, sop[0][cb], bf);
#pragma unroll
                for (int mb = 0; mb < LMB; ++mb) acc[mb][cb] = mfma32<BF16>(af[mb], bf, acc[mb][cb]);
                if constexpr (DUAL) {
                    uint32_t bg[4];
                    frag(bwc[NB - 1][cb][ks], q32, sop[NB - 1][cb], bg);
#pragma unroll
                    for (int mb = 0; mb < LMB; ++mb) acc2[mb][cb] = mfma32<BF16>(af[mb], bg, acc2[mb][cb]);
                }
            }
        }
        cur = nxt;
    };
    auto run = [&](auto LMB_) __attribute__((always_inline)) {
        for (int st = 0; st < stages; st += 2) {
            stage(st, 0, LMB_);
            stage(st + 1, 1, LMB_);
        }
    };
    if constexpr (SHORT) {
        if (kDeadWaves && dead) run(std::integral_constant<int, 0>{});
        else if (MB2 > 1 && lmb == 1) run(std::integral_constant<int, 1>{});
        else run(std::integral_constant<int, MB2>{});
    } else {
        run(std::integral_constant<int, MB2>{});
    }

    // Epilogue through LDS, one 32-column block and 16-row half of each 32-row
    // block at a time: lane (c32, q32) holds rows 32mb + 8(i/4) + 4q32 + i%4 of
    // column 32cb + c32, so elements i in [8hf, 8hf + 8) are the rows
    // 32mb + 16hf + [0, 16).  Every lane writes those to its wave's
    // [8 NMB][kEpPitch] fp32 block, then reads back 4 adjacent columns of one
    // row for epi_store4 (8 lanes cover a row's 32 columns).  The accumulators
    // are read only in fully unrolled loops, which keeps them in registers.
    const float fix = BF16 ? 1.0f : 0.5f;  // fp16 fragments carry 2x the weight
    float *ct = (float *)lds + (size_t)wave * 8 * NMB * kEpPitch;
    __syncthreads();  // the A buffers are free
    auto put = [&](auto &a, int cb, int hf) __attribute__((always_inline)) {
#pragma unroll
        for (int mb = 0; mb < MB2; ++mb)
#pragma unroll
            for (int j = 0; j < 8; ++j)
                ct[(16 * mb + 8 * (j >> 2) + 4 * q32 + (j & 3)) * kEpPitch + c32] = a[mb][cb][8 * hf + j] * fix;
        __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
        __builtin_amdgcn_wave_barrier();
    };
    // The postop and output type are fixed at compile time inside: one uniform
    // branch here instead of a switch per output (which cost more than the
    // rest of the epilogue together).
    auto epilogue = [&](auto P_, auto F_) __attribute__((always_inline)) {
        constexpr int P = decltype(P_)::value;
        constexpr bool F32 = decltype(F_)::value;
#pragma unroll
        for (int cb = 0; cb < CB2; ++cb) {
            const int n = n0 + wn + 32 * cb + 4 * (lane & 7);
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
                float up[DUAL ? NMB : 1][4];  // DUAL: DT(up) of this lane's 4 outputs per pass
                if constexpr (DUAL) {
                    put(acc, cb, hf);
#pragma unroll
                    for (int pass = 0; pass < NMB; ++pass) {
                        const float4 t = *(const float4 *)(ct + (8 * pass + (lane >> 3)) * kEpPitch + 4 * (lane & 7));
                        const float v4[4] = {t.x, t.y, t.z, t.w};
#pragma unroll
                        for (int i = 0; i < 4; ++i) up[pass][i] = dt2f<BF16>(f2dt<BF16>(v4[i]));
                    }
                    __builtin_amdgcn_s_waitcnt(0xc07f);
                    __builtin_amdgcn_wave_barrier();
                    put(acc2, cb, hf);
                } else {
                    put(acc, cb, hf);
                }
#pragma unroll
                for (int pass = 0; pass < NMB; ++pass) {
                    // block row 8 pass + lane / 8 = 16 mb + j -> tile row 32 mb + 16 hf + j
                    const int br = 8 * pass + (lane >> 3);
                    const int r = wm + 32 * (br >> 4) + 16 * hf + (br & 15);
                    const float4 t = *(const float4 *)(ct + br * kEpPitch + 4 * (lane & 7));
                    const float v4[4] = {t.x, t.y, t.z, t.w};
                    // (PAIR: row r of the second half is row r - kPairSplit of expert b's segment)
                    const int rr = hb ? r - kPairSplit : r;
                    const int crow = (hb ? pt.crowB : crow0) + rr;
                    if (rr < (PAIR ? (hb ? pt.nB : pt.nA) : mrows) && n < N) {
                        if constexpr (DUAL) {
                            uint32_t o[4];
#pragma unroll
                            for (int i = 0; i < 4; ++i) o[i] = f2dt<BF16>(epi_apply_c<1>(v4[i], up[pass][i], 0.0f));
                            *(uint2 *)((uint16_t *)C + (size_t)crow * N + n) =
                                make_uint2(o[0] | (o[1] << 16), o[2] | (o[3] << 16));
                        } else {
                            epi_store4_c<BF16, P, F32, !SHORT>(C, Other, Bias, N, crow, n, v4);  // (SHORT: MoE)
                        }
                    }
                }
                __builtin_amdgcn_wave_barrier();  // reads done before the next block's writes
            }
        }
    };
    if constexpr (DUAL) epilogue(std::integral_constant<int, 1>{}, std::integral_constant<bool, false>{});
    else epi_dispatch(postop, out_f32, epilogue);
}

// splits > 1 (deterministic split-K): workgroup (tile, slice s) runs K rows
// [s K / splits, (s + 1) K / splits) and writes its fp32 partial tile into
// part + s M N (no epilogue); k_splitk_reduce adds the slices in order.  The
// slices of a tile are adjacent in the XCD order, so they share its A rows.
template <class Cfg, bool BF16>
__global__ void __launch_bounds__(Cfg::THREADS)
k_int2_gemm(const uint16_t *__restrict__ A, const uint32_t *__restrict__ B,
            const uint16_t *__restrict__ S, void *__restrict__ C, const uint16_t *__restrict__ Other,
            const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32, int splits = 1,
            float *__restrict__ part = nullptr) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::lds_elems];
    const int mt = (M + Cfg::BM - 1) / Cfg::BM, nt = (N + Cfg::BN - 1) / Cfg::BN;
    int tm, tns;
    if (!xcd_tile_ashare(blockIdx.x, mt, nt * splits, tm, tns)) return;  // whole workgroup: padding
    // (uniform: kept in scalar registers, so the buffer descriptors built
    // from them stay scalar -- a divided value otherwise reads as per-lane)
    const int tn = __builtin_amdgcn_readfirstlane(tns / splits), sl = __builtin_amdgcn_readfirstlane(tns - tn * splits);
    const int kseg = __builtin_amdgcn_readfirstlane(K / splits), k0 = sl * kseg;
    const ARows ar{A + (size_t)tm * Cfg::BM * K + k0, nullptr, 1};
    const int mrows = min(Cfg::BM, M - tm * Cfg::BM);
    if (splits > 1) {
        C = part + (size_t)sl * M * N;
        Other = nullptr;
        Bias = nullptr;
        postop = 0;
        out_f32 = 1;
    }
    gemm_tile<Cfg, BF16>(ar, (uint32_t)(((size_t)mrows * K - k0) * 2), mrows, B + (size_t)(k0 / 16) * N,
                         S + (size_t)(k0 / kGS) * N, C, Other, Bias, tm * Cfg::BM, N, K, kseg, tn * Cfg::BN,
                         postop, out_f32, lds);
}

// The split-K reduction and epilogue: C[m, n..n+3] = ct(epi(sum over slices
// s = 0, 1, ... in order of part[s][m][n..n+3])), one thread per 4 outputs.
template <bool BF16>
__global__ void __launch_bounds__(256)
k_splitk_reduce(const float *__restrict__ part, int splits, void *__restrict__ C, const uint16_t *__restrict__ Other,
                const void *__restrict__ Bias, int M, int N, int postop, int out_f32) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, mn = (size_t)M * N;
    if (i >= mn / 4) return;
    float4 t = ((const float4 *)part)[i];
    for (int s = 1; s < splits; ++s) {
        const float4 u = ((const float4 *)(part + s * mn))[i];
        t.x += u.x;
        t.y += u.y;
        t.z += u.z;
        t.w += u.w;
    }
    const float v[4] = {t.x, t.y, t.z, t.w};
    const int m = (int)(4 * i / N), n = (int)(4 * i - (size_t)m * N);
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
        epi_store4_c<BF16, decltype(P_)::value, decltype(F_)::value, true>(C, Other, Bias, N, m, n, v);
    });
}

// The M-tiled BITCOS GEMM (bitcos_fp16_upcvt/bitcos_fp16_upcvt.cl:279-368)
// without a re-pack: the prefill engine's tiles decode the BITCOS weights
// themselves (gemm_tile BC).  The table maps (presence nibble m, next four sign
// bits s) to the nibble's four 2-bit int2 codes (0 / 1 / 3 = 0 / +1 / -1):
// row j present takes the next sign bit, 1 = -1.
template <class Cfg, bool BF16>
__global__ void __launch_bounds__(Cfg::THREADS)
k_bitcos_gemm(const uint16_t *__restrict__ A, const uint32_t *__restrict__ Bc, const uint16_t *__restrict__ S,
              void *__restrict__ C, const uint16_t *__restrict__ Other, const void *__restrict__ Bias, int M,
              int N, int K, int postop, int out_f32) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::lds_elems];
    __shared__ uint8_t lut[256];
    for (int i = threadIdx.x; i < 256; i += Cfg::THREADS) {
        const uint32_t m = (uint32_t)i >> 4, sg = (uint32_t)i & 15u;
        uint32_t taken = 0, out = 0;
        for (int j = 0; j < 4; ++j) {
            if (!((m >> j) & 1u)) continue;
            out |= (((sg >> taken) & 1u) ? 3u : 1u) << (2 * j);
            ++taken;
        }
        lut[i] = (uint8_t)out;
    }
    __syncthreads();
    const int mt = (M + Cfg::BM - 1) / Cfg::BM, nt = (N + Cfg::BN - 1) / Cfg::BN;
    int tm, tn;
    if (!xcd_tile_ashare(blockIdx.x, mt, nt, tm, tn)) return;  // whole workgroup: padding
    const ARows ar{A + (size_t)tm * Cfg::BM * K, nullptr, 1};
    const int mrows = min(Cfg::BM, M - tm * Cfg::BM);
    gemm_tile<Cfg, BF16, false, false, true>(ar, (uint32_t)((size_t)mrows * K * 2), mrows, Bc, S, C, Other, Bias,
                                             tm * Cfg::BM, N, K, K, tn * Cfg::BN, postop, out_f32, lds, nullptr,
                                             nullptr, lut);
}

// Grouped GEMM of the MoE prefill (int2_moe/int2_moe_prefill.cl:72-141): the
// rows of each expert e are meta[e] .. meta[e+1]-1 of the expert-sorted order,
// cut into tiles of moe_tile_rows() rows numbered from meta[E+1+e]; workgroup
// (tile, column block) finds its expert by a ballot over the tile offsets
// (moe_tile_expert).  A rows come from A_all[perm[p] / topk] when perm is given (the
// gather fused into the A-tile load), else from A_all[p].  Expert e's weights:
// B_all + e*(K/16)*N, S_all + e*(K/128)*N; C and Other are indexed by the
// sorted row p.
// PCfg (not void): the layer's tile list (desc, from k_moe_route) in place of
// the tile offsets: desc[0].x tiles, then per tile {row0 a, e_a << 8 | rows a,
// row0 b, e_b << 8 | rows b} with e_b < 0 for a tile of one expert; a tile of
// two experts' tails (each <= 64 rows) runs as PCfg, two 64-row wave rows of
// the same columns, the second row of waves on expert b's weights.
template <class Cfg, bool BF16, bool DUAL, class PCfg = void>
__global__ void __launch_bounds__(Cfg::THREADS)
k_int2_moe_gemm(const int *__restrict__ meta, const uint16_t *__restrict__ A_all,
                const int *__restrict__ perm, int topk, const uint32_t *__restrict__ B_all,
                const uint16_t *__restrict__ S_all, void *__restrict__ C_all,
                const uint16_t *__restrict__ Other_all, int E, int N, int K, int postop, int out_f32,
                int ntn, int arows, const uint32_t *__restrict__ B2_all, const uint16_t *__restrict__ S2_all,
                const int4 *__restrict__ desc = nullptr) {
    static_assert(Cfg::BM == kMoeTileRows, "MoE row tiles are kMoeTileRows rows");
    __shared__ __attribute__((aligned(16))) uint16_t lds[Cfg::lds_elems];
    int tile, tn;
    moe_tile_of(blockIdx.x, ntn, tile, tn);
    if constexpr (!std::is_void_v<PCfg>) {
        static_assert(PCfg::THREADS == Cfg::THREADS && PCfg::BN == Cfg::BN && PCfg::lds_elems <= Cfg::lds_elems,
                      "a pair tile fits the launch");
        if (tile >= desc[0].x) return;  // whole workgroup: past the last tile
        const int4 d = desc[1 + tile];
        const int ea = d.y >> 8, na = d.y & 255, r0a = d.x;
        const size_t boa = (size_t)ea * (K / 16) * N, soa = (size_t)ea * (K / kGS) * N;
        if (d.w < 0) {  // (uniform) one expert's rows
            const ARows ar = perm ? ARows{A_all, perm + r0a, topk} : ARows{A_all + (size_t)r0a * K, nullptr, 1};
            const uint32_t a_bytes = (uint32_t)((size_t)(perm ? arows : na) * K * 2);
            gemm_tile<Cfg, BF16, DUAL, true>(ar, a_bytes, na, B_all + boa, S_all + soa, C_all, Other_all, nullptr, r0a,
                                             N, K, K, tn * Cfg::BN, postop, out_f32, lds,
                                             DUAL ? B2_all + boa : nullptr, DUAL ? S2_all + soa : nullptr);
        } else {  // two experts' tails
            const int eb = d.w >> 8, nb = d.w & 255, r0b = d.z;
            const size_t bob = (size_t)eb * (K / 16) * N, sob = (size_t)eb * (K / kGS) * N;
            const ARows ar = perm ? ARows{A_all, perm + r0a, topk, perm + r0b, 0, kPairSplit}
                                  : ARows{A_all + (size_t)r0a * K, nullptr, 1, nullptr, r0b - r0a, kPairSplit};
            const uint32_t a_bytes = (uint32_t)((size_t)(perm ? arows : r0b - r0a + nb) * K * 2);
            const PairTile pt{B_all + bob, S_all + sob, DUAL ? B2_all + bob : nullptr, DUAL ? S2_all + sob : nullptr,
                              na, nb, r0b};
            gemm_tile<PCfg, BF16, DUAL, true, false, true>(ar, a_bytes, na, B_all + boa, S_all + soa, C_all, Other_all,
                                                           nullptr, r0a, N, K, K, tn * Cfg::BN, postop, out_f32, lds,
                                                           DUAL ? B2_all + boa : nullptr,
                                                           DUAL ? S2_all + soa : nullptr, nullptr, pt);
        }
        return;
    }
    const int tiles = meta[2 * E + 1];
    const int e = moe_tile_expert(meta, E, tile, threadIdx.x & 63);
    if (tile >= tiles) return;  // whole workgroup: past the last row tile
    const int row0 = meta[e];
    const int m0 = (tile - meta[E + 1 + e]) * Cfg::BM;
    const int mrows = min(Cfg::BM, meta[e + 1] - row0 - m0);
    // A rows: token rows of A_all through perm (arows rows in all), or the
    // sorted rows themselves
    const ARows ar = perm ? ARows{A_all, perm + row0 + m0, topk}
                          : ARows{A_all + (size_t)(row0 + m0) * K, nullptr, 1};
    const uint32_t a_bytes = (uint32_t)((size_t)(perm ? arows : mrows) * K * 2);
    const size_t bo = (size_t)e * (K / 16) * N, so = (size_t)e * (K / kGS) * N;
    gemm_tile<Cfg, BF16, DUAL, true>(ar, a_bytes, mrows, B_all + bo, S_all + so, C_all, Other_all, nullptr, row0 + m0,
                               N, K, K, tn * Cfg::BN, postop, out_f32, lds, DUAL ? B2_all + bo : nullptr,
                               DUAL ? S2_all + so : nullptr);
}

// Test hook: the B fragments the GEMM builds at unit scale (DT 1.0),
// D[word][0..3] = half 0, D[word][4..7] = half 1.
template <bool BF16>
__global__ void k_int2_gemm_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D, int words) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    ScaleOp<BF16> one;
    one.set(BF16 ? 0x3F80u : 0x3C00u);
    uint32_t b[8];
    frag(B[i], 0, one, b);
    frag(B[i], 1, one, b + 4);
    uint4 *d = (uint4 *)(D + (size_t)i * 8);
    d[0] = make_uint4(b[0], b[1], b[2], b[3]);
    d[1] = make_uint4(b[4], b[5], b[6], b[7]);
}

// ---- host side: tile choice ----------------------------------------------------

struct GemmPlan {
    int nmb, ncb, wvm, wvn;
};

// Tile choice between the shapes the engine compiles.  The 128 x 512 tile
// of eight 128 x 64 waves is the fastest per FLOP (measured 1.1-1.2 PFLOPS at
// M = 1024..4096), so it is taken whenever it yields at least 192 tiles (three
// quarters of the CUs busy in its first round; at N = 21504 its second,
// partial round still beats the 128 x 128 tile).  Below that the 128 x 128
// tile of 2 x 2 waves, two resident workgroups per CU (measured at 0.78 of
// the wide tile's MAC rate), wins while all of its tiles fit in one round of
// 512; past that one round of the wide tile is shorter.  The 128 x 128 tile
// runs as eight waves of 64 x 32 (two per SIMD with one workgroup per CU)
// rather than four of 64 x 64: fp16, M = 1024 K = N = 4096 47.5 -> 44.8 us,
// M = 512 47.2 -> 40.5 us, M = 1024 K = 2048 N = 6144 (384 tiles) 37.4 ->
// 35.9 us, M = 1000 K = 4096 N = 4112 61.9 -> 60.4 us.  Where those tiles
// number more than 256 (some CUs would hold two) and 128 x 256 tiles fit one
// per CU, the 128 x 256 tile of eight 128 x 32 waves runs instead: the same
// work on the busiest CU with half the weight decodes per MFMA (fp16, same
// box, two runs each, against the 128 x 128 tile: M = 1024 K = 4096 N = 6144
// 76.7 / 86.6 -> 69.0 / 74.1 us, M = 1024 K = 6144 N = 5120 110.0 / 115.8 ->
// 96.2 / 99.2, M = 512 K = 4096 N = 14336 89.7 / 85.0 -> 74.2 / 74.2, M =
// 2048 K = N = 4096 85.2 / 88.7 -> 75.0 / 79.5, M = 1024 K = 2048 N = 6144
// 39.5 / 39.3 -> 37.2 / 36.9).  (A 256 x 256 tile is slower per FLOP than
// the wide one, and a shape small enough to run it in one round runs the
// 128 x 128 tile in one round too.)
GemmPlan gemm_plan(int M, int N) {
    auto tiles = [&](int BM, int BN) { return (long)((M + BM - 1) / BM) * ((N + BN - 1) / BN); };
    const GemmPlan wide = {8, 4, 1, 8}, half = {8, 2, 1, 8}, square = {4, 2, 2, 4};
    if (tiles(128, 512) >= 192) return wide;
    if (gemm_half_tile(M, N)) return half;
    return tiles(128, 128) <= 512 ? square : wide;
}

template <class Cfg, bool BF16>
void gemm_launch(const void *A, const uint32_t *B, const void *S, void *C, const void *Other, const void *Bias,
                 int M, int N, int K, int postop, int out_f32, hipStream_t st) {
    const int mt = (M + Cfg::BM - 1) / Cfg::BM, nt = (N + Cfg::BN - 1) / Cfg::BN;
    hipLaunchKernelGGL((k_int2_gemm<Cfg, BF16>), dim3(xcd_ashare_grid(mt, nt)), dim3(Cfg::THREADS), 0, st,
                       (const uint16_t *)A, B, (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M, N, K,
                       postop, out_f32);
}

template <bool BF16>
void gemm_dispatch(const GemmPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                   const void *Other, const void *Bias, int M, int N, int K, int postop, int out_f32,
                   hipStream_t st) {
    if (p.wvn == 8 && p.ncb == 4) gemm_launch<TileCfg<8, 4, 1, 8>, BF16>(A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    else if (p.wvn == 8) gemm_launch<TileCfg<8, 2, 1, 8>, BF16>(A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    else gemm_launch<TileCfg<4, 2, 2, 4>, BF16>(A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
}

template <class Cfg, bool BF16, bool DUAL = false, class PCfg = void>
void moe_launch(const int *meta, const void *A_all, const int *perm, int topk, const uint32_t *B_all,
                const void *S_all, void *C_all, const void *Other_all, int E, int G, int N, int K, int postop,
                int out_f32, hipStream_t st, const uint32_t *B2_all = nullptr, const void *S2_all = nullptr,
                const int4 *desc = nullptr) {
    const int ntn = (N + Cfg::BN - 1) / Cfg::BN;
    const int max_tiles = moe_grid_tiles(G, Cfg::BM, E);
    hipLaunchKernelGGL((k_int2_moe_gemm<Cfg, BF16, DUAL, PCfg>), dim3((unsigned)(max_tiles * ntn)),
                       dim3(Cfg::THREADS), 0, st, meta, (const uint16_t *)A_all, perm, topk, B_all,
                       (const uint16_t *)S_all, C_all, (const uint16_t *)Other_all, E, N, K, postop, out_f32, ntn,
                       perm ? G / topk : G, B2_all, (const uint16_t *)S2_all, desc);
}

template <class Cfg, bool BF16>
void bitcos_gemm_launch(const void *A, const uint32_t *Bc, const void *S, void *C, const void *Other,
                        const void *Bias, int M, int N, int K, int postop, int out_f32, hipStream_t st) {
    const int mt = (M + Cfg::BM - 1) / Cfg::BM, nt = (N + Cfg::BN - 1) / Cfg::BN;
    hipLaunchKernelGGL((k_bitcos_gemm<Cfg, BF16>), dim3(xcd_ashare_grid(mt, nt)), dim3(Cfg::THREADS), 0, st,
                       (const uint16_t *)A, Bc, (const uint16_t *)S, C, (const uint16_t *)Other, Bias, M, N, K,
                       postop, out_f32);
}

}  // namespace

// The M-tiled BITCOS GEMM decoding the weights in its tiles (no workspace);
// tile choice as the int2 prefill GEMM's.
ternocl_status bitcos_gemm_mt_run(int dtype, const void *A, const uint32_t *Bc, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K, int postop,
                                  int out_f32, hipStream_t st) {
    // (the 128 x 256 tile against the 128 x 128 one here, same box, z = .5, two
    // runs each: M = 512 K = 5120 N = 14336 149.9 / 153.0 -> 110.6 / 113.4 us,
    // M = 1024 K = 4096 N = 6144 115.0 / 115.5 -> 85.7 / 84.8 us)
    const GemmPlan p = gemm_plan(M, N);
    const bool bf = dtype == TERNOCL_BF16;
    if (p.wvn == 8 && p.ncb == 4) {
        if (bf) bitcos_gemm_launch<TileCfg<8, 4, 1, 8>, true>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        else bitcos_gemm_launch<TileCfg<8, 4, 1, 8>, false>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    } else if (p.wvn == 8) {
        if (bf) bitcos_gemm_launch<TileCfg<8, 2, 1, 8>, true>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        else bitcos_gemm_launch<TileCfg<8, 2, 1, 8>, false>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    } else {
        if (bf) bitcos_gemm_launch<TileCfg<4, 4>, true>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        else bitcos_gemm_launch<TileCfg<4, 4>, false>(A, Bc, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
    return check_launch();
}

int moe_tile_rows() { return kMoeTileRows; }

// Column tile of the MoE GEMMs: the widest of 512 / 256 / 128 columns whose
// ragged last tile idles at most 1/10 of the MFMA work.
static int moe_bn(int N, int widest) {
    for (int bn = widest; bn > 128; bn >>= 1)
        if ((long)((N + bn - 1) / bn) * bn * 10 <= (long)N * 11) return bn;
    return 128;
}

ternocl_status moe_gemm_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                            const uint32_t *B_all, const void *S_all, void *C_all, const void *Other_all,
                            int E, int G, int N, int K, int postop, int out_f32, hipStream_t st,
                            const int4 *desc) {
    // 128-row tiles of eight waves side by side, each wave 128 rows x 64
    // columns (the dense engine's wave shape: 0.5 LDS fragment reads and 0.25
    // weight-word decodes per MFMA) on 512-column tiles; 128 x 32 waves on 256,
    // or 64 x 32 waves (2 x 4) on 128
    typedef TileCfg<8, 4, 1, 8> W512;
    typedef TileCfg<8, 2, 1, 8> W256;
    typedef TileCfg<4, 2, 2, 4> W128;
    typedef TileCfg<4, 8, 2, 4> P512;  // pair tiles: 2 x 4 waves of 64 rows, the same columns
    typedef TileCfg<4, 4, 2, 4> P256;
    const int bn = moe_bn(N, 512);
    if (dtype == TERNOCL_BF16) {
        if (desc) {  // the layer's tile list: two experts' tails may share a tile
            if (bn == 512) moe_launch<W512, true, false, P512>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
            else if (bn == 256) moe_launch<W256, true, false, P256>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
            else moe_launch<W128, true, false, W128>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
        } else if (bn == 512) moe_launch<W512, true>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
        else if (bn == 256) moe_launch<W256, true>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
        else moe_launch<W128, true>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
    } else {
        if (desc) {  // the layer's tile list: two experts' tails may share a tile
            if (bn == 512) moe_launch<W512, false, false, P512>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
            else if (bn == 256) moe_launch<W256, false, false, P256>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
            else moe_launch<W128, false, false, W128>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st, nullptr, nullptr, desc);
        } else if (bn == 512) moe_launch<W512, false>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
        else if (bn == 256) moe_launch<W256, false>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
        else moe_launch<W128, false>(meta, A_all, perm, topk, B_all, S_all, C_all, Other_all, E, G, N, K, postop, out_f32, st);
    }
    return check_launch();
}

// The gate/up pair of the MoE layer in one launch: Hs = DT(silu(A x Bg) * DT(A x Bu)),
// bit-identical to moe_gemm_run(up, postop 0) followed by moe_gemm_run(gate, postop 1).
// Eight waves side by side, each 128 rows x 32 columns of both products (one
// A fragment feeds four MFMAs per weight set) on 256-column tiles, or 2 x 4
// waves of 64 x 32 on 128.
ternocl_status moe_gate_up_run(int dtype, const int *meta, const void *A_all, const int *perm, int topk,
                               const uint32_t *Bu, const void *Su, const uint32_t *Bg, const void *Sg, void *Hs,
                               int E, int G, int N, int K, hipStream_t st, const int4 *desc) {
    typedef TileCfg<8, 2, 1, 8> W256;
    typedef TileCfg<4, 2, 2, 4> W128;
    typedef TileCfg<4, 4, 2, 4> P256;  // pair tiles: 2 x 4 waves of 64 rows, the same columns
    const bool wide = moe_bn(N, 256) == 256;
    if (desc) {  // the layer's tile list: two experts' tails may share a tile
        if (dtype == TERNOCL_BF16) {
            if (wide) moe_launch<W256, true, true, P256>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg, desc);
            else moe_launch<W128, true, true, W128>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg, desc);
        } else {
            if (wide) moe_launch<W256, false, true, P256>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg, desc);
            else moe_launch<W128, false, true, W128>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg, desc);
        }
        return check_launch();
    }
    if (dtype == TERNOCL_BF16) {
        if (wide) moe_launch<W256, true, true>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg);
        else moe_launch<W128, true, true>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg);
    } else {
        if (wide) moe_launch<W256, false, true>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg);
        else moe_launch<W128, false, true>(meta, A_all, perm, topk, Bu, Su, Hs, nullptr, E, G, N, K, 1, 0, st, Bg, Sg);
    }
    return check_launch();
}

ternocl_status int2_gemm_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st) {
    const int words = K / 16 * N;
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_gemm_decode<true>, dim3((words + 255) / 256), dim3(256), 0, st, B, D, words);
    else
        hipLaunchKernelGGL(k_int2_gemm_decode<false>, dim3((words + 255) / 256), dim3(256), 0, st, B, D, words);
    return check_launch();
}

// Split-K slices for a shape whose 128 x 512 tiles would leave CUs idle: the
// fewest slices (2, 4 or 8) that make >= 192 work units, each slice a
// multiple of 128 rows and at least 2048 rows of K (1024 up to M = 256); 1 =
// no split.  The slices' partials cost 8 bytes per output and slice of
// memory traffic against 2 K flops per output of the GEMM, so short slices
// lose to the unsplit 128 x 128 tiles.  Same box, fp16 / int8 with quant_a,
// the 1024-row minimum against this rule: M = 1024 K = N = 4096 53.3 / 52.8
// -> 47.5 / 51.7 us, M = 1024 K = 6144 N = 5120 101.1 / 97.7 -> 94.7 / 94.6,
// M = 1000 K = 4096 N = 4112 76.0 / 75.1 -> 62.0 / 66.8; at M = 200 K = 5120
// N = 16384 the 1280-row slices still win (int8 52.4 against 58.1 unsplit).
int gemm_splits(int M, int N, int K) {
    const long tiles = (long)((M + 127) / 128) * ((N + 511) / 512);
    if (tiles >= 192) return 1;
    const int kmin = M <= 256 ? 1024 : 2048;
    for (int s = 2; s <= 8; s *= 2)
        if (K % (128 * s) == 0 && K / s >= kmin && tiles * s >= 192) return s;
    return 1;
}

// The split-K reduction: C = ct(epi(sum of the slices in order)) (also the
// int8 GEMM's, int2_int8.hip).
hipError_t splitk_reduce_launch(int dtype, const float *part, int splits, void *C, const void *Other,
                                const void *Bias, int M, int N, int postop, int out_f32, hipStream_t st) {
    const unsigned blocks = (unsigned)(((size_t)M * N / 4 + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_splitk_reduce<true>, dim3(blocks), dim3(256), 0, st, part, splits, C,
                           (const uint16_t *)Other, Bias, M, N, postop, out_f32);
    else
        hipLaunchKernelGGL(k_splitk_reduce<false>, dim3(blocks), dim3(256), 0, st, part, splits, C,
                           (const uint16_t *)Other, Bias, M, N, postop, out_f32);
    return hipGetLastError();
}

// Workspace of the split-K path: the header, then the fp32 partial tiles of
// every slice.
size_t int2_gemm_ws_need(int M, int N, int K) {
    const int s = gemm_splits(M, N, K);
    return s > 1 ? kWsHeader + (size_t)s * M * N * 4 : 0;
}

// With a workspace of int2_gemm_ws_need bytes (16-byte aligned), shapes that
// split run the 128 x 512 tile over K-slices into it and a reduction kernel
// adds the slices in order and applies the epilogue (deterministic: the same
// bits on every run); without one they take the plan of gemm_plan.  Shapes
// of the 128 x 256 tile with at least 192 such tiles take it with or without
// a workspace: it beat the split (fp16, same box: M = 1024 K = 4096 N = 6144
// 72.0-76.4 -> 68.7-71.1 us, M = 512 K = 4096 N = 14336 81.0-84.5 ->
// 71.7-75.1, M = 2048 K = N = 4096 84.4-94.4 -> 75.1-81.3); with fewer the
// CUs it leaves idle cost more than the split (M = 1024 K = 17408 N = 5120,
// 160 tiles: 240.2 / 237.9 us split against 255.5 / 254.7; M = 1000 K = 8192
// N = 4112, 136 tiles: 124.3 / 129.7 against 121.4 / 123.7).  (The int8 GEMM
// keeps its split there; the workspace size covers both.)
ternocl_status int2_gemm_mfma_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K,
                                  int postop, int out_f32, hipStream_t st, void *ws, size_t ws_bytes) {
    const bool half_first = gemm_half_tile(M, N) && (long)((M + 127) / 128) * ((N + 255) / 256) >= 192;
    const int splits = half_first ? 1 : gemm_splits(M, N, K);
    const bool bf = dtype == TERNOCL_BF16;
    if (splits > 1 && ws && ws_bytes >= int2_gemm_ws_need(M, N, K) && ((uintptr_t)ws & 15) == 0) {
        typedef TileCfg<8, 4, 1, 8> Cfg;
        const int mt = (M + Cfg::BM - 1) / Cfg::BM, nt = (N + Cfg::BN - 1) / Cfg::BN;
        float *part = (float *)((uint8_t *)ws + kWsHeader);
        const dim3 grid(xcd_ashare_grid(mt, nt * splits));
        if (bf)
            hipLaunchKernelGGL((k_int2_gemm<Cfg, true>), grid, dim3(Cfg::THREADS), 0, st, (const uint16_t *)A, B,
                               (const uint16_t *)S, C, nullptr, nullptr, M, N, K, 0, 1, splits, part);
        else
            hipLaunchKernelGGL((k_int2_gemm<Cfg, false>), grid, dim3(Cfg::THREADS), 0, st, (const uint16_t *)A, B,
                               (const uint16_t *)S, C, nullptr, nullptr, M, N, K, 0, 1, splits, part);
        // (an error of the slices' launch stays pending for the reduction's check)
        return launch_status(splitk_reduce_launch(dtype, part, splits, C, Other, Bias, M, N, postop, out_f32, st));
    }
    const GemmPlan p = gemm_plan(M, N);
    if (bf) gemm_dispatch<true>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    else gemm_dispatch<false>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return check_launch();
}

}  // namespace tcl
