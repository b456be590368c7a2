// int2_int8.hip -- the int2 x int8 prefill path on gfx950: the activation
// quantization pre-kernel and the s8 x s2 GEMM, replacing quant_a and
// int2_int8_{gemv,gemm_mt} of int2_via_int2_x_int8_dpas/int2_int8_dpas.cl
// (:101-123, :210-281, :313-385) in both of its quantization modes (QMODE 0:
// upfront, the GEMM reads int8 Aq; QMODE 1: the GEMM quantizes DT A tiles).
//
//   SA[g, m] = DT(127 / max(absmax_{k in g} |A[m, k]|, FLT_EPSILON))
//   Aq[m, k] = sat_int8(rte(A[m, k] * SA[k/128, m]))
//   C[m, n]  = ct(epi(sum_g float(sum_{k in g} Aq[m,k] * v(B[k,n])) * (SB[g,n] * (1 / SA[g,m]))))
//
// with v the 2-bit two's-complement value of the code ({0,1,2,3} = {0,1,-2,-1}).
//
// quant_a is HBM-bound: one thread per 16 activations (two 16-byte loads), the 8
// threads of a 128-group reduce the absmax with cross-lane xor shuffles.  The
// scale is 127 / x with a correctly rounded fp32 divide (the reference builds
// with -cl-fp32-correctly-rounded-divide-sqrt), q = rint(a * sa) saturated; the
// product of two 16-bit floats is exact in fp32, so q is bit-exact.
//
// The GEMM: a workgroup of 4 waves computes a 128 x 128 tile of C, each wave a
// 64 x 64 quarter as 4 x 4 v_mfma_i32_16x16x64_i8 tiles; K advances one
// 128-row scale group at a time (two MFMA k-steps of 64).  Two workgroups share
// a CU (183 VGPRs: two waves per SIMD).
//   * B stays packed in HBM / L2: lane (c, q) of a wave loads, per k-step and
//     16-column block, the word of k rows 16*(4*ks+q) .. +15 of its column and
//     turns it into the 16 int8 of its MFMA B fragment with v_perm_b32 through
//     the byte table {0x00, 0x01, 0xFE, 0xFF} indexed by the code:
//     dword i = codes of rows i, i+4, i+8, i+12 (selector (w >> 2i) & 0x03030303);
//   * A goes global -> registers -> LDS once per workgroup and group, each
//     16-byte chunk of int8 4x4 byte-transposed on the way (QMODE 1: quantized
//     and packed straight into that order) so that its dword i holds rows i,
//     i+4, i+8, i+12 too (the same k order as B: the int32 dot is exact
//     whatever the order, as long as A and B agree);
//   * 1 / SA[g, m] of the tile's 128 rows is computed once per group into LDS;
//   * each 16-row block's dot products start from zero in int32 accumulators
//     and are folded into fp32 accumulators with acc += float(dot) * (SB * inv),
//     the order of the reference's host gold (int2_via_int2_x_int8_dpas/main.cpp:113-116);
//     the fold of block mb runs between the MFMAs of block mb + 1;
//   * all loads are buffer loads with offsets computed once per kernel.
#include "common.hpp"

#include <cfloat>

namespace tcl {
// (int2_gemm_mfma.hip: the split-K slice count and reduction of the prefill GEMM,
// and its rule for 128 x 256 tiles)
int gemm_splits(int M, int N, int K);
bool gemm_half_tile(int M, int N);
hipError_t splitk_reduce_launch(int dtype, const float *part, int splits, void *C, const void *Other,
                                const void *Bias, int M, int N, int postop, int out_f32, hipStream_t st);
namespace {

typedef int i32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr float kEps = FLT_EPSILON;  // xetla's absmax floor, int2_int8_dpas.cl:59

__host__ __device__ constexpr int ldsa_of(int M) { return (M + 31) & ~31; }

// ---- quant_a ---------------------------------------------------------------

template <bool BF16>
__global__ void __launch_bounds__(256)
k_quant_a(const uint16_t *__restrict__ A, uint16_t *__restrict__ SA, int8_t *__restrict__ Aq, int M,
          int K, const int *__restrict__ perm = nullptr, int topk = 1, const int *__restrict__ nrows = nullptr) {
    const int cpr = K >> 4;  // 16-element chunks per row (a multiple of 8)
    const size_t t = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    // the 8 chunks of a group are 8 aligned consecutive threads: they leave together
    if (t >= (size_t)M * cpr) return;
    const int m = (int)(t / cpr), c = (int)(t - (size_t)m * cpr);
    // nrows (the MoE layer): only the *nrows rows the route kept are read and
    // written; perm: row m of the output is row perm[m] / topk of A
    if (nrows && m >= *nrows) return;
    const int src = perm ? perm[m] / topk : m;
    const uint16_t *row = A + (size_t)src * K + 16 * (size_t)c;
    const uint4 v0 = *(const uint4 *)row, v1 = *(const uint4 *)(row + 8);
    const uint32_t w[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
    float a[16];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[2 * i] = dt2f<BF16>(w[i] & 0xffffu);
        a[2 * i + 1] = dt2f<BF16>(w[i] >> 16);
    }
    float mx = 0.0f;
#pragma unroll
    for (int i = 0; i < 16; ++i) mx = fmaxf(mx, fabsf(a[i]));
#pragma unroll
    for (int o = 4; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 8));
    const uint32_t sh = f2dt<BF16>(127.0f / fmaxf(mx, kEps));
    if ((c & 7) == 0) SA[(size_t)(c >> 3) * ldsa_of(M) + m] = (uint16_t)sh;
    const float s = dt2f<BF16>(sh);
    uint32_t q[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        // exact product, rounded to nearest even and saturated; NaN (0 * inf
        // when an fp16 scale overflows) gives 0, as convert_char8_sat_rte
        const float p = a[i] * s;
        const float r = p == p ? fminf(fmaxf(__builtin_rintf(p), -128.0f), 127.0f) : 0.0f;
        q[i >> 2] |= ((uint32_t)(int)r & 0xffu) << (8 * (i & 3));
    }
    if (Aq) *(uint4 *)(Aq + (size_t)m * K + 16 * (size_t)c) = make_uint4(q[0], q[1], q[2], q[3]);
}

// ---- s8 x s2 GEMM ------------------------------------------------------------

constexpr int QA_PITCH = 144;  // bytes per LDS row of the A tile (128 + 16: conflict-free b128 reads)
constexpr uint32_t kCodeLut = 0xFFFE0100u;  // int8 of code 0, 1, 2, 3

// out[i] byte b = byte i of d[b] (4 x 4 byte transpose)
__device__ __forceinline__ void transpose4x4(const uint32_t d[4], uint32_t o[4]) {
    const uint32_t p0 = __builtin_amdgcn_perm(d[1], d[0], 0x06020400u);  // d0.b0 d1.b0 d0.b2 d1.b2
    const uint32_t p1 = __builtin_amdgcn_perm(d[1], d[0], 0x07030501u);  // d0.b1 d1.b1 d0.b3 d1.b3
    const uint32_t p2 = __builtin_amdgcn_perm(d[3], d[2], 0x06020400u);
    const uint32_t p3 = __builtin_amdgcn_perm(d[3], d[2], 0x07030501u);
    o[0] = __builtin_amdgcn_perm(p2, p0, 0x05040100u);
    o[1] = __builtin_amdgcn_perm(p3, p1, 0x05040100u);
    o[2] = __builtin_amdgcn_perm(p2, p0, 0x07060302u);
    o[3] = __builtin_amdgcn_perm(p3, p1, 0x07060302u);
}

// B fragment of one word: dword i byte b = int8 value of row 4b + i.
__device__ __forceinline__ i32x4_t decode_s2(uint32_t w) {
    i32x4_t r;
    r[0] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, w & 0x03030303u);
    r[1] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 2) & 0x03030303u);
    r[2] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 4) & 0x03030303u);
    r[3] = (int)__builtin_amdgcn_perm(kCodeLut, kCodeLut, (w >> 6) & 0x03030303u);
    return r;
}

// Tile shape: WVM x WVN waves, each owning MB x CB blocks of 16 x 16 outputs.
template <int MB_, int CB_, int WVM_, int WVN_> struct QTile {
    static constexpr int MB = MB_, CB = CB_, WVM = WVM_, WVN = WVN_;
    static constexpr int THREADS = 64 * WVM * WVN;
    static constexpr int BM = 16 * MB * WVM, BN = 16 * CB * WVN;
    static constexpr int A_PER_THREAD = BM * 8 / THREADS;  // 16-byte A chunks per thread and group
    static_assert(BM * 8 % THREADS == 0, "A chunks must divide evenly");
    static_assert(THREADS % BM == 0 && (BM & (BM - 1)) == 0, "threads cover the tile rows evenly (1 / SA)");
    static constexpr int EP_PITCH = 20;  // epilogue floats per row: 16 + 4 (16-byte aligned rows)
    static constexpr int STAGE_BYTES = 2 * BM * QA_PITCH + 2 * BM * 4;
    static constexpr int EPI_BYTES = (THREADS / 64) * 16 * MB * EP_PITCH * 4;
    static constexpr int LDS_BYTES = STAGE_BYTES > EPI_BYTES ? STAGE_BYTES : EPI_BYTES;
};

// This wave's packed B words and raw scale bits of one group.
template <int CB> struct QBSlab {
    uint32_t w[CB][2], sb[CB];
};

// In-GEMM quantization (the reference's QMODE 1, int2_int8_dpas.cl:61-68 and
// quant8x32 :70-99): the int8 of a DT activation is the low byte of
// fma(a, sa, 1.5 * 2^23), which rounds a * sa (exact in fp32) to the nearest
// even integer; |a * sa| <= 127.06 by the construction of sa, so it equals
// quant_a's saturating conversion for every finite input.
template <bool BF16>
__device__ __forceinline__ uint32_t q8_bits(uint32_t h, float sa) {
    return __float_as_uint(__builtin_fmaf(dt2f<BF16>(h), sa, 12582912.0f));
}

// QA = false: A tiles come from Aq (int8, written by quant_a: the reference's
// QMODE 0).  QA = true: from the DT activations A, quantized while staged.
template <class TC, bool BF16, bool QA>
__global__ void __launch_bounds__(TC::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_int2_int8_gemm(const void *__restrict__ Asrc, const uint16_t *__restrict__ SA,
                 const uint32_t *__restrict__ B, const uint16_t *__restrict__ SB,
                 void *__restrict__ C, const uint16_t *__restrict__ Other,
                 const void *__restrict__ Bias, int M, int N, int K, int postop, int out_f32) {
    constexpr int MB = TC::MB, CB = TC::CB, BM = TC::BM, BN = TC::BN, AP = TC::A_PER_THREAD;
    // LDS: two A tiles [BM][QA_PITCH] and two 1 / SA vectors [BM] while K runs,
    // then the epilogue's per-wave transposition blocks
    __shared__ __attribute__((aligned(16))) uint8_t lds[TC::LDS_BYTES];
    uint8_t (*lds_a)[BM * QA_PITCH] = (uint8_t (*)[BM * QA_PITCH])lds;
    float (*lds_inv)[BM] = (float (*)[BM])(lds + 2 * BM * QA_PITCH);

    int tm, tn;
    const int lda = ldsa_of(M);
    const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
    if (!xcd_tile_ashare(blockIdx.x, mt, nt, tm, tn)) return;  // whole workgroup: padding
    const int m0 = tm * BM, n0 = tn * BN;
    const int mrows = min(BM, M - m0);
    const int groups = K / kGS;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int c16 = lane & 15, q = lane >> 4;
    const int wm = (wave / TC::WVN) * (16 * MB), wn = (wave % TC::WVN) * (16 * CB);

    // All operand loads are buffer loads whose per-lane offsets are set up
    // once: per group only scalar offsets (A, SA) or one add per pointer (B,
    // SB) change.  Loads are unconditional -- a load under a branch would be
    // waited for at the branch's end -- and those of the group after the last
    // read in-range memory or return 0.
    //
    // A staging: thread tid owns the 16-byte chunk (tid & 7) of rows
    // (tid >> 3) + (THREADS / 8) u; rows past mrows lie past the buffer's end
    // and load as 0.
    // (QA: the chunk is 16 DT activations, 32 bytes.)
    constexpr int RSTEP = TC::THREADS / 8;
    constexpr int ES = QA ? 2 : 1;  // bytes per staged A element in memory
    const int arow0 = tid >> 3, achunk = tid & 7;
    const __amdgpu_buffer_rsrc_t rA =
        buf_rsrc((const uint8_t *)Asrc + (size_t)m0 * K * ES, (uint32_t)((size_t)mrows * K * ES));
    uint32_t va[AP];
#pragma unroll
    for (int u = 0; u < AP; ++u) va[u] = (uint32_t)(((arow0 + RSTEP * u) * K + 16 * achunk) * ES);
    uint4 av[AP][ES];
    auto a_load = [&](int g) {
        const int gc = g < groups ? g : groups - 1;
#pragma unroll
        for (int u = 0; u < AP; ++u)
#pragma unroll
            for (int e = 0; e < ES; ++e) {
                const i32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rA, va[u] + 16 * e, gc * kGS * ES, 0);
                av[u][e] = make_uint4((uint32_t)t[0], (uint32_t)t[1], (uint32_t)t[2], (uint32_t)t[3]);
            }
    };
    // 1 / SA of the tile's rows (thread tid < BM: row tid)
    const __amdgpu_buffer_rsrc_t rSA = buf_rsrc(SA + m0, (uint32_t)(((size_t)groups * lda - m0) * 2));
    // QA: SA of the rows this thread stages (row clamped below mrows)
    uint32_t vsq[QA ? AP : 1], sq_raw[QA ? AP : 1];
    if constexpr (QA) {
#pragma unroll
        for (int u = 0; u < AP; ++u) vsq[u] = (uint32_t)min(arow0 + RSTEP * u, mrows - 1) * 2;
    }
    auto sq_load = [&](int g) {
        if constexpr (QA) {
            const int gc = g < groups ? g : groups - 1;
#pragma unroll
            for (int u = 0; u < AP; ++u) sq_raw[u] = __builtin_amdgcn_raw_buffer_load_b16(rSA, vsq[u], gc * lda * 2, 0);
        }
    };
    // threads t and t + BM (when THREADS = 2 BM) load and write the same row's
    // value, so the store below needs no branch
    const int srow = tid & (BM - 1);
    // (rows past mrows load row mrows - 1: the last group's row m0 + srow may
    // lie past SA's end, and the SGPR offset is not range-checked)
    const uint32_t vsa = (uint32_t)min(srow, mrows - 1) * 2;
    uint32_t sa_raw = 0;
    auto sa_load = [&](int g) {
        const int gc = g < groups ? g : groups - 1;
        sa_raw = __builtin_amdgcn_raw_buffer_load_b16(rSA, vsa, gc * lda * 2, 0);
    };
    auto a_store = [&](int buf) {
#pragma unroll
        for (int u = 0; u < AP; ++u) {
            uint32_t o[4];
            if constexpr (QA) {
                // quantize the 16 activations; dword i gathers the int8 of
                // k = i, i + 4, i + 8, i + 12 (the transposed order)
                const float sa = dt2f<BF16>(sq_raw[u]);
                const uint32_t h[8] = {av[u][0].x, av[u][0].y, av[u][0].z, av[u][0].w,
                                       av[u][1].x, av[u][1].y, av[u][1].z, av[u][1].w};
                uint32_t qb[16];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    qb[2 * j] = q8_bits<BF16>(h[j] & 0xffffu, sa);
                    qb[2 * j + 1] = q8_bits<BF16>(h[j] >> 16, sa);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    o[i] = __builtin_amdgcn_perm(qb[4 + i], qb[i], 0x0c0c0400u) |
                           __builtin_amdgcn_perm(qb[12 + i], qb[8 + i], 0x04000c0cu);
            } else {
                const uint32_t d[4] = {av[u][0].x, av[u][0].y, av[u][0].z, av[u][0].w};
                transpose4x4(d, o);
            }
            *(uint4 *)(&lds_a[buf][(arow0 + RSTEP * u) * QA_PITCH + 16 * achunk]) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        const float sa = dt2f<BF16>(sa_raw);
        lds_inv[buf][srow] = (srow < mrows && sa != 0.0f) ? 1.0f / sa : 0.0f;
    };
    // B words of this wave for group g: block cb, k-step ks -> word kp = 8g + 4ks + q
    // of column n0 + wn + 16 cb + c16.  The offsets advance by a group per load
    // (vb0, vb1, vsb), so a 16-column block past N (when N % BN != 0) reads the
    // next row's words -- in range, and only feeding outputs that are not
    // stored -- or, in the last row, 0.
    const __amdgpu_buffer_rsrc_t rB = buf_rsrc(B + n0, (uint32_t)(((size_t)(K / 16) * N - n0) * 4));
    const __amdgpu_buffer_rsrc_t rSB = buf_rsrc(SB + n0, (uint32_t)(((size_t)groups * N - n0) * 2));
    uint32_t vb0 = (uint32_t)((q * N + wn + c16) * 4), vb1 = vb0 + (uint32_t)(16 * N);
    uint32_t vsb = (uint32_t)((wn + c16) * 2);
    auto b_load = [&](QBSlab<CB> &sl) {
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
            sl.w[cb][0] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rB, vb0 + 64 * cb, 0, 0);
            sl.w[cb][1] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rB, vb1 + 64 * cb, 0, 0);
            sl.sb[cb] = __builtin_amdgcn_raw_buffer_load_b16(rSB, vsb + 32 * cb, 0, 0);
        }
        vb0 += (uint32_t)(32 * N);
        vb1 += (uint32_t)(32 * N);
        vsb += (uint32_t)(2 * N);
    };

    f32x4_t acc[MB][CB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) acc[mb][cb] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    // One group: issue the next group's loads, then the MFMAs of this group
    // one 16-row block at a time, each block's int32 dots folded into the
    // fp32 accumulators right away: acc += float(dot) * (SB * (1 / SA)).
    auto group = [&](int g, const QBSlab<CB> &cur, QBSlab<CB> &nxt) __attribute__((always_inline)) {
        __syncthreads();  // tile g staged; tile g - 1 consumed
        const int buf = g & 1;
        a_load(g + 1);
        sa_load(g + 1);
        sq_load(g + 1);
        b_load(nxt);
        i32x4_t bf[CB][2];
        float sbf[CB];
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) bf[cb][ks] = decode_s2(cur.w[cb][ks]);
            sbf[cb] = dt2f<BF16>(cur.sb[cb]);
        }
        // Software pipeline over the 16-row blocks: the two MFMAs of (mb, cb)
        // are issued next to the fold of (mb - 1, cb), pinned in that order by
        // scheduling barriers, so the matrix core and the VALU work side by
        // side within the wave instead of in two long phases.
        auto a_frag = [&](int mb, i32x4_t af[2]) __attribute__((always_inline)) {
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
                const uint4 v = *(const uint4 *)(&lds_a[buf][(wm + 16 * mb + c16) * QA_PITCH + (4 * ks + q) * 16]);
                af[ks] = i32x4_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
        };
        auto inv_of = [&](int mb) __attribute__((always_inline)) {
            return *(const f32x4_t *)(&lds_inv[buf][wm + 16 * mb + 4 * q]);
        };
        i32x4_t dp[CB], dc[CB];
        {
            i32x4_t af[2];
            a_frag(0, af);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                dp[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0], bf[cb][0], i32x4_t{0, 0, 0, 0}, 0, 0, 0);
                dp[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[1], bf[cb][1], dp[cb], 0, 0, 0);
            }
        }
#pragma unroll
        for (int mb = 1; mb <= MB; ++mb) {
            i32x4_t af[2];
            if (mb < MB) a_frag(mb, af);
            const f32x4_t inv = inv_of(mb - 1);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) {
                if (mb < MB) {
                    dc[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[0], bf[cb][0], i32x4_t{0, 0, 0, 0}, 0, 0, 0);
                    dc[cb] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[1], bf[cb][1], dc[cb], 0, 0, 0);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mb - 1][cb][i] += (float)dp[cb][i] * (sbf[cb] * inv[i]);
                __builtin_amdgcn_sched_barrier(0);
            }
#pragma unroll
            for (int cb = 0; cb < CB; ++cb) dp[cb] = dc[cb];
        }
        a_store(buf ^ 1);  // after the last group: harmless, never read
    };

    QBSlab<CB> cur;
    a_load(0);
    sa_load(0);
    sq_load(0);
    b_load(cur);
    a_store(0);
    for (int g = 0; g < groups; ++g) {
        QBSlab<CB> nxt;
        group(g, cur, nxt);
        cur = nxt;
    }

    // Epilogue through LDS, one 16-column block at a time: lane (c16, q) holds
    // rows wm + 16mb + 4q + i of column wn + 16cb + c16; it writes them to its
    // wave's [16 MB][EP_PITCH] fp32 block, then reads back 4 adjacent columns of
    // one row for epi_store4.  (Reading the accumulators only in fully unrolled
    // loops with small bodies keeps the array in registers.)
    constexpr int EP = TC::EP_PITCH;
    float *ct = (float *)lds + (size_t)wave * 16 * MB * EP;
    __syncthreads();  // the A tiles are free
    // postop and output type fixed at compile time inside (one uniform branch
    // instead of a switch per output)
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
        constexpr int P = decltype(P_)::value;
        constexpr bool F32 = decltype(F_)::value;
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb)
#pragma unroll
                for (int i = 0; i < 4; ++i) ct[(16 * mb + 4 * q + i) * EP + c16] = acc[mb][cb][i];
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
            __builtin_amdgcn_wave_barrier();
            const int n = n0 + wn + 16 * cb + 4 * (lane & 3);
#pragma unroll
            for (int pass = 0; pass < MB; ++pass) {
                const int r = wm + 16 * pass + (lane >> 2);
                const float4 t = *(const float4 *)(ct + (16 * pass + (lane >> 2)) * EP + 4 * (lane & 3));
                const float v4[4] = {t.x, t.y, t.z, t.w};
                if (r < mrows && n < N) epi_store4_c<BF16, P, F32, true>(C, Other, Bias, N, m0 + r, n, v4);
            }
            __builtin_amdgcn_wave_barrier();  // reads of this block done before the next block's writes
        }
    });
}

// ---- wide-tile s8 x s2 GEMM (v_mfma_i32_32x32x32_i8) ------------------------
//
// The fold acc += float(dot) * (SB * (1 / SA)) is due once per output and
// 128-row group whatever the tiling, and on gfx950 one VALU instruction of a
// wave takes 4 cycles against 32 for a 32 x 32 x 32 int8 MFMA that covers 32
// of the group's 128 rows: the fold's three VALU operations per output and
// group cost 1.5x the group's MFMA time.  What the tiling changes is the rest
// of the VALU work (the B decode, amortised over a wave's rows) and the LDS
// traffic (the A fragments, amortised over a wave's columns).  This engine:
//   * a workgroup of WVN waves side by side, each 32 RMB rows x 64 columns
//     (RMB x 2 blocks of 32 x 32 outputs), 128 x 512 at the default shape:
//     each 16-byte A chunk staged once serves 512 columns and each decoded
//     B word 128 rows;
//   * one LDS stage per 128-row group: the tile's A rows (4 x 4
//     byte-transposed as in the 128 x 128 engine) and 1 / SA of its rows;
//     three stage buffers, the next stage stored in the middle of the current
//     one, one barrier per stage;
//   * lane (c, h) = (l % 32, l / 32) holds k rows 16 h .. 16 h + 15 of each
//     32-row k-chunk: the B fragment is one packed word per (column, k-chunk)
//     through decode_s2, the A fragment the 16-byte chunk 2 kc + h of its row;
//   * each block's dot products run from zero over the group's four k-chunks
//     in int32 and are folded into the fp32 accumulators as in the 128 x 128
//     engine.
// GRP (the int8 MoE prefill's grouped GEMM, int2_moe/int2_moe_prefill_int8.cl:
// 86-176): M = G sorted rows, SA [K/128][ldsa(G)]; expert e owns rows meta[e]
// .. meta[e+1]-1 cut into BM-row tiles numbered from meta[E+1+e] (BM equals the
// route's tile rows); workgroup (tile, column block) finds its expert with a
// ballot over the tile offsets and runs the GEMM on its segment: weights B + e (K/16) N, SB + e
// (K/128) N, and Aq, SA's columns, C and Other shifted to the segment's rows.
// With perm, the A rows are gathered instead: sorted row p reads row
// perm[p] / topk of Aq [arows][K] and its column of SA [K/128][ldsa(arows)]
// (the token rows quantized once, as the reference's quant_x + gather_q).
// DUAL (the int8 MoE layer's up and gate in one pass over the gathered rows,
// int2_moe/prefill.cpp:268-279 with --int8 1): each wave's two 32-column
// blocks are the same 32 columns of B (up) and B2 (gate), BN = 32 WVN; C =
// DT(silu(gate) * DT(up)), the bits of the up launch (postop 0, DT out)
// followed by the gate launch (postop 1 with Other = that DT output).
template <int RMB_, int WVN_, int CB_ = 2> struct WTile {
    static constexpr int RMB = RMB_, WVN = WVN_, CB = CB_;  // CB: 32-column blocks per wave
    static constexpr int THREADS = 64 * WVN;
    static constexpr int BM = 32 * RMB, BN = 32 * CB * WVN;
    static constexpr int AP = BM * 8 / THREADS;  // 16-byte A chunks per thread and stage
    static_assert(BM * 8 % THREADS == 0, "A chunks must divide evenly");
    static_assert(THREADS % BM == 0 && (BM & (BM - 1)) == 0, "threads cover the tile rows evenly");
    static constexpr int ABYTES = BM * QA_PITCH;
    static constexpr int SBYTES = ABYTES + BM * 4;  // one stage buffer: A rows, 1 / SA
    static constexpr int EP_PITCH = 36;              // epilogue floats per row: 32 + 4
    static constexpr int STAGE_BYTES = 3 * SBYTES;
    static constexpr int EPI_BYTES = WVN * 16 * RMB * EP_PITCH * 4;
    static constexpr int LDS_BYTES = STAGE_BYTES > EPI_BYTES ? STAGE_BYTES : EPI_BYTES;
};
typedef WTile<4, 8> WideTile;  // 128 x 512, eight waves of 128 x 64

typedef int i32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i32x16_t mfma_i8_32(const i32x4_t &a, const i32x4_t &b, const i32x16_t &c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

template <class TC, bool BF16, bool GRP = false, bool DUAL = false>
__global__ void __launch_bounds__(TC::THREADS) __attribute__((amdgpu_waves_per_eu(2, 2)))
k_int2_int8_gemm_w(const int8_t *__restrict__ Aq, const uint16_t *__restrict__ SA,
                   const uint32_t *__restrict__ B, const uint16_t *__restrict__ SB, void *__restrict__ C,
                   const uint16_t *__restrict__ Other, const void *__restrict__ Bias, int M, int N, int K,
                   int postop, int out_f32, const int *__restrict__ meta = nullptr, int E = 0, int splits = 1,
                   float *part = nullptr, const int *__restrict__ perm = nullptr, int topk = 1, int arows = 0,
                   const uint32_t *__restrict__ B2 = nullptr, const uint16_t *__restrict__ SB2 = nullptr) {
    static_assert(!DUAL || GRP, "the dual mode is the grouped MoE GEMM's");
    constexpr int RMB = TC::RMB, BM = TC::BM, AP = TC::AP, TH = TC::THREADS;
    static_assert(!DUAL || TC::CB == 2, "dual: the two weight sets as the wave's two column blocks");
    constexpr int NCB = TC::CB;                  // 32-column blocks per wave (DUAL: up, gate)
    constexpr int WCOLS = DUAL ? 32 : 32 * NCB;  // output columns per wave
    constexpr int BN = WCOLS * TC::WVN;
    __shared__ __attribute__((aligned(16))) uint8_t lds[TC::LDS_BYTES];
    int tm, tn, sa_off = 0;
    const bool gat = GRP && perm != nullptr;  // (uniform) A rows gathered through perm
    const int lda = ldsa_of(gat ? arows : M);  // (GRP: of all G rows, or of the arows gathered from)
    [[maybe_unused]] const int *prow = nullptr;  // gat: perm of the segment's rows
    if constexpr (GRP) {
        const int ntn = (N + BN - 1) / BN;
        int tile;
        moe_tile_of(blockIdx.x, ntn, tile, tn);
        const int tiles = meta[2 * E + 1];
        const int e = moe_tile_expert(meta, E, tile, threadIdx.x & 63);
        if (tile >= tiles) return;  // whole workgroup: past the last row tile
        // (wave-uniform values: kept in scalar registers)
        const int row0 = __builtin_amdgcn_readfirstlane(meta[e]);
        tm = __builtin_amdgcn_readfirstlane(tile - meta[E + 1 + e]);
        M = __builtin_amdgcn_readfirstlane(meta[e + 1] - row0);
        if (gat) {
            prow = perm + row0;
        } else {
            Aq += (size_t)row0 * K;
            sa_off = row0;
            SA += row0;
        }
        B += (size_t)e * (K / 16) * N;
        SB += (size_t)e * (K / kGS) * N;
        if constexpr (DUAL) {
            B2 += (size_t)e * (K / 16) * N;
            SB2 += (size_t)e * (K / kGS) * N;
        }
        C = (uint8_t *)C + (size_t)row0 * N * (out_f32 ? 4 : 2);
        if (Other) Other += (size_t)row0 * N;
    }
    // splits > 1 (deterministic split-K, the dense mode): workgroup (tile,
    // slice sl) runs groups [sl gs, (sl + 1) gs) and stores its fp32 tile into
    // part + sl M N with no epilogue; a reduction kernel adds the slices in
    // order.  (slice values kept in scalar registers: the buffer descriptors
    // built from them stay scalar)
    int g0 = 0, groups = K / kGS;
    if constexpr (!GRP) {
        const int mt = (M + BM - 1) / BM, nt = (N + BN - 1) / BN;
        int tns;
        if (!xcd_tile_ashare(blockIdx.x, mt, nt * splits, tm, tns)) return;  // whole workgroup: padding
        tn = __builtin_amdgcn_readfirstlane(tns / splits);
        const int sl = __builtin_amdgcn_readfirstlane(tns - tn * splits);
        groups = __builtin_amdgcn_readfirstlane(groups / splits);
        g0 = sl * groups;
        if (splits > 1) {
            C = part + (size_t)sl * M * N;
            Other = nullptr;
            Bias = nullptr;
            postop = 0;
            out_f32 = 1;
        }
    }
    const int m0 = tm * BM, n0 = tn * BN;
    const int mrows = min(BM, M - m0);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c32 = lane & 31, h = lane >> 5;
    const int wn = WCOLS * wave;

    // A staging: chunk id = tid + THREADS u -> row id >> 3, 16-byte chunk id & 7
    // of the stage's 128 bytes; rows past mrows lie past the buffer's end and
    // load as 0; the stage index is clamped, so every load is in range.
    // (gat: the buffer is all arows rows; rows past mrows re-read the tile's
    // last row, whose outputs are never stored)
    const __amdgpu_buffer_rsrc_t rA = gat ? buf_rsrc(Aq, (uint32_t)((size_t)arows * K))
                                          : buf_rsrc(Aq + (size_t)m0 * K, (uint32_t)((size_t)mrows * K));
    uint32_t va[AP];
#pragma unroll
    for (int u = 0; u < AP; ++u) {
        const int id = tid + TH * u;
        const int r = gat ? prow[m0 + min(id >> 3, mrows - 1)] / topk : id >> 3;
        va[u] = (uint32_t)(r * K + 16 * (id & 7));
    }
    uint4 av[AP];
    auto a_load = [&](int g) __attribute__((always_inline)) {
        const int gc = g0 + (g < groups ? g : groups - 1);
#pragma unroll
        for (int u = 0; u < AP; ++u) {
            const i32x4_t t = __builtin_amdgcn_raw_buffer_load_b128(rA, va[u], gc * kGS, 0);
            av[u] = make_uint4((uint32_t)t[0], (uint32_t)t[1], (uint32_t)t[2], (uint32_t)t[3]);
        }
    };
    // 1 / SA of the tile's rows: threads t, t + BM, ... stage row t % BM (rows
    // past mrows load row mrows - 1, as the last group's row m0 + srow may lie
    // past SA's end and the SGPR offset is not range-checked, and store 0)
    const __amdgpu_buffer_rsrc_t rSA = gat ? buf_rsrc(SA, (uint32_t)((size_t)(K / kGS) * lda * 2))
                                           : buf_rsrc(SA + m0, (uint32_t)(((size_t)(K / kGS) * lda - sa_off - m0) * 2));
    const int srow = tid & (BM - 1);
    const uint32_t vsa = (uint32_t)(gat ? prow[m0 + min(srow, mrows - 1)] / topk : min(srow, mrows - 1)) * 2;
    uint32_t sa_raw = 0;
    auto sa_load = [&](int g) __attribute__((always_inline)) {
        const int gc = g0 + (g < groups ? g : groups - 1);
        sa_raw = __builtin_amdgcn_raw_buffer_load_b16(rSA, vsa, gc * lda * 2, 0);
    };
    auto a_store = [&](int buf) __attribute__((always_inline)) {
        uint8_t *base = lds + buf * TC::SBYTES;
#pragma unroll
        for (int u = 0; u < AP; ++u) {
            const int id = tid + TH * u;
            const uint32_t d[4] = {av[u].x, av[u].y, av[u].z, av[u].w};
            uint32_t o[4];
            transpose4x4(d, o);
            *(uint4 *)(base + (id >> 3) * QA_PITCH + 16 * (id & 7)) = make_uint4(o[0], o[1], o[2], o[3]);
        }
        const float sa = dt2f<BF16>(sa_raw);
        *(float *)(base + TC::ABYTES + 4 * srow) = (srow < mrows && sa != 0.0f) ? 1.0f / sa : 0.0f;
    };

    // B words of this wave: 32-column block cb, k-chunk kc of group g -> word
    // kp = 8 g + 2 kc + h of column n0 + wn + 32 cb + c32.  The offsets advance
    // a group per load, so the loads past the last group (and a block past N
    // in the last word row) return 0; a block past N elsewhere reads the next
    // row's words, in range, feeding outputs that are not stored.
    // (a slice's loads past its last group read the next slice's words, in
    // range, or past the weights' end 0; never used)
    const __amdgpu_buffer_rsrc_t rB = buf_rsrc(B + (size_t)g0 * 8 * N + n0,
                                               (uint32_t)(((size_t)(K / 16 - 8 * g0) * N - n0) * 4));
    const __amdgpu_buffer_rsrc_t rSB = buf_rsrc(SB + (size_t)g0 * N + n0, (uint32_t)(((size_t)(K / kGS - g0) * N - n0) * 2));
    // DUAL: the second column block reads the gate weights at the same columns
    [[maybe_unused]] __amdgpu_buffer_rsrc_t rB2 = rB, rSB2 = rSB;
    if constexpr (DUAL) {
        rB2 = buf_rsrc(B2 + (size_t)g0 * 8 * N + n0, (uint32_t)(((size_t)(K / 16 - 8 * g0) * N - n0) * 4));
        rSB2 = buf_rsrc(SB2 + (size_t)g0 * N + n0, (uint32_t)(((size_t)(K / kGS - g0) * N - n0) * 2));
    }
    uint32_t vb[4];
#pragma unroll
    for (int kc = 0; kc < 4; ++kc) vb[kc] = (uint32_t)(((2 * kc + h) * N + wn + c32) * 4);
    uint32_t vsb = (uint32_t)((wn + c32) * 2);
    uint32_t bw[NCB][4], sraw[NCB];
    auto b_load = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int kc = 0; kc < 4; ++kc)
                bw[cb][kc] = DUAL ? (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(cb ? rB2 : rB, vb[kc], 0, 0)
                                  : (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rB, vb[kc] + 128 * cb, 0, 0);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
            sraw[cb] = DUAL ? __builtin_amdgcn_raw_buffer_load_b16(cb ? rSB2 : rSB, vsb, 0, 0)
                            : __builtin_amdgcn_raw_buffer_load_b16(rSB, vsb + 64 * cb, 0, 0);
#pragma unroll
        for (int kc = 0; kc < 4; ++kc) vb[kc] += (uint32_t)(32 * N);
        vsb += (uint32_t)(2 * N);
    };

    f32x16_t acc[RMB][NCB];
#pragma unroll
    for (int mb = 0; mb < RMB; ++mb)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) acc[mb][cb] = f32x16_t{};

    // Stage g reads buffer g % 3.  B words and scales are loaded one stage
    // ahead, A and SA one and a half: at the middle of stage g every wave
    // stores stage g + 1's A into buffer (g + 1) % 3 and meets the stage's one
    // barrier; that buffer was last read in stage g - 2, before the previous
    // stage's barrier.
    a_load(0);
    sa_load(0);
    b_load();
    a_store(0);
    a_load(1);
    sa_load(1);
    __syncthreads();
    int cur = 0;
    for (int g = 0; g < groups; ++g) {
        const int nxt = cur == 2 ? 0 : cur + 1;
        const uint8_t *abuf = lds + cur * TC::SBYTES;
        i32x4_t bf[NCB][4];
        float sbf[NCB];
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) {
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) bf[cb][kc] = decode_s2(bw[cb][kc]);
            sbf[cb] = dt2f<BF16>(sraw[cb]);
        }
        b_load();
#pragma unroll
        for (int mb = 0; mb < RMB; ++mb) {
            if (mb == RMB / 2) {
                a_store(nxt);  // past the last stage: never read
                __syncthreads();
                a_load(g + 2);
                sa_load(g + 2);
            }
            const int row = 32 * mb + c32;
            i32x4_t af[4];
#pragma unroll
            for (int kc = 0; kc < 4; ++kc) {
                const uint4 v = *(const uint4 *)(abuf + row * QA_PITCH + 16 * (2 * kc + h));
                af[kc] = i32x4_t{(int)v.x, (int)v.y, (int)v.z, (int)v.w};
            }
            // 1 / SA of this lane's rows 32 mb + 8 j + 4 h + i (i = 0..3)
            f32x4_t inv4[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) inv4[j] = *(const f32x4_t *)(abuf + TC::ABYTES + 4 * (32 * mb + 8 * j + 4 * h));
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                i32x16_t dot = mfma_i8_32(af[0], bf[cb][0], i32x16_t{});
#pragma unroll
                for (int kc = 1; kc < 4; ++kc) dot = mfma_i8_32(af[kc], bf[cb][kc], dot);
#pragma unroll
                for (int v = 0; v < 16; ++v) acc[mb][cb][v] += (float)dot[v] * (sbf[cb] * inv4[v >> 2][v & 3]);
            }
        }
        cur = nxt;
    }

    // Epilogue through LDS, one 32-column block and 16-row half of each 32-row
    // block at a time: element e of lane (c32, h) is row 8 (e / 4) + 4 h + e % 4
    // of its 32-row block, column c32; the wave writes its [16 RMB][EP_PITCH]
    // fp32 block and reads back 4 adjacent columns of one row per lane
    // (8 lanes per row of 32 columns) for epi_store4_c.
    constexpr int EP = TC::EP_PITCH;
    float *ct = (float *)lds + (size_t)wave * 16 * RMB * EP;
    // DUAL: h = DT(silu(gate) * DT(up)) in place of the up sums, as a float
    // that DT-rounds back to the same bits, then block 0 goes out with postop 0
    if constexpr (DUAL) {
#pragma unroll
        for (int mb = 0; mb < RMB; ++mb)
#pragma unroll
            for (int v = 0; v < 16; ++v) {
                const float up = dt2f<BF16>(f2dt<BF16>(acc[mb][0][v]));
                acc[mb][0][v] = dt2f<BF16>(f2dt<BF16>(epi_apply_c<1>(acc[mb][1][v], up, 0.0f)));
            }
    }
    __syncthreads();  // the stage buffers are free
    auto epilogue = [&](auto P_, auto F_) __attribute__((always_inline)) {
        constexpr int P = decltype(P_)::value;
        constexpr bool F32 = decltype(F_)::value;
#pragma unroll
        for (int cb = 0; cb < (DUAL ? 1 : NCB); ++cb) {
            const int n = n0 + wn + 32 * cb + 4 * (lane & 7);
#pragma unroll
            for (int hf = 0; hf < 2; ++hf) {
#pragma unroll
                for (int mb = 0; mb < RMB; ++mb)
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        ct[(16 * mb + 8 * (j >> 2) + 4 * h + (j & 3)) * EP + c32] = acc[mb][cb][8 * hf + j];
                __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): this wave's LDS writes done
                __builtin_amdgcn_wave_barrier();
#pragma unroll
                for (int pass = 0; pass < 2 * RMB; ++pass) {
                    const int br = 8 * pass + (lane >> 3);
                    const int r = 32 * (br >> 4) + 16 * hf + (br & 15);
                    const float4 t = *(const float4 *)(ct + br * EP + 4 * (lane & 7));
                    const float v4[4] = {t.x, t.y, t.z, t.w};
                    if (r < mrows && n < N) epi_store4_c<BF16, P, F32, !GRP>(C, Other, Bias, N, m0 + r, n, v4);
                }
                __builtin_amdgcn_wave_barrier();  // reads done before the next block's writes
            }
        }
    };
    if constexpr (DUAL) epilogue(std::integral_constant<int, 0>{}, std::integral_constant<bool, false>{});
    else epi_dispatch(postop, out_f32, epilogue);
}

// Test hook: the MFMA B fragment each word decodes to (4 dwords per word).
__global__ void k_int2_s8_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D, int words) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    const i32x4_t r = decode_s2(B[i]);
    *(uint4 *)(D + (size_t)i * 4) = make_uint4((uint32_t)r[0], (uint32_t)r[1], (uint32_t)r[2], (uint32_t)r[3]);
}

}  // namespace

// nrows non-NULL (the int8 MoE layer): only rows m < *nrows are quantized and
// written (rows past it belong to dropped assignments); perm non-NULL: output
// row m quantizes row perm[m] / topk of A, the gather fused into the
// quantization.
ternocl_status quant_a_run(int dtype, const void *A, void *SA, int8_t *Aq, int M, int K, hipStream_t st,
                           const int *perm, int topk, const int *nrows) {
    const size_t threads = (size_t)M * (K / 16);
    const unsigned blocks = (unsigned)((threads + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_quant_a<true>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)A,
                           (uint16_t *)SA, Aq, M, K, perm, topk, nrows);
    else
        hipLaunchKernelGGL(k_quant_a<false>, dim3(blocks), dim3(256), 0, st, (const uint16_t *)A,
                           (uint16_t *)SA, Aq, M, K, perm, topk, nrows);
    return check_launch();
}

template <class TC, bool QA>
static hipError_t int8_gemm_launch(int dtype, const void *Asrc, const void *SA, const uint32_t *B,
                                   const void *SB, void *C, const void *Other, const void *Bias, int M,
                                   int N, int K, int postop, int out_f32, hipStream_t st) {
    const int mt = (M + TC::BM - 1) / TC::BM, nt = (N + TC::BN - 1) / TC::BN;
    const dim3 grid(xcd_ashare_grid(mt, nt)), block(TC::THREADS);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL((k_int2_int8_gemm<TC, true, QA>), grid, block, 0, st, Asrc, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    else
        hipLaunchKernelGGL((k_int2_int8_gemm<TC, false, QA>), grid, block, 0, st, Asrc, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32);
    return hipGetLastError();
}

// The wide-tile engine (QMODE 0: int8 Aq from quant_a); splits > 1: K slices
// into part (fp32 [splits][M][N]), then the in-order reduction.
template <class TC = WideTile>
static hipError_t int8_gemm_w_launch(int dtype, const int8_t *Aq, const void *SA, const uint32_t *B,
                                     const void *SB, void *C, const void *Other, const void *Bias, int M, int N,
                                     int K, int postop, int out_f32, hipStream_t st, int splits = 1,
                                     float *part = nullptr) {
    const int mt = (M + TC::BM - 1) / TC::BM, nt = (N + TC::BN - 1) / TC::BN;
    const dim3 grid(xcd_ashare_grid(mt, nt * splits)), block(TC::THREADS);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, true>), grid, block, 0, st, Aq, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32,
                           nullptr, 0, splits, part);
    else
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, false>), grid, block, 0, st, Aq, (const uint16_t *)SA, B,
                           (const uint16_t *)SB, C, (const uint16_t *)Other, Bias, M, N, K, postop, out_f32,
                           nullptr, 0, splits, part);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || splits == 1) return e;
    return splitk_reduce_launch(dtype, part, splits, C, Other, Bias, M, N, postop, out_f32, st);
}

// The int8 MoE prefill's grouped GEMM on the expert-sorted rows: Aq [G][K]
// int8 from quant_a, the wide-tile engine; SA [K/128][ldsa(G)].  Grid: an
// upper bound of the row tiles (each expert's ragged tail adds at most one)
// times the column blocks.  Its tiles have the route's 128 rows.
static hipError_t int8_moe_launch(int dtype, const int *meta, const int8_t *Aq, const void *SA,
                                  const uint32_t *B, const void *SB, void *C, const void *Other, int E, int G,
                                  int N, int K, int postop, int out_f32, hipStream_t st, const int *perm, int topk,
                                  int arows) {
    const bool bf = dtype == TERNOCL_BF16;
    const uint16_t *sa = (const uint16_t *)SA, *sb = (const uint16_t *)SB, *oth = (const uint16_t *)Other;
    typedef WideTile TC;
    const int ntn = (N + TC::BN - 1) / TC::BN, max_tiles = moe_grid_tiles(G, TC::BM, E);
    const dim3 grid((unsigned)(max_tiles * ntn)), block(TC::THREADS);
    if (bf)
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, true, true>), grid, block, 0, st, Aq, sa, B, sb, C, oth,
                           nullptr, G, N, K, postop, out_f32, meta, E, 1, nullptr, perm, topk, arows);
    else
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, false, true>), grid, block, 0, st, Aq, sa, B, sb, C, oth,
                           nullptr, G, N, K, postop, out_f32, meta, E, 1, nullptr, perm, topk, arows);
    return hipGetLastError();
}

// perm (optional): the A rows gathered from Aq [arows][K] (row perm[p] / topk
// for sorted row p), SA [K/128][ldsa(arows)].
ternocl_status int8_moe_gemm_run(int dtype, const int *meta, const int8_t *Aq, const void *SA, const uint32_t *B,
                                 const void *SB, void *C, const void *Other, int E, int G, int N, int K, int postop,
                                 int out_f32, hipStream_t st, const int *perm, int topk, int arows) {
    return launch_status(int8_moe_launch(dtype, meta, Aq, SA, B, SB, C, Other, E, G, N, K, postop, out_f32, st,
                                         perm, topk, arows));
}

// The int8 MoE layer's up and gate in one launch (DUAL): Hs = DT(silu(A x Bg)
// * DT(A x Bu)) over the sorted rows, the bits of int8_moe_gemm_run(up,
// postop 0) followed by int8_moe_gemm_run(gate, postop 1, Other = up).
ternocl_status int8_moe_dual_run(int dtype, const int *meta, const int8_t *Aq, const void *SA,
                                 const uint32_t *Bu, const void *Su, const uint32_t *Bg, const void *Sg, void *Hs,
                                 int E, int G, int N, int K, hipStream_t st, const int *perm, int topk, int arows) {
    typedef WideTile TC;
    constexpr int BN = 32 * TC::WVN;
    const int ntn = (N + BN - 1) / BN, max_tiles = moe_grid_tiles(G, TC::BM, E);
    const dim3 grid((unsigned)(max_tiles * ntn)), block(TC::THREADS);
    const uint16_t *sa = (const uint16_t *)SA, *su = (const uint16_t *)Su, *sg = (const uint16_t *)Sg;
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, true, true, true>), grid, block, 0, st, Aq, sa, Bu, su, Hs,
                           nullptr, nullptr, G, N, K, 0, 0, meta, E, 1, nullptr, perm, topk, arows, Bg, sg);
    else
        hipLaunchKernelGGL((k_int2_int8_gemm_w<TC, false, true, true>), grid, block, 0, st, Aq, sa, Bu, su, Hs,
                           nullptr, nullptr, G, N, K, 0, 0, meta, E, 1, nullptr, perm, topk, arows, Bg, sg);
    return launch_status(hipGetLastError());
}

int int8_moe_tile_rows() { return WideTile::BM; }

// Tile planner: the 128 x 512 wide tile whenever it yields at least 192 tiles
// (three quarters of the 256 CUs, one workgroup each); else the 128 x 256
// tile of the same engine (eight waves of 128 x 32) where 128 x 128 tiles
// would number more than 256 and 128 x 256 tiles fit one per CU; else 128 x
// 128 tiles (2 x 2 waves of 64 x 64, two workgroups per CU; 2 x 4 waves of
// 64 x 32 where they number at most 256), which fill the chip at a quarter of
// the wide tile's width (at M = 1024, K = 14336, N = 4096: 64 wide tiles, 252 us,
// against 147 us on 256 narrow ones).  QMODE 1 (DT A quantized while staged)
// always runs the 2 x 2-wave 128 x 128 engine.
ternocl_status int2_int8_gemm_run(int dtype, const void *A, const int8_t *Aq, const void *SA,
                                  const uint32_t *B, const void *SB, void *C, const void *Other,
                                  const void *Bias, int M, int N, int K, int postop, int out_f32,
                                  hipStream_t st, void *ws, size_t ws_bytes) {
    typedef QTile<4, 4, 2, 2> Tile;
    const size_t es = Aq ? 1 : 2;
    if ((size_t)M * K * es >= (1u << 31) || (size_t)(K / 16) * N * 4 >= (1u << 31)) {
        set_error("int2_int8_gemm: the A operand and B must each be below 2^31 bytes");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    // 128 x 256 tiles of eight 128 x 32 waves where 128 x 128 tiles would
    // number more than 256 and 128 x 256 tiles fit one per CU (the fp16
    // prefill GEMM's rule): they decode each weight word for 128 rows, the
    // 128 x 128 engine for 64.  Same box, quant_a'd fp16 A, against that
    // engine / the split (two runs each, us): M = 1024 K = 4096 N = 6144
    // 69.3 / 67.8 -> 54.4, M = 1024 K = 6144 N = 5120 96.3 -> 76.7, M = 512
    // K = 4096 N = 14336 72.6 / 70.4 -> 58.5, M = 2048 K = N = 4096 73.2 /
    // 75.9 -> 58.0-62.0, M = 1000 K = 2048 N = 6160 41.3 -> 31.6; at 160 and
    // 136 tiles too, against the split: M = 1024 K = 17408 N = 5120 207.2 /
    // 202.6 -> 198.7 / 199.4, M = 1000 K = 8192 N = 4112 113.8 / 112.9 ->
    // 96.9 / 96.6.  Elsewhere the wide tile over K slices where its tiles
    // alone leave CUs idle and the caller gives the partials' workspace (the
    // fp16 prefill GEMM's rule).
    const bool half = Aq && gemm_half_tile(M, N);
    const int splits = Aq && !half ? gemm_splits(M, N, K) : 1;
    if (splits > 1 && ws && ((uintptr_t)ws & 15) == 0 && ws_bytes >= kWsHeader + (size_t)splits * M * N * 4)
        return launch_status(int8_gemm_w_launch(dtype, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st,
                                                splits, (float *)((uint8_t *)ws + kWsHeader)));
    const bool wide = Aq && (size_t)((M + WideTile::BM - 1) / WideTile::BM) * ((N + WideTile::BN - 1) / WideTile::BN) >= 192;
    // 128 x 128 tiles numbering at most 256 (one workgroup per CU) as eight
    // waves of 64 x 32, two per SIMD: M = 1024 K = N = 4096 51.7 -> 46.3 us,
    // M = 512 47.2 -> 41.3 us (quant_a included)
    const bool one_round = (size_t)((M + 127) / 128) * ((N + 127) / 128) <= 256;
    const hipError_t e =
        wide  ? int8_gemm_w_launch(dtype, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
        : half ? int8_gemm_w_launch<WTile<4, 8, 1>>(dtype, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
        : (Aq && one_round)
              ? int8_gemm_launch<QTile<4, 2, 2, 4>, false>(dtype, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop,
                                                           out_f32, st)
        : Aq  ? int8_gemm_launch<Tile, false>(dtype, Aq, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st)
              : int8_gemm_launch<Tile, true>(dtype, A, SA, B, SB, C, Other, Bias, M, N, K, postop, out_f32, st);
    return launch_status(e);
}

ternocl_status int2_s8_decode_run(const uint32_t *B, uint32_t *D, int K, int N, hipStream_t st) {
    const int words = K / 16 * N;
    hipLaunchKernelGGL(k_int2_s8_decode, dim3((words + 255) / 256), dim3(256), 0, st, B, D, words);
    return check_launch();
}

}  // namespace tcl
