// int2_gemv_mfma.hip -- decode GEMV (M <= 16) for packed 2-bit ternary weights
// on gfx950, matrix-core edition: the default engine replacing
// int2_fp16_upcvt_gemm (int2_fp16_upcvt/int2_fp16_upcvt.cl:193-290).
//
//   C[m,n] = ct(epi(sum_g S[g,n] * sum_{k in g} A[m,k] * code(B[k,n])))
//
// Why MFMA in a bandwidth-bound GEMV: at decode sizes (5-30 MB per call) the
// whole weight stream arrives within ~2-4 us, and the VALU has to finish the
// unpack *and* the MACs in that window.  With v_dot2 MACs fed by LDS-staged
// activations the kernel measured 2x the streaming-read time of the same bytes;
// here the VALU only unpacks (10-12 ops per 16 weights) and
// v_mfma_f32_16x16x32_{f16,bf16} does the MACs, so the kernel runs at the
// streaming-read time.  Rows 1..15 of the 16-row MFMA tile are free, so M up
// to 16 costs the same as M = 1.
//
// Layout (lane l of a wave, c = l % 16, q = l / 16):
//   * a workgroup owns a strip of 16*CPL adjacent columns over all of K (no
//     inter-workgroup communication, hence no fences or atomics);
//   * lane (c, q) loads CPL adjacent words (columns 16*strip*CPL + CPL*c + j)
//     of kp rows 8g + q and 8g + 4 + q for each 128-row group g: a wave reads
//     4 rows x 64*CPL contiguous bytes per load;
//   * MFMA operand B of "column set" j, half h of a word: the 4 dwords the
//     mantissa-field decode builds from pairs (rows 4h+i, 4h+i+8), i = 0..3;
//     operand A: the matching activation pairs, pre-scaled by 2^-p_i and staged
//     by each wave for its own groups in LDS (one ds_read_b128 serves all CPL
//     column sets; no workgroup barrier before the MACs);
//   * the per-group correction beta = BASE * sum a' + 2 * sum a is summed while
//     staging (a 16-lane reduction) and seeds the group's accumulators, so the
//     MAC chains have no extra dependency and the scale costs one FMA per output;
//   * waves split K into contiguous group ranges and reduce through LDS in
//     wave order: deterministic bit for bit;
//   * the epilogue's residual and bias are loaded at kernel start.
#include "common.hpp"
#include "int2_decode.hpp"

#include <climits>

namespace tcl {
namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf168_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

// field shift of dword i (pairs (4h+i, 4h+i+8)) of a B fragment
__host__ __device__ constexpr int mf_shift(bool bf16, int i) { return bf16 ? (i < 3 ? 2 * i : 5) : 2 * i; }

// v_and_or_b32 with mask in an SGPR and base in a VGPR (see int2_decode.hpp)
__device__ __forceinline__ uint32_t mfld(uint32_t t, int p, uint32_t base2) {
    return and_or(t, (3u << p) | (3u << (p + 16)), base2);
}

// Decode one B word (after the xor) into the two 4-dword B fragments.
template <bool BF16>
__device__ __forceinline__ void mf_decode(uint32_t w, uint32_t b0[4], uint32_t b1[4], uint32_t B2) {
    const uint32_t t = w ^ 0xAAAAAAAAu;
    const uint32_t t8 = t >> 8;
    if constexpr (!BF16) {
        b0[0] = mfld(t, 0, B2); b0[1] = mfld(t, 2, B2); b0[2] = mfld(t, 4, B2); b0[3] = mfld(t, 6, B2);
        b1[0] = mfld(t8, 0, B2); b1[1] = mfld(t8, 2, B2); b1[2] = mfld(t8, 4, B2); b1[3] = mfld(t8, 6, B2);
    } else {
        // bf16 keeps 7 mantissa bits: the field of row 3 (bits 6-7) moves to bits 5-6
        b0[0] = mfld(t, 0, B2); b0[1] = mfld(t, 2, B2); b0[2] = mfld(t, 4, B2); b0[3] = mfld(t >> 1, 5, B2);
        b1[0] = mfld(t8, 0, B2); b1[1] = mfld(t8, 2, B2); b1[2] = mfld(t8, 4, B2); b1[3] = mfld(t >> 9, 5, B2);
    }
}

template <bool BF16>
__device__ __forceinline__ f32x4_t mfma(const uint32_t a[4], const uint32_t b[4], f32x4_t c) {
    if constexpr (BF16) {
        bf168_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(x, y, c, 0, 0, 0);
    } else {
        half8_t x, y;
        __builtin_memcpy(&x, a, 16);
        __builtin_memcpy(&y, b, 16);
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(x, y, c, 0, 0, 0);
    }
}

// Per-wave LDS staging of the wave's GPW groups of one window: for row m < MR,
// group gl (0..GPW-1) and kp row r (0..7) of the group, the 8 pairs (h, i) =
// (a[16kp+4h+i], a[16kp+4h+i+8]) * 2^-p_i, as 64 dwords + 4 of padding per
// (m, gl).  A wave stages exactly the groups it consumes, so no workgroup
// barrier stands between a wave's own loads and its MACs (LDS operations of
// one wave execute in order).  Staging is split in two so that a window's
// activation loads can be issued before the weight loads of the same window:
// s_waitcnt vmcnt counts loads in issue order, so consuming activations issued
// first does not wait for weights.  A lane stages QPT "quads" (4 pairs: one
// (m, gl, r, h)), QPT = MR*GPW/4 rounded up; quad index = lane + 64 u.
constexpr int kMfGroupStride = 68;

template <int MR, int GPW> struct Stage {
    static constexpr int QPT = (MR * GPW + 3) / 4;
    static constexpr int TOTAL = MR * GPW * 16;  // quads per wave
    uint2 lo[QPT], hi[QPT];
    // Issue the activation loads of groups [g0, g0 + GPW).  Loads are
    // unconditional (indices clamped in range, out-of-range quads zeroed at
    // store time): a load under a branch makes the compiler wait for it at the
    // branch's end, which would serialise the memory latencies.
    bool ok[QPT];
    __device__ __forceinline__ void load(const uint16_t *__restrict__ A, int M, int K, int groups,
                                         int g0, int lane) {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int idx = lane + u * 64;
            const int mg = idx >> 4, r = (idx >> 1) & 7, h = idx & 1;
            const int m = mg / GPW, gl = mg % GPW;
            const int g = g0 + gl;
            ok[u] = idx < TOTAL && m < M && g < groups;
            const int mc = m < M ? m : M - 1, gc = g < groups ? g : groups - 1;
            const uint16_t *p = A + (size_t)mc * K + (size_t)gc * kGS + r * 16 + 4 * h;
            lo[u] = *(const uint2 *)p;        // a[k .. k+3]
            hi[u] = *(const uint2 *)(p + 8);  // a[k+8 .. k+11]
        }
    }
    // Convert (scale pair i by 2^-p_i) and write the groups into buf; also
    // beta[m][gl] = BASE * sum a' + 2 * sum a over the group's 128 activations
    // (the group's 16 quads are 16 consecutive lanes: a 16-lane reduction),
    // stored at beta_base[gl * 16 + row] for every row = m (mod MR) so a lane
    // reads the 4 rows it accumulates with one ds_read_b128.
    template <bool BF16>
    __device__ __forceinline__ void store(uint32_t *buf, float *beta_base, int lane) const {
#pragma unroll
        for (int u = 0; u < QPT; ++u) {
            const int idx = lane + u * 64;
            const int mg = idx >> 4, r = (idx >> 1) & 7, h = idx & 1;
            const bool live = idx < TOTAL && ok[u];
            const uint2 l = live ? lo[u] : make_uint2(0, 0), hh = live ? hi[u] : make_uint2(0, 0);
            const uint32_t a[4] = {l.x & 0xffffu, l.x >> 16, l.y & 0xffffu, l.y >> 16};
            const uint32_t b[4] = {hh.x & 0xffffu, hh.x >> 16, hh.y & 0xffffu, hh.y >> 16};
            uint32_t v[4];
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float sc = 1.0f / (float)(1 << mf_shift(BF16, i));
                const float fa = dt2f<BF16>(a[i]), fb = dt2f<BF16>(b[i]);
                const uint32_t pa = f2dt<BF16>(fa * sc), pb = f2dt<BF16>(fb * sc);
                v[i] = pa | (pb << 16);
                part += gemv_base(BF16) * (dt2f<BF16>(pa) + dt2f<BF16>(pb)) + 2.0f * (fa + fb);
            }
            if (idx < TOTAL)
                *(uint4 *)(buf + (size_t)mg * kMfGroupStride + r * 8 + 4 * h) = make_uint4(v[0], v[1], v[2], v[3]);
#pragma unroll
            for (int o = 8; o >= 1; o >>= 1) part += __shfl_xor(part, o, 16);
            if ((idx & 15) == 0 && idx < TOTAL) {
                const int m = mg / GPW, gl = mg % GPW;
#pragma unroll
                for (int rep = 0; rep < 16 / MR; ++rep) beta_base[gl * 16 + m + rep * MR] = part;
            }
        }
    }
};

// a wave's window buffer: the pairs, then beta [gw][16] floats (gw = GPW)
__host__ __device__ inline size_t mf_pairs_dwords(int MR, int gw) {
    return ((size_t)MR * gw * kMfGroupStride + 3) & ~(size_t)3;
}
__host__ __device__ inline size_t mf_window_dwords(int MR, int gw) {
    return mf_pairs_dwords(MR, gw) + (size_t)gw * 16;
}

template <int CPL> struct Words;
template <> struct Words<1> {
    uint32_t v[1];
    __device__ void load(const uint32_t *p) { v[0] = *p; }
};
template <> struct Words<2> {
    uint32_t v[2];
    __device__ void load(const uint32_t *p) {
        const uint2 t = *(const uint2 *)p;
        v[0] = t.x; v[1] = t.y;
    }
};
template <> struct Words<4> {
    uint32_t v[4];
    __device__ void load(const uint32_t *p) {
        const uint4 t = *(const uint4 *)p;
        v[0] = t.x; v[1] = t.y; v[2] = t.z; v[3] = t.w;
    }
};

// This wave's weight words and raw scale bits of one window.  Loads are
// unconditional (group index clamped; groups past K are never consumed), and
// the scale halves are split only where they are used.
template <int CPL, int GPW> struct Slab {
    Words<CPL> w[GPW][2];
    uint32_t sc[GPW][(CPL + 1) / 2];  // CPL DT scales, packed in pairs
    __device__ __forceinline__ void load(const uint32_t *__restrict__ B, const uint16_t *__restrict__ S,
                                         int N, int groups, int g0w, int q, int n0) {
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = g0w + gi < groups ? g0w + gi : groups - 1;
#pragma unroll
            for (int t = 0; t < 2; ++t) w[gi][t].load(B + ((size_t)g * 8 + 4 * t + q) * N + n0);
            if constexpr (CPL == 4) {
                const uint2 t = *(const uint2 *)(S + (size_t)g * N + n0);
                sc[gi][0] = t.x;
                sc[gi][1] = t.y;
            } else if constexpr (CPL == 2) {
                sc[gi][0] = *(const uint32_t *)(S + (size_t)g * N + n0);
            } else {
                sc[gi][0] = S[(size_t)g * N + n0];
            }
        }
    }
    __device__ __forceinline__ uint32_t scale(int gi, int j) const {
        return CPL == 1 ? sc[gi][0] : ((j & 1) ? sc[gi][j >> 1] >> 16 : sc[gi][j >> 1] & 0xffffu);
    }
};

// Epilogue operands of the outputs a lane stores (rows 4q + i, i < min(4, MR),
// columns n0 + j), loaded at kernel start so the epilogue does not pay a memory
// latency after the last MAC.  The loads are unconditional -- a load under a
// branch is waited for at the branch's end -- so an operand the post-op does
// not use is read from element 0 of `dummy` (any valid array) and ignored.
template <int MR, int CPL, bool BF16> struct EpiIn {
    static constexpr int ROWS = MR < 4 ? MR : 4;
    float o[ROWS][CPL], b[CPL];
    __device__ __forceinline__ void load(const uint16_t *__restrict__ Other, const void *__restrict__ Bias,
                                         const uint16_t *__restrict__ dummy, int postop, int out_f32,
                                         int M, int N, int q, int n0) {
        const bool uo = postop_needs_other(postop);
        const bool b32 = postop_needs_bias(postop) && out_f32, b16 = postop_needs_bias(postop) && !out_f32;
        const uint16_t *op = uo ? Other : dummy;
        const float *bp32 = b32 ? (const float *)Bias : (const float *)dummy;
        const uint16_t *bp16 = b16 ? (const uint16_t *)Bias : dummy;
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int m = 4 * q + i < M ? 4 * q + i : M - 1;
#pragma unroll
            for (int j = 0; j < CPL; ++j) o[i][j] = dt2f<BF16>(op[uo ? (size_t)m * N + n0 + j : 0]);
        }
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const float f = bp32[b32 ? n0 + j : 0];
            const float h = dt2f<BF16>(bp16[b16 ? n0 + j : 0]);
            b[j] = out_f32 ? f : h;
        }
    }
};

// Workgroup barrier between a window's activation loads and its weight loads:
// every wave's activation requests enter the CU's memory pipeline ahead of any
// weight request, so they return at cache latency instead of queuing behind the
// weight stream.  There is no data wait (s_barrier alone); the weight and scale
// base pointers pass through an asm after it, so their loads stay below it.
__device__ __forceinline__ int loads_after_barrier() {
    __builtin_amdgcn_s_barrier();
    int zero = 0;
    asm volatile("" : "+s"(zero));
    return zero;
}

// MR: staged activation rows (power of two >= M), CPL: words (columns) per
// lane, GPW: groups per wave per window.  W = blockDim.x / 64 waves; a window
// is W * GPW groups, wave w taking groups [w * GPW, (w + 1) * GPW) of it.
__host__ __device__ constexpr int mf_max_waves(int) { return 8; }  // 16-wave workgroups measured slower

template <int MR, int CPL, int GPW, bool BF16>
__global__ void __launch_bounds__(64 * mf_max_waves(MR))
k_int2_gemv_mfma(const uint16_t *__restrict__ A, const uint32_t *__restrict__ B,
                 const uint16_t *__restrict__ S, void *__restrict__ C,
                 const uint16_t *__restrict__ Other, const void *__restrict__ Bias, int M, int N,
                 int K, int postop, int out_f32, int swz) {
    extern __shared__ uint32_t lds[];
    const int W = blockDim.x >> 6;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int c = lane & 15, q = lane >> 4;
    const int groups = K / kGS;
    const int gw = W * GPW;                       // groups per window
    const int windows = (groups + gw - 1) / gw;
    int strip = blockIdx.x;
    if (swz) {  // strips 2j, 2j+1 (sharing 128-byte lines) on the same XCD
        const int qq = blockIdx.x >> 3, x = blockIdx.x & 7;
        strip = (((qq >> 1) << 3) + x) * 2 + (qq & 1);
    }
    const int n0 = strip * 16 * CPL + CPL * c;    // this lane's first column
    const size_t wd = mf_window_dwords(MR, GPW);
    const int nbuf = windows > 1 ? 2 : 1;
    uint32_t *wlds = lds + (size_t)wave * nbuf * wd;  // this wave's staging buffers
    const int mrow = (c & (MR - 1));              // A row this lane feeds (rows >= M are don't-care)

    uint32_t B2 = gemv_base2(BF16);
    asm volatile("" : "+v"(B2));

    EpiIn<MR, CPL, BF16> ein;
    ein.load(Other, Bias, S, postop, out_f32, M, N, q, n0);

    // window 0: activations first, then weights, then the activation staging
    Stage<MR, GPW> st;
    st.load(A, M, K, groups, wave * GPW, lane);
    int after = loads_after_barrier();  // 0, known only after the barrier
    Slab<CPL, GPW> cur;
    cur.load(B + after, S + after, N, groups, wave * GPW, q, n0);
    st.template store<BF16>(wlds, (float *)(wlds + mf_pairs_dwords(MR, GPW)), lane);

    f32x4_t acc[CPL];
#pragma unroll
    for (int j = 0; j < CPL; ++j) acc[j] = f32x4_t{0.f, 0.f, 0.f, 0.f};

    for (int win = 0; win < windows; ++win) {
        // this wave's staging writes precede its reads (in-order LDS); the
        // asm keeps the compiler from reordering them
        asm volatile("" ::: "memory");
        const uint32_t *buf = wlds + (size_t)(win & 1) * wd;
        const bool more = win + 1 < windows;
        Slab<CPL, GPW> nxt;
        if (more) {  // next window in flight while this one computes
            st.load(A, M, K, groups, (win + 1) * gw + wave * GPW, lane);
            after = loads_after_barrier();
            nxt.load(B + after, S + after, N, groups, (win + 1) * gw + wave * GPW, q, n0);
        }
#pragma unroll
        for (int gi = 0; gi < GPW; ++gi) {
            const int g = win * gw + wave * GPW + gi;
            if (g >= groups) break;  // uniform across the wave
            // A fragments (t, h): pairs of kp row 4t + q of this group, row mrow
            uint32_t af[2][2][4];
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int h = 0; h < 2; ++h) {
                    const uint4 v = *(const uint4 *)(buf + ((size_t)mrow * GPW + gi) * kMfGroupStride +
                                                     (4 * t + q) * 8 + 4 * h);
                    af[t][h][0] = v.x; af[t][h][1] = v.y; af[t][h][2] = v.z; af[t][h][3] = v.w;
                }
            // -beta of rows 4q..4q+3 seeds each column set's accumulator
            const f32x4_t beta = -*(const f32x4_t *)((const float *)(buf + mf_pairs_dwords(MR, GPW)) + gi * 16 + 4 * q);
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                f32x4_t d = beta;
#pragma unroll
                for (int t = 0; t < 2; ++t) {
                    uint32_t b0[4], b1[4];
                    mf_decode<BF16>(cur.w[gi][t].v[j], b0, b1, B2);
                    d = mfma<BF16>(af[t][0], b0, d);
                    d = mfma<BF16>(af[t][1], b1, d);
                }
                const float s = dt2f<BF16>(cur.scale(gi, j));
                acc[j] = d * s + acc[j];
            }
        }
        if (more) {
            asm volatile("" ::: "memory");
            uint32_t *nb = wlds + (size_t)((win + 1) & 1) * wd;
            st.template store<BF16>(nb, (float *)(nb + mf_pairs_dwords(MR, GPW)), lane);
            cur = nxt;
        }
    }

    // ---- reduction over waves (wave order), then epilogue -------------------
    // Lane (c, q) holds rows 4q + i (i < 4) of columns n0 + j; only lanes
    // q < QV hold rows < MR, so only their ROWS live values travel through LDS
    // (its own region past the staging buffers: one barrier).
    constexpr int ROWS = EpiIn<MR, CPL, BF16>::ROWS, QV = (MR + 3) / 4;
    const bool live = q < QV;
    if (W > 1) {
        float *red = (float *)(lds + (size_t)nbuf * W * wd);  // [W-1][CPL][QV*16][ROWS]
        constexpr int JS = QV * 16 * ROWS;
        if (wave != 0 && live) {
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int i = 0; i < ROWS; ++i)
                    red[((wave - 1) * CPL + j) * JS + (q * 16 + c) * ROWS + i] = acc[j][i];
        }
        __syncthreads();
        if (wave != 0 || !live) return;
        for (int w2 = 1; w2 < W; ++w2)
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int i = 0; i < ROWS; ++i)
                    acc[j][i] += red[((w2 - 1) * CPL + j) * JS + (q * 16 + c) * ROWS + i];
    }
    if (!live) return;
    epi_dispatch(postop, out_f32, [&](auto P_, auto F_) __attribute__((always_inline)) {
        constexpr int PO = decltype(P_)::value;
        constexpr bool F32 = decltype(F_)::value;
#pragma unroll
        for (int i = 0; i < ROWS; ++i) {
            const int m = 4 * q + i;
            if (m >= M) break;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const float r = epi_apply_c<PO>(acc[j][i], ein.o[i][j], ein.b[j]);
                const size_t oi = (size_t)m * N + n0 + j;
                if constexpr (F32) ((float *)C)[oi] = r;
                else ((uint16_t *)C)[oi] = (uint16_t)f2dt<BF16>(r);
            }
        }
    });
}

struct MfPlan {
    int cpl, waves, gpw, mr;
    size_t lds;
};

constexpr size_t kMfMaxLds = 64 * 1024;

int mf_mr(int M) { return M <= 1 ? 1 : M <= 2 ? 2 : M <= 4 ? 4 : M <= 8 ? 8 : 16; }

size_t mf_lds(int MR, int waves, int gpw, int cpl, int groups) {
    const int gw = waves * gpw;
    const int windows = (groups + gw - 1) / gw;
    const size_t stage = (size_t)(windows > 1 ? 2 : 1) * waves * mf_window_dwords(MR, gpw) * 4;
    const int rows = MR < 4 ? MR : 4, qv = (MR + 3) / 4;
    return stage + (size_t)(waves - 1) * cpl * qv * 16 * rows * 4;
}

// Automatic tile: 2 words per lane (32-column strips) when that still gives
// >= 384 workgroups, else 1 (16-column strips); then waves x groups-per-wave
// covering K in as few windows as the LDS budget allows, preferring more waves.
MfPlan mf_plan(int M, int N, int K, int waves, int cpl, int gpw) {
    const int MR = mf_mr(M), groups = K / kGS;
    MfPlan p;
    p.mr = MR;
    p.cpl = cpl > 0 ? cpl : ((N % 32 == 0 && N / 32 >= 384) ? 2 : 1);
    int bw = 8, bg = 1;
    if (waves > 0 && gpw > 0) {
        bw = waves; bg = gpw;
    } else {
        long best = LONG_MIN;
        for (int g : {1, 2, 4, 8, 16}) {
            if (gpw > 0 ? g != gpw : g > 4) continue;  // automatic: <= 4 groups per wave (measured best)
            if (MR * g > 16) continue;     // staging registers: MR * GPW / 4 quads per thread
            if (p.cpl * g > 16) continue;  // weight registers: 2 * CPL * GPW words per lane
            for (int w = 1; w <= 8; ++w) {
                if (waves > 0 && w != waves) continue;
                if (mf_lds(MR, w, g, p.cpl, groups) > kMfMaxLds) continue;
                const int gw = w * g, windows = (groups + gw - 1) / gw;
                const int idle = windows * gw - groups;
                // fewest idle group slots, then fewest windows, then more waves
                const long score = -(long)idle * 100000 - (long)windows * 100 + w;
                if (score > best) { best = score; bw = w; bg = g; }
            }
        }
    }
    p.waves = bw;
    p.gpw = bg;
    p.lds = mf_lds(MR, bw, bg, p.cpl, groups);
    return p;
}

template <int MR, int CPL, int GPW, bool BF16>
hipError_t mf_launch_t(const MfPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    const int strips = N / (16 * CPL);
    const int swz = (CPL == 1 && strips % 16 == 0) ? 1 : 0;
    hipLaunchKernelGGL((k_int2_gemv_mfma<MR, CPL, GPW, BF16>), dim3(strips), dim3(64 * p.waves), p.lds,
                       st, (const uint16_t *)A, B, (const uint16_t *)S, C, (const uint16_t *)Other,
                       Bias, M, N, K, postop, out_f32, swz);
    return hipGetLastError();
}

template <int MR, int CPL, bool BF16>
hipError_t mf_launch_g(const MfPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    switch (p.gpw) {
    case 1: return mf_launch_t<MR, CPL, 1, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return mf_launch_t<MR, CPL, 2, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 4: return mf_launch_t<MR, CPL, 4, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 8:
        if constexpr (MR <= 2 && CPL <= 2) return mf_launch_t<MR, CPL, 8, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        return hipErrorInvalidValue;
    default:
        if constexpr (MR == 1 && CPL == 1) return mf_launch_t<MR, CPL, 16, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
        return hipErrorInvalidValue;
    }
}

template <int MR, bool BF16>
hipError_t mf_launch_c(const MfPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                       const void *Other, const void *Bias, int M, int N, int K, int postop,
                       int out_f32, hipStream_t st) {
    if (p.cpl == 4) return mf_launch_g<MR, 4, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    if (p.cpl == 2) return mf_launch_g<MR, 2, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return mf_launch_g<MR, 1, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
}

template <bool BF16>
hipError_t mf_launch(const MfPlan &p, const void *A, const uint32_t *B, const void *S, void *C,
                     const void *Other, const void *Bias, int M, int N, int K, int postop,
                     int out_f32, hipStream_t st) {
    switch (p.mr) {
    case 1: return mf_launch_c<1, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 2: return mf_launch_c<2, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 4: return mf_launch_c<4, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    case 8: return mf_launch_c<8, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    default: return mf_launch_c<16, BF16>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    }
}

// Decode hook: the B fragments of each word as the kernel builds them,
// D[word][0..3] = half 0, D[word][4..7] = half 1.
template <bool BF16>
__global__ void k_int2_mfma_decode(const uint32_t *__restrict__ B, uint32_t *__restrict__ D,
                                   size_t words) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= words) return;
    uint32_t B2 = gemv_base2(BF16);
    asm volatile("" : "+v"(B2));
    uint32_t b0[4], b1[4];
    mf_decode<BF16>(B[i], b0, b1, B2);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        D[i * 8 + j] = b0[j];
        D[i * 8 + 4 + j] = b1[j];
    }
}

}  // namespace

ternocl_status int2_gemv_mfma_run(int dtype, const void *A, const uint32_t *B, const void *S, void *C,
                                  const void *Other, const void *Bias, int M, int N, int K,
                                  int postop, int out_f32, int waves, int cpl, int gpw,
                                  hipStream_t st) {
    if (cpl != 0 && cpl != 1 && cpl != 2 && cpl != 4) {
        set_error("cols_per_lane must be 0 (automatic), 1, 2 or 4");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (gpw != 0 && gpw != 1 && gpw != 2 && gpw != 4 && gpw != 8 && gpw != 16) {
        set_error("groups_per_wave must be 0 (automatic), 1, 2, 4, 8 or 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (gpw * mf_mr(M) > 16 || gpw * (cpl ? cpl : 1) > 16) {
        set_error("groups_per_wave * (M rounded up to a power of two) and groups_per_wave * "
                  "cols_per_lane must be <= 16");
        return TERNOCL_ERR_INVALID_ARG;
    }
    if (waves < 0 || waves > mf_max_waves(mf_mr(M))) {
        set_error("waves must be 0 (automatic) .. 8");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const MfPlan p = mf_plan(M, N, K, waves, cpl, gpw);
    if (N % (16 * p.cpl)) {
        set_error("N must be a multiple of 16 * cols_per_lane");
        return TERNOCL_ERR_UNSUPPORTED_SHAPE;
    }
    if (p.lds > kMfMaxLds) {
        set_error("GEMV tile needs more than 64 KiB of LDS: use fewer waves or groups per wave");
        return TERNOCL_ERR_INVALID_ARG;
    }
    const hipError_t e = dtype == TERNOCL_BF16
        ? mf_launch<true>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st)
        : mf_launch<false>(p, A, B, S, C, Other, Bias, M, N, K, postop, out_f32, st);
    return launch_status(e);
}

ternocl_status int2_mfma_decode_run(int dtype, const uint32_t *B, uint32_t *D, int K, int N,
                                    hipStream_t st) {
    const size_t words = (size_t)(K / 16) * N;
    const unsigned blocks = (unsigned)((words + 255) / 256);
    if (dtype == TERNOCL_BF16)
        hipLaunchKernelGGL(k_int2_mfma_decode<true>, dim3(blocks), dim3(256), 0, st, B, D, words);
    else
        hipLaunchKernelGGL(k_int2_mfma_decode<false>, dim3(blocks), dim3(256), 0, st, B, D, words);
    return check_launch();
}

}  // namespace tcl
