// common.hpp -- device helpers shared by the gfx950 kernels: DT (fp16 / bf16)
// conversions, the fused epilogue and host-side launch plumbing.
#pragma once

#include <hip/hip_runtime.h>
#include <type_traits>
#include <stddef.h>
#include <stdint.h>

#include "../../include/ternocl_amd.h"

namespace tcl {

constexpr int kGS = 128;  // scale group size (K rows per scale)
// Front of every caller workspace: the cross-workgroup counters of the K
// splits (zero between calls); partials and buffers start after it.
constexpr size_t kWsHeader = TERNOCL_WS_HEADER_BYTES;

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf162_t __attribute__((ext_vector_type(2)));

// ---- DT conversions (round to nearest even), as common/dt16.hpp:18-42 ----

template <bool BF16>
__device__ __forceinline__ float dt2f(uint32_t h) {
    if constexpr (BF16) {
        return __uint_as_float(h << 16);
    } else {
        const uint16_t b = (uint16_t)h;
        _Float16 x;
        __builtin_memcpy(&x, &b, 2);
        return (float)x;
    }
}

template <bool BF16>
__device__ __forceinline__ uint32_t f2dt(float f) {
    if constexpr (BF16) {
        // v_cvt_pk_bf16_f32 (round to nearest even; a NaN keeps its sign and
        // upper payload bits and gets the quiet bit): the bits of the
        // reference's fromf (common/dt16.hpp:30-36), (u + 0x7fff + lsb) >> 16
        // and (u >> 16) | 0x40 for a NaN, in one instruction per two values
        // instead of five per value
        asm volatile("" : "+v"(f));
        const __bf16 x = (__bf16)f;
        uint16_t b;
        __builtin_memcpy(&b, &x, 2);
        return b;
    } else {
        // Materialise the fp32 value first: otherwise a product feeding the
        // conversion fuses into v_fma_mixlo_f16, which rounds once straight to
        // fp16 instead of fp32 then fp16 as the reference's DT stores do.
        asm volatile("" : "+v"(f));
        const _Float16 x = (_Float16)f;  // v_cvt_f16_f32, RTE
        uint16_t b;
        __builtin_memcpy(&b, &x, 2);
        return b;
    }
}

// Workgroup -> (row tile, column tile) of a grouped GEMM launch with ntn
// column tiles per row tile and a multiple of 8 row tiles (moe_grid_tiles):
// workgroups are dealt to the 8 XCDs round-robin, and XCD x takes row tiles
// x, x + 8, ... with all their column tiles in turn, so a row tile's gathered
// A rows are fetched into one XCD's L2 (row tile after row tile would spread
// its column tiles over the XCDs).  C5, same box: the bf16 layer's GEMMs fetch
// 38-42% fewer bytes from memory (FETCH_SIZE, gate/up 501 -> 313 MB, down
// 285 -> 166 MB); the layer's time moved by 1% at most (389.8 / 388.6 /
// 390.7 -> 380.9 / 384.8 / 386.4 us alternating), so the fetches are not what
// bounds it.
__device__ __forceinline__ void moe_tile_of(int id, int ntn, int &tile, int &tn) {
    const int x = id & 7, s = id >> 3, r = s / ntn;
    tile = x + 8 * r;
    tn = s - r * ntn;
}
// Row tiles a grouped GEMM launches: each expert's ragged tail adds at most
// one to the full tiles, rounded up to a multiple of 8 (past the route's
// count a workgroup returns at once).
__host__ __device__ inline int moe_grid_tiles(int G, int BM, int E) { return ((G + BM - 1) / BM + E + 7) / 8 * 8; }

// The expert owning row tile `tile` of a grouped GEMM (int2_moe_prefill.cl:79-88
// searches it): the last e whose first tile meta[E + 1 + e] is <= tile.  The
// offsets never decrease, so that is the count of such experts less one: one
// load per lane, 64 experts at a time, and a ballot, in place of a binary
// search's chain of dependent loads.  (tile >= meta[E + 1] = 0.)
__device__ __forceinline__ int moe_tile_expert(const int *meta, int E, int tile, int lane) {
    int n = 0;
    for (int b = 0; b < E; b += 64) {
        const int i = b + lane;
        const bool le = i < E && meta[E + 1 + i] <= tile;
        n += __builtin_popcountll(__ballot(le));
    }
    return __builtin_amdgcn_readfirstlane(n - 1);
}

// A K-split workgroup's arrival at its column strip's counter (lane 0's atomic,
// broadcast): the value before this arrival.  atomic_inc wraps to 0 at the
// last of ksn arrivals, so the counters return to zero after every call.  A
// counter found above ksn - 1 holds no value any call leaves there (a
// workspace that was never zeroed): the increment has just reset it to 0, and
// this workgroup arrives once more, so the ksn increments from 0 still elect
// exactly the last arrival, after every slice's sums are stored.  (A stale
// value in 1 .. ksn - 1 cannot be told apart from a live count.)
__device__ __forceinline__ uint32_t split_arrive(uint32_t *c, int ksn, int lane) {
    uint32_t prev = 0;
    if (lane == 0) {
        prev = __builtin_amdgcn_atomic_inc32(c, (uint32_t)(ksn - 1), __ATOMIC_RELAXED, "agent");
        if (prev > (uint32_t)(ksn - 1)) prev = __builtin_amdgcn_atomic_inc32(c, (uint32_t)(ksn - 1), __ATOMIC_RELAXED, "agent");
    }
    return __builtin_amdgcn_readfirstlane(prev);
}

// c + w.lo * a.lo + w.hi * a.hi on packed DT pairs (v_dot2_f32_{f16,bf16})
template <bool BF16>
__device__ __forceinline__ float dot2(uint32_t w, uint32_t a, float c) {
    if constexpr (BF16) {
        bf162_t x, y;
        __builtin_memcpy(&x, &w, 4);
        __builtin_memcpy(&y, &a, 4);
        return __builtin_amdgcn_fdot2_f32_bf16(x, y, c, false);
    } else {
        half2_t x, y;
        __builtin_memcpy(&x, &w, 4);
        __builtin_memcpy(&y, &a, 4);
        return __builtin_amdgcn_fdot2(x, y, c, false);
    }
}

// ---- fused epilogue: common/epilogue.clh:22-48, common/epilogue.hpp:82 ----
// postop 0 none, 1 silu(acc)*other, 2 acc+other, 3 acc+bias, 4 sigmoid,
// 5 (acc+bias)+other (bias add + residual add, an extension).
// The sigmoid as the reference's kernels compute it (common/epilogue.clh:22-25:
// native_recip(native_exp(-x) + 1), 0 for x <= -10): the hardware's 2^x
// (v_exp_f32) of -x log2(e) and its reciprocal (v_rcp_f32), each within about
// an ulp; four VALU operations instead of ~20 for expf and an IEEE division.
// x = +inf gives 1, -inf 0 and NaN NaN, as the exact form does.
__device__ __forceinline__ float sigmoid_ref(float x) {
    const float e = __builtin_amdgcn_exp2f(-x * 1.44269504088896341f);
    return x <= -10.0f ? 0.0f : __builtin_amdgcn_rcpf(e + 1.0f);
}

__host__ __device__ constexpr bool postop_needs_other(int p) { return p == 1 || p == 2 || p == 5; }
__host__ __device__ constexpr bool postop_needs_bias(int p) { return p == 3 || p == 5; }

// Epilogue with the postop and output type fixed at compile time: kernels
// dispatch once (a uniform branch, epi_dispatch) to one of these instead of
// evaluating the postop switch per output.
template <int P> __device__ __forceinline__ float epi_apply_c(float v, float other, float bias) {
    if constexpr (P == 1) return v * sigmoid_ref(v) * other;
    else if constexpr (P == 2) return v + other;
    else if constexpr (P == 3) return v + bias;
    else if constexpr (P == 4) return sigmoid_ref(v);
    else if constexpr (P == 5) return (v + bias) + other;
    else return v;
}
// Epilogue + store of 4 consecutive outputs (m, n..n+3), n % 4 == 0.  NT: a
// non-temporal store, for outputs no kernel of the same call re-reads (the
// dense prefill GEMMs' C, 28 MB at M = 1024 N = 14336: written through, it
// would evict the weight and activation tiles other workgroups still read;
// same box, two runs each: C3's quant_a + int8 GEMM 98.8-99.1 -> 97.1-97.4
// us, the fp16 GEMM 106.6-106.7 -> 105.7-106.3 us; the MoE layer's outputs,
// re-read by its next GEMM, measured slower so: 383-391 -> 391-398 us).
template <bool BF16, int P, bool F32, bool NT = false>
__device__ __forceinline__ void epi_store4_c(void *C, const uint16_t *Other, const void *Bias, int N, int m, int n,
                                             const float v[4]) {
    const size_t i = (size_t)m * N + n;
    float o[4] = {0.f, 0.f, 0.f, 0.f}, b[4] = {0.f, 0.f, 0.f, 0.f};
    if constexpr (postop_needs_other(P)) {
        const uint2 t = *(const uint2 *)(Other + i);
        o[0] = dt2f<BF16>(t.x & 0xffffu); o[1] = dt2f<BF16>(t.x >> 16);
        o[2] = dt2f<BF16>(t.y & 0xffffu); o[3] = dt2f<BF16>(t.y >> 16);
    }
    if constexpr (postop_needs_bias(P)) {
        if constexpr (F32) {
            const float4 t = *(const float4 *)((const float *)Bias + n);
            b[0] = t.x; b[1] = t.y; b[2] = t.z; b[3] = t.w;
        } else {
            const uint2 t = *(const uint2 *)((const uint16_t *)Bias + n);
            b[0] = dt2f<BF16>(t.x & 0xffffu); b[1] = dt2f<BF16>(t.x >> 16);
            b[2] = dt2f<BF16>(t.y & 0xffffu); b[3] = dt2f<BF16>(t.y >> 16);
        }
    }
    float r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = epi_apply_c<P>(v[c], o[c], b[c]);
    typedef float epi_f32x4 __attribute__((ext_vector_type(4)));
    typedef uint32_t epi_u32x2 __attribute__((ext_vector_type(2)));
    if constexpr (F32) {
        const epi_f32x4 t = {r[0], r[1], r[2], r[3]};
        if constexpr (NT) __builtin_nontemporal_store(t, (epi_f32x4 *)((float *)C + i));
        else *(epi_f32x4 *)((float *)C + i) = t;
    } else {
        const epi_u32x2 t = {f2dt<BF16>(r[0]) | (f2dt<BF16>(r[1]) << 16), f2dt<BF16>(r[2]) | (f2dt<BF16>(r[3]) << 16)};
        if constexpr (NT) __builtin_nontemporal_store(t, (epi_u32x2 *)((uint16_t *)C + i));
        else *(epi_u32x2 *)((uint16_t *)C + i) = t;
    }
}

// Calls f(std::integral_constant<int, P>, std::integral_constant<bool, F32>)
// for the runtime (postop, out_f32); postop outside 0..5 acts as 0.
template <class Fn> __device__ __forceinline__ void epi_dispatch(int postop, int out_f32, Fn &&f) {
    auto go = [&](auto p) __attribute__((always_inline)) {
        if (out_f32) f(p, std::integral_constant<bool, true>{});
        else f(p, std::integral_constant<bool, false>{});
    };
    switch (postop) {
    case 1: go(std::integral_constant<int, 1>{}); break;
    case 2: go(std::integral_constant<int, 2>{}); break;
    case 3: go(std::integral_constant<int, 3>{}); break;
    case 4: go(std::integral_constant<int, 4>{}); break;
    case 5: go(std::integral_constant<int, 5>{}); break;
    default: go(std::integral_constant<int, 0>{}); break;
    }
}

// One output with the postop and output type fixed at compile time.
template <bool BF16, int P, bool F32>
__device__ __forceinline__ void epi_store1_c(void *C, const uint16_t *Other, const void *Bias, int N, int m, int n,
                                             float v) {
    const size_t i = (size_t)m * N + n;
    const float o = postop_needs_other(P) ? dt2f<BF16>(Other[i]) : 0.0f;
    float b = 0.0f;
    if constexpr (postop_needs_bias(P)) b = F32 ? ((const float *)Bias)[n] : dt2f<BF16>(((const uint16_t *)Bias)[n]);
    const float r = epi_apply_c<P>(v, o, b);
    if constexpr (F32) ((float *)C)[i] = r;
    else ((uint16_t *)C)[i] = (uint16_t)f2dt<BF16>(r);
}

// Raw buffer resource over [p, p + bytes).  A buffer load whose VGPR offset
// (plus its immediate offset) reaches `bytes` returns 0 instead of touching
// memory; the SGPR offset is not range-checked.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buf_rsrc(const void *p, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(p), (short)0, (int)bytes, 0x00020000);
}

// Workgroup -> (m tile, n tile) of a GEMM grid of mt x nt tiles, for a
// launch of 8 * ceil(mt * nt / 8) workgroups.  Workgroups are dealt to the 8
// XCDs round-robin (id % 8 runs on XCD id % 8); XCD x takes the contiguous
// range [x * per, (x + 1) * per) of the tiles in M-major order, so the
// workgroups of one XCD share the same few A row blocks (the larger operand
// per tile: DT or int8 rows against 2-bit weight columns) in that XCD's L2,
// and each row block is fetched into about one L2 instead of all eight.
// Returns false for the padding workgroups past the last tile.
__device__ __forceinline__ bool xcd_tile_ashare(int id, int mt, int nt, int &tm, int &tn) {
    const int tiles = mt * nt, per = (tiles + 7) / 8;
    const int t = (id & 7) * per + (id >> 3);
    if (t >= tiles) return false;
    tm = t / nt;
    tn = t - tm * nt;
    return true;
}
__host__ __device__ inline int xcd_ashare_grid(int mt, int nt) { return 8 * ((mt * nt + 7) / 8); }

// Workgroup -> (m tile, n tile) of a GEMM grid of mt x nt tiles.  Workgroups
// are dealt to the 8 XCDs round-robin (x, x+8, x+16, ... run on XCD x); those
// take all M tiles of column strip x, then of strip x+8, ... (when the strip
// count is a multiple of 8), so a strip's weights are fetched into one XCD's
// L2 once.
__device__ __forceinline__ void xcd_tile_of(int id, int mt, int nt, int &tm, int &tn) {
    if (nt % 8 == 0) {
        const int x = id & 7, r = id >> 3;
        tm = r % mt;
        tn = (r / mt) * 8 + x;
    } else {
        tm = id % mt;
        tn = id / mt;
    }
}

}  // namespace tcl

// ---- host side ----------------------------------------------------------
namespace tcl {
// Byte offsets of the MoE layer's workspace regions (moe.hip: moe_ws_layout).
struct MoeWs {
    size_t meta, desc, perm, inv, h, y, total;
};
// The int8 MoE prefill layer's workspace (byte offsets, each 256-byte aligned).
struct MoeI8Ws {
    size_t meta, perm, inv, sa1, h, sa2, y, xq, hq, total;
};
// Records the HIP error text for ternocl_last_error() and maps it to a status.
// Scratch bytes of the allocation-free MoE decode entry (moe.hip).
constexpr size_t kNoAllocScratchBytes = TERNOCL_NOALLOC_SCRATCH_BYTES;

ternocl_status launch_status(hipError_t e);
ternocl_status check_launch();
void set_error(const char *msg);
inline size_t align_up(size_t x, size_t a) { return (x + a - 1) / a * a; }
}  // namespace tcl
