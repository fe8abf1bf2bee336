// dh_common.hpp -- internal helpers shared by the HIP translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/dream_hip.h"

namespace dh {

// ---- status plumbing (defined in dh_backend.hip) --------------------------------
int set_error(int code, const char* fmt, ...);
int ensure_init();                 // DH_OK or DH_ERR_NO_DEVICE
hipStream_t stream();
int check_launch(const char* what);   // hipGetLastError after a launch
int num_cus();
// C = beta C + sum_s part[s] (+ bias, then ReLU: the DH_EPI_* epilogue) over S fp32 partials
// of M x N (part[s] at part + s M N), added in a fixed order; defined in dh_gemm_f32.hip.
int splitk_reduce_launch(const float* part, int S, int M, int N, float beta, float* C, int ldc,
                         const float* bias, int epi);
// The fp32 flash backward's dQ (head dimension D = 128 or 64) from stored scale*dS, every
// 128-row query tile of every slice in one launch: dQ[bh][tile t] = beta dQ + dS_t K[bh]
// (dS_t's layout in flash_dq_from_ds_kernel); defined in dh_gemm_f32.hip.
int flash_dq_from_ds_f32(int BH, int S, int D, int causal, const float* dS, long long slice,
                         const float* K, float beta, float* dQ);

#define DH_TRY(expr)                      \
    do {                                  \
        int _s = (expr);                  \
        if (_s != DH_OK) return _s;       \
    } while (0)

// ---- division by a launch-invariant divisor -------------------------------------
// Multiply-high, add and shift (the round-up method of Granlund & Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994): for 1 <= d < 2^31,
// s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 (< 2^32), and for every
// 0 <= n < 2^31, n / d = (umulhi(n, m) + n) >> s (the sum stays below 2^32).
struct FastDiv {
    uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    uint32_t s = 0;
    while ((1ull << s) < d) ++s;
    const uint64_t m = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
    return {d, (uint32_t)m, s};
}

__device__ inline uint32_t fdiv(uint32_t n, const FastDiv& f) {
    return (__umulhi(n, f.m) + n) >> f.s;
}

// ---- vector types -------------------------------------------------------------
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// ---- bf16 bit helpers -----------------------------------------------------------
// Round to nearest even by bias-and-truncate, the rule of dream_to_bf16
// (runtime/nn/training.inc:1969-1976); NaN payloads follow the same arithmetic.
__host__ __device__ inline uint16_t f32_to_bf16_bits(float x) {
    uint32_t u = __builtin_bit_cast(uint32_t, x);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}
__host__ __device__ inline float bf16_bits_to_f32(uint16_t b) {
    return __builtin_bit_cast(float, (uint32_t)b << 16);
}
// Two fp32 -> packed bf16 pair (lo in bits 0-15).
__device__ inline uint32_t pack_bf16x2(float lo, float hi) {
    return (uint32_t)f32_to_bf16_bits(lo) | ((uint32_t)f32_to_bf16_bits(hi) << 16);
}

// ---- 16-bit lane shuffles used by register transposes ------------------------------
// lo16(a) | lo16(b) << 16 and hi16(a) | hi16(b) << 16 as single v_perm_b32 ops.
__device__ inline uint32_t pack_lo16(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ inline uint32_t pack_hi16(uint32_t a, uint32_t b) {
    return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// ---- wavefront reductions (64 lanes) ----------------------------------------------
// DPP for distances 1, 2 (quad permutes), 4 (half-row mirror), 8 (row mirror);
// the 16- and 32-lane steps use the gfx950 permlane swaps.  Every lane ends
// with the reduction over the full wave.
__device__ inline float dpp_quad_xor1(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, false));
}
__device__ inline float dpp_quad_xor2(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, false));
}
__device__ inline float dpp_half_mirror(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), 0x141, 0xF, 0xF, false));
}
__device__ inline float dpp_row_mirror(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(
        0, __builtin_bit_cast(int, v), 0x140, 0xF, 0xF, false));
}
// v_permlane32_swap with both operands = v returns {v[l & 31], v[(l & 31) + 32]}
// in every lane, i.e. the lane's own value and its partner l ^ 32 in half order.
// v_permlane16_swap does the same for partners l ^ 16 inside each 32-lane half.
__device__ inline void halves32(float v, float& lo, float& hi) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, (uint32_t)r[0]);
    hi = __builtin_bit_cast(float, (uint32_t)r[1]);
}
__device__ inline void halves16(float v, float& lo, float& hi) {
    uint32_t u = __builtin_bit_cast(uint32_t, v);
    auto r = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    lo = __builtin_bit_cast(float, (uint32_t)r[0]);
    hi = __builtin_bit_cast(float, (uint32_t)r[1]);
}
// Value held by lane l ^ 32.
__device__ inline float xor32(float v) {
    float lo, hi;
    halves32(v, lo, hi);
    return (__lane_id() & 32) ? lo : hi;
}

template <typename Op>
__device__ inline float wave_reduce(float v, Op op) {
    v = op(v, dpp_quad_xor1(v));
    v = op(v, dpp_quad_xor2(v));
    v = op(v, dpp_half_mirror(v));
    v = op(v, dpp_row_mirror(v));
    float lo, hi;
    halves16(v, lo, hi);
    v = op(lo, hi);
    halves32(v, lo, hi);
    return op(lo, hi);
}
struct OpMax { __device__ float operator()(float a, float b) const { return fmaxf(a, b); } };
struct OpSum { __device__ float operator()(float a, float b) const { return a + b; } };

// ---- LDS transfer primitives -------------------------------------------------------
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));

// ds_read_b64_tr_b16.  Within each group of 16 lanes, lane i supplies the address of 4
// consecutive 16-bit values R_i; lane j receives R_{j/4 + 4e}[j % 4] for e = 0..3.
__device__ inline s16x4 ds_read_tr(const uint16_t* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16(
        (s16x4 __attribute__((address_space(3)))*)(p));
}

// 16-byte direct-to-LDS load: lane l's 16 bytes land at lds_base + 16 l.  Issued as
// inline assembly so that the compiler's wait insertion, which cannot tell the DMA
// target from the stage being read, does not serialise every LDS read behind it; the
// kernel waits (vmcnt) itself before each barrier.  m0 holds the wave's LDS base; one
// wait state separates the m0 write from the DMA, as the hardware requires.  The
// compiler treats m0 as reserved and does not see this write: that is safe only while
// no compiler-generated instruction of the calling kernels reads m0 (none does in the
// gfx950 code of this library; LDS instructions there do not use it).
__device__ inline void lds_dma16(const void* g, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off"
                 :
                 : "s"(lds_base), "v"(g)
                 : "memory", "m0");
}

// Raw buffer resource (gfx9 family): 48-bit base, no stride, `bytes` addressable; loads
// beyond `bytes` (checked per dword) return zero.
__device__ inline u32x4 make_rsrc(const void* base, uint32_t bytes) {
    const uint64_t a = (uint64_t)(uintptr_t)base;
    return u32x4{(uint32_t)a, (uint32_t)(a >> 32) & 0xFFFFu, bytes, 0x00020000u};
}

// 16-byte direct-to-LDS buffer load: lane l's 16 bytes at rsrc base + voff land at
// lds_base + 16 l (zeros past the resource's range).  Same waiting rules as lds_dma16.
__device__ inline void lds_dma16_buf(uint32_t voff, u32x4 rsrc, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc)
                 : "memory", "m0");
}

// As lds_dma16_buf with a wave-uniform byte offset soff added to every lane's address.
__device__ inline void lds_dma16_buf_so(uint32_t voff, u32x4 rsrc, uint32_t soff, uint32_t lds_base) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                 :
                 : "s"(lds_base), "v"(voff), "s"(rsrc), "s"(soff)
                 : "memory", "m0");
}

__device__ inline uint32_t lds_addr(const void* p) {
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// N consecutive floats from p (16-byte loads for N a multiple of 4, one 8-byte load for 2;
// p aligned to match).
template <int N>
__device__ inline void load_floats(const float* __restrict__ p, float (&v)[N]) {
    if constexpr (N % 4 == 0) {
#pragma unroll
        for (int q = 0; q < N / 4; ++q) {
            const f32x4 t = *reinterpret_cast<const f32x4*>(p + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) v[4 * q + e] = t[e];
        }
    } else {
        static_assert(N == 2, "2, or a multiple of 4");
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        const f32x2 t = *reinterpret_cast<const f32x2*>(p);
        v[0] = t[0];
        v[1] = t[1];
    }
}

// N consecutive floats at byte offset off of a buffer resource; words past the resource's
// range read as zero.  Issued as 32-bit loads at consecutive offsets, which the backend merges
// into one wide load (this toolchain's 64- and 128-bit raw buffer load builtins emit a single
// dword load).  Offsets are signed ints so that constant parts fold into the instruction's
// immediate offset (an unsigned sum may wrap, which keeps each load's offset in its own
// register and the loads unmerged).
template <int N>
__device__ inline void buf_load_floats(__amdgpu_buffer_rsrc_t rs, int off, float (&v)[N]) {
#pragma unroll
    for (int e = 0; e < N; ++e)
        v[e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off + 4 * e, 0, 0));
}

// Wait until at most N of this wave's vector-memory operations are in flight.
template <int N>
__device__ inline void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---- XCD-aware tile order --------------------------------------------------------
// Logical tile index -> (tile row, tile column), walking groups of `group_m` tile-rows.
__device__ inline void grouped_tile(int logical, int tiles_m, int tiles_n, int group_m, int& tm,
                                    int& tn) {
    const int width = group_m * tiles_n;
    const int group = logical / width;
    const int first_m = group * group_m;
    const int gsz = min(tiles_m - first_m, group_m);
    const int in = logical - group * width;
    tm = first_m + in % gsz;
    tn = in / gsz;
}

// Work-groups are dealt round-robin to the 8 XCDs (block b runs on XCD b % 8).
// Remap so that each XCD receives a contiguous run of logical tiles, then walk
// tiles in groups of `group_m` tile-rows so neighbouring tiles on one XCD share
// A rows and B columns in that XCD's L2.
__device__ inline void xcd_tile_order(int bid, int nblocks, int tiles_m, int tiles_n,
                                      int group_m, int& tm, int& tn) {
    int logical = bid;
    if ((nblocks & 7) == 0) {
        const int per = nblocks >> 3;
        logical = (bid & 7) * per + (bid >> 3);
    }
    grouped_tile(logical, tiles_m, tiles_n, group_m, tm, tn);
}

// Work-group -> (slice bh, tile rank rr) for BH slices x n_t tiles per slice.  Work-groups are
// dealt round-robin to the 8 XCDs; XCD x takes the slices bh = x (mod 8) in groups of G and
// finishes one group before the next, rank 0 (the caller's heaviest tile) first within a
// group: the few slices in flight keep their operands in the XCD's L2.  The grid then has
// slice_grid(BH, n_t) = 8 ceil(BH / 8) n_t work-groups: when 8 does not divide BH an XCD
// holds ceil or floor of BH / 8 slices, and its work-groups past its last tile get bh = -1
// (nothing to do).  G <= 0: rank-major over all slices (bh = bid mod BH) on a grid of
// BH n_t, for BH that slice_grouping() declines.
__device__ inline void slice_group_order(int bid, int BH, int n_t, int G, int& bh, int& rr) {
    if (G <= 0) {
        bh = bid % BH;
        rr = bid / BH;
        return;
    }
    const int x = bid & 7, k = bid >> 3, spx = (BH - x + 7) >> 3;
    if (k >= spx * n_t) {
        bh = -1;
        rr = 0;
        return;
    }
    const int g = k / (G * n_t);
    const int gsz = min(G, spx - g * G);
    const int w = k - g * G * n_t;
    rr = w / gsz;
    bh = 8 * (g * G + w % gsz) + x;
}

// Whether to group slices by XCD: always when 8 divides BH; otherwise when the XCDs' unequal
// slice counts leave at most ~6% of the work's time with XCDs idle (rank-major order costs
// ~13% at config 4's shape with BH = 127 or 131: every XCD fetches every slice's operands).
inline bool slice_grouping(int BH) {
    return (BH & 7) == 0 || 100LL * BH >= 94LL * 8 * ((BH + 7) / 8);
}
inline long long slice_grid(int BH, int n_t) { return 8LL * ((BH + 7) / 8) * n_t; }

}  // namespace dh
