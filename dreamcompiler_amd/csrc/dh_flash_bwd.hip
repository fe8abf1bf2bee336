// dh_flash_bwd.hip -- FlashAttention backward on gfx950 matrix cores.
//
// Gradients of O = softmax(Q K^T * scale) V (causal or not) given O and the row LSE
// saved by the forward: P is recomputed as exp(S * scale - LSE) instead of the
// reference's two extra recompute passes for (m, l) and D_i
// (runtime/ops/autograd.inc:779-840).  Three launches, no floating-point atomics, so
// every run gives bit-identical gradients:
//   1. Dvec_i = dO_i . O_i                                   (one pass over O, dO)
//   2. per key tile:   dV += P^T dO,  dK += scale * dS^T Q    (dS = P o (dP - Dvec))
//   3. per query tile: dQ += scale * dS K                     (S and dP recomputed)
// MFMA layouts: in launch 2 the scores are formed as S = Q K^T so the lane index is the
// key (the row of dK / dV); in launch 3 as S^T = K Q^T so the lane index is the query.
// Either way the product that consumes P or dS takes it straight from the score
// registers (the same interleaved-key trick as the forward), and the second operand
// is read from an LDS tile staged transposed ([d][row]) for bf16 or row-major for fp32.
#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int NT = 256;
constexpr int RB = 32;   // rows (queries or keys) per LDS stage

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline uint32_t cvt_pk_bf16(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}

template <typename T> __device__ inline float to_f(T x);
template <> __device__ inline float to_f<float>(float x) { return x; }
template <> __device__ inline float to_f<uint16_t>(uint16_t x) { return bf16_bits_to_f32(x); }

// ---------------------------------------------------------------------------------
// 1. Dvec = rowsum(dO * O), 16 lanes per row, 8 elements per lane per step.
// ---------------------------------------------------------------------------------
template <typename T, int D>
__global__ void __launch_bounds__(NT)
dvec_kernel(int rows, const T* __restrict__ O, const T* __restrict__ dO, float* __restrict__ Dv) {
    const int row = blockIdx.x * (NT / 16) + (threadIdx.x >> 4);
    const int sub = threadIdx.x & 15;
    float acc = 0.f;
    if (row < rows) {
        const T* o = O + (size_t)row * D;
        const T* g = dO + (size_t)row * D;
        for (int d = sub; d < D; d += 16) acc += to_f<T>(o[d]) * to_f<T>(g[d]);
    }
    // reduce over the 16 lanes of a DPP row
    acc += dpp_quad_xor1(acc);
    acc += dpp_quad_xor2(acc);
    acc += dpp_half_mirror(acc);
    acc += dpp_row_mirror(acc);
    if (row < rows && sub == 0) Dv[row] = acc;
}

// ---------------------------------------------------------------------------------
// bf16 staging: a 32-row x D tile fetched as 4-row x 8-column blocks, written to LDS
// row-major ([row][d], stride D + 8) and optionally transposed ([d][row], stride 36).
// ---------------------------------------------------------------------------------
template <int D>
struct Tile16 {
    static constexpr int NS = D + 8;          // natural row stride (bf16)
    static constexpr int TS = RB + 4;         // transposed row stride (bf16)
    static constexpr int NAT = RB * NS;       // elements of a natural tile
    static constexpr int TRN = D * TS;        // elements of a transposed tile
    static constexpr int NB = (RB / 4) * (D / 8);   // blocks per tile

    u32x4 v[4];

    __device__ void fetch(const uint16_t* __restrict__ g, int r0, int S, int b) {
        const int kq = b % (RB / 4), db = b / (RB / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int row = r0 + 4 * kq + r;
            v[r] = row < S ? *reinterpret_cast<const u32x4*>(g + (size_t)row * D + 8 * db)
                           : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __device__ void store(uint16_t* nat, uint16_t* trn, int b) const {
        const int kq = b % (RB / 4), db = b / (RB / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<u32x4*>(&nat[(4 * kq + r) * NS + 8 * db]) = v[r];
        if (trn) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x2 lo = {pack_lo16(v[0][q], v[1][q]), pack_lo16(v[2][q], v[3][q])};
                u32x2 hi = {pack_hi16(v[0][q], v[1][q]), pack_hi16(v[2][q], v[3][q])};
                *reinterpret_cast<u32x2*>(&trn[(8 * db + 2 * q) * TS + 4 * kq]) = lo;
                *reinterpret_cast<u32x2*>(&trn[(8 * db + 2 * q + 1) * TS + 4 * kq]) = hi;
            }
        }
    }
};

// MFMA operand of 8 interleaved rows (4h + 16kk + {0..3} and +8) from a transposed tile.
__device__ inline bf16x8 trn_frag(const uint16_t* trn_row, int kk, int h) {
    const uint16_t* p = trn_row + 16 * kk + 4 * h;
    u32x2 a = *reinterpret_cast<const u32x2*>(p);
    u32x2 b = *reinterpret_cast<const u32x2*>(p + 8);
    return __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]});
}

// ---------------------------------------------------------------------------------
// 2. dK, dV (bf16).  Work-group: 128 keys (wave w owns keys k0 + 32w .. +31); loops
//    over 32-query stages.  S[i][j] and dP[i][j] come out with lane = key j and
//    register r = query 8(r/4) + 4h + r%4.
// ---------------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
bwd_dkdv_bf16_kernel(int BH, int S, float scale, float sl2, const uint16_t* __restrict__ Q,
                     const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                     const uint16_t* __restrict__ dO, const float* __restrict__ LSE,
                     const float* __restrict__ Dv, float* __restrict__ dK,
                     float* __restrict__ dV, int accumulate) {
    using Tl = Tile16<D>;
    constexpr int ND = D / 32, NTK = D / 16;
    constexpr int STAGE = 2 * Tl::NAT + 2 * Tl::TRN;     // bf16 elements per stage
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    __shared__ __attribute__((aligned(16))) float s_lse[2][RB], s_dv[2][RB];

    const int bh = blockIdx.x % BH;
    const int kt = blockIdx.x / BH;      // causal: small kt = longest query range, first
    const int kbase = kt * 128;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int k0 = kbase + 32 * wave;
    const int j = k0 + l32;

    // K and V rows of this lane's key as B operands: K[j][16t + 8h .. +7].
    bf16x8 kf[NTK], vf[NTK];
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
        const size_t off = base + (size_t)j * D + 16 * t + 8 * h;
        kf[t] = __builtin_bit_cast(bf16x8, j < S ? *reinterpret_cast<const u32x4*>(K + off)
                                                 : u32x4{0u, 0u, 0u, 0u});
        vf[t] = __builtin_bit_cast(bf16x8, j < S ? *reinterpret_cast<const u32x4*>(V + off)
                                                 : u32x4{0u, 0u, 0u, 0u});
    }
    f32x16 dkacc[ND], dvacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dkacc[d][r] = dvacc[d][r] = 0.f;

    const int qstart = CAUSAL ? kbase : 0;
    const int nst = qstart < S ? (S - qstart + RB - 1) / RB : 0;
    Tl tq, tg;
    float pre_lse = 0.f, pre_dv = 0.f;
    auto fetch = [&](int st) {
        const int r0 = qstart + st * RB;
        if (tid < Tl::NB) tq.fetch(Q + base, r0, S, tid);
        else if (tid < 2 * Tl::NB) tg.fetch(dO + base, r0, S, tid - Tl::NB);
        if (tid < RB) {
            const int row = r0 + tid;
            pre_lse = row < S ? LSE[(size_t)bh * S + row] * 1.4426950408889634f : 0.f;
            pre_dv = row < S ? Dv[(size_t)bh * S + row] : 0.f;
        }
    };
    auto store = [&](int buf) {
        uint16_t* sb = smem + buf * STAGE;
        if (tid < Tl::NB) tq.store(sb, sb + 2 * Tl::NAT, tid);
        else if (tid < 2 * Tl::NB)
            tg.store(sb + Tl::NAT, sb + 2 * Tl::NAT + Tl::TRN, tid - Tl::NB);
        if (tid < RB) {
            s_lse[buf][tid] = pre_lse;
            s_dv[buf][tid] = pre_dv;
        }
    };
    if (nst > 0) {
        fetch(0);
        store(0);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) fetch(st + 1);
        const int i0 = qstart + st * RB;
        // causal: queries i0..i0+31 all precede this wave's first key -> nothing to add
        if (!(CAUSAL && i0 + RB - 1 < k0)) {
            const uint16_t* qs = smem + cur * STAGE;
            const uint16_t* gs = qs + Tl::NAT;
            const uint16_t* qt = qs + 2 * Tl::NAT;
            const uint16_t* gt = qt + Tl::TRN;
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
            for (int t = 0; t < NTK; ++t) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(&qs[l32 * Tl::NS + 16 * t + 8 * h]);
                const bf16x8 g = *reinterpret_cast<const bf16x8*>(&gs[l32 * Tl::NS + 16 * t + 8 * h]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, kf[t], s, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(g, vf[t], dp, 0, 0, 0);
            }
            uint32_t pk[8], dk[8];
#pragma unroll
            for (int r = 0; r < 16; r += 4) {
                const int il = 8 * (r >> 2) + 4 * h;             // local query of reg r
                const f32x4 lse4 = *reinterpret_cast<const f32x4*>(&s_lse[cur][il]);
                const f32x4 dv4 = *reinterpret_cast<const f32x4*>(&s_dv[cur][il]);
                float p[4], ds[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = i0 + il + e;
                    const bool ok = i < S && j < S && (!CAUSAL || j <= i);
                    p[e] = ok ? fast_exp2(s[r + e] * sl2 - lse4[e]) : 0.f;
                    ds[e] = p[e] * (dp[r + e] - dv4[e]);
                }
                pk[r / 2] = cvt_pk_bf16(p[0], p[1]);
                pk[r / 2 + 1] = cvt_pk_bf16(p[2], p[3]);
                dk[r / 2] = cvt_pk_bf16(ds[0], ds[1]);
                dk[r / 2 + 1] = cvt_pk_bf16(ds[2], ds[3]);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const bf16x8 pf = __builtin_bit_cast(
                    bf16x8, u32x4{pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]});
                const bf16x8 sf = __builtin_bit_cast(
                    bf16x8, u32x4{dk[4 * kk], dk[4 * kk + 1], dk[4 * kk + 2], dk[4 * kk + 3]});
#pragma unroll
                for (int d = 0; d < ND; ++d) {
                    dvacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        trn_frag(&gt[(32 * d + l32) * Tl::TS], kk, h), pf, dvacc[d], 0, 0, 0);
                    dkacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        trn_frag(&qt[(32 * d + l32) * Tl::TS], kk, h), sf, dkacc[d], 0, 0, 0);
                }
            }
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    if (j >= S) return;
    // lane (j, h) holds dK^T[d][j], dV^T[d][j] for d = 32*db + 8q + 4h + (0..3)
    float* dkr = dK + base + (size_t)j * D;
    float* dvr = dV + base + (size_t)j * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = 32 * d + 8 * q + 4 * h;
            f32x4 a = {dkacc[d][4 * q] * scale, dkacc[d][4 * q + 1] * scale,
                       dkacc[d][4 * q + 2] * scale, dkacc[d][4 * q + 3] * scale};
            f32x4 b = {dvacc[d][4 * q], dvacc[d][4 * q + 1], dvacc[d][4 * q + 2],
                       dvacc[d][4 * q + 3]};
            if (accumulate) {
                a += *reinterpret_cast<const f32x4*>(dkr + col);
                b += *reinterpret_cast<const f32x4*>(dvr + col);
            }
            *reinterpret_cast<f32x4*>(dkr + col) = a;
            *reinterpret_cast<f32x4*>(dvr + col) = b;
        }
}

// ---------------------------------------------------------------------------------
// 3. dQ (bf16).  Work-group: 128 queries (wave w owns queries q0 + 32w .. +31); loops
//    over 32-key stages.  S^T and dP^T come out with lane = query.
// ---------------------------------------------------------------------------------
template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
bwd_dq_bf16_kernel(int BH, int S, float scale, float sl2, const uint16_t* __restrict__ Q,
                   const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                   const uint16_t* __restrict__ dO, const float* __restrict__ LSE,
                   const float* __restrict__ Dv, float* __restrict__ dQ, int accumulate) {
    using Tl = Tile16<D>;
    constexpr int ND = D / 32, NTK = D / 16;
    constexpr int STAGE = 2 * Tl::NAT + Tl::TRN;     // K natural, V natural, K^T
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];

    const int n_qt = (S + 127) / 128;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int qbase = qt * 128;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = qbase + 32 * wave;
    const int i = r0 + l32;

    bf16x8 qf[NTK], gf[NTK];
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
        const size_t off = base + (size_t)i * D + 16 * t + 8 * h;
        qf[t] = __builtin_bit_cast(bf16x8, i < S ? *reinterpret_cast<const u32x4*>(Q + off)
                                                 : u32x4{0u, 0u, 0u, 0u});
        gf[t] = __builtin_bit_cast(bf16x8, i < S ? *reinterpret_cast<const u32x4*>(dO + off)
                                                 : u32x4{0u, 0u, 0u, 0u});
    }
    const float lse2 = i < S ? LSE[(size_t)bh * S + i] * 1.4426950408889634f : 0.f;
    const float dvi = i < S ? Dv[(size_t)bh * S + i] : 0.f;
    f32x16 dqacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqacc[d][r] = 0.f;

    const int kend = CAUSAL ? min(S, qbase + 128) : S;
    const int nst = (kend + RB - 1) / RB;
    Tl tk, tv;
    auto fetch = [&](int st) {
        if (tid < Tl::NB) tk.fetch(K + base, st * RB, S, tid);
        else if (tid < 2 * Tl::NB) tv.fetch(V + base, st * RB, S, tid - Tl::NB);
    };
    auto store = [&](int buf) {
        uint16_t* sb = smem + buf * STAGE;
        if (tid < Tl::NB) tk.store(sb, sb + 2 * Tl::NAT, tid);
        else if (tid < 2 * Tl::NB) tv.store(sb + Tl::NAT, nullptr, tid - Tl::NB);
    };
    if (nst > 0) {
        fetch(0);
        store(0);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) fetch(st + 1);
        const int j0 = st * RB;
        if (!(CAUSAL && j0 > r0 + 31)) {
            const uint16_t* ks = smem + cur * STAGE;
            const uint16_t* vs = ks + Tl::NAT;
            const uint16_t* kt = ks + 2 * Tl::NAT;
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
            for (int t = 0; t < NTK; ++t) {
                const bf16x8 a = *reinterpret_cast<const bf16x8*>(&ks[l32 * Tl::NS + 16 * t + 8 * h]);
                const bf16x8 v = *reinterpret_cast<const bf16x8*>(&vs[l32 * Tl::NS + 16 * t + 8 * h]);
                s = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[t], s, 0, 0, 0);
                dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(v, gf[t], dp, 0, 0, 0);
            }
            uint32_t dk[8];
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                float ds[2];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int jj = j0 + 8 * ((r + e) >> 2) + 4 * h + ((r + e) & 3);
                    const bool ok = i < S && jj < S && (!CAUSAL || jj <= i);
                    const float p = ok ? fast_exp2(s[r + e] * sl2 - lse2) : 0.f;
                    ds[e] = p * (dp[r + e] - dvi);
                }
                dk[r / 2] = cvt_pk_bf16(ds[0], ds[1]);
            }
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const bf16x8 sf = __builtin_bit_cast(
                    bf16x8, u32x4{dk[4 * kk], dk[4 * kk + 1], dk[4 * kk + 2], dk[4 * kk + 3]});
#pragma unroll
                for (int d = 0; d < ND; ++d)
                    dqacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        trn_frag(&kt[(32 * d + l32) * Tl::TS], kk, h), sf, dqacc[d], 0, 0, 0);
            }
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    if (i >= S) return;
    float* dqr = dQ + base + (size_t)i * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = 32 * d + 8 * q + 4 * h;
            f32x4 a = {dqacc[d][4 * q] * scale, dqacc[d][4 * q + 1] * scale,
                       dqacc[d][4 * q + 2] * scale, dqacc[d][4 * q + 3] * scale};
            if (accumulate) a += *reinterpret_cast<const f32x4*>(dqr + col);
            *reinterpret_cast<f32x4*>(dqr + col) = a;
        }
}

// ---------------------------------------------------------------------------------
// fp32 variants (v_mfma_f32_32x32x2_f32).  All LDS tiles row-major [row][d] (stride
// D + 4): the per-key / per-query operands of the 32x32x2 MFMA are single floats, so
// a row-major tile read at column 32*db + l32 already yields the "transposed" operand.
// ---------------------------------------------------------------------------------
template <int D>
struct Tile32 {
    static constexpr int LS = D + 4;
    static constexpr int ELEMS = RB * LS;
    static constexpr int CH = RB * D / 4;           // float4 chunks per tile
    f32x4 v[(CH + NT - 1) / NT];
    __device__ void fetch(const float* __restrict__ g, int r0, int S, int tid) {
#pragma unroll
        for (int c = 0; c < (CH + NT - 1) / NT; ++c) {
            const int f = tid + c * NT;
            const int row = f / (D / 4), dq = f % (D / 4);
            v[c] = (f < CH && r0 + row < S)
                       ? *reinterpret_cast<const f32x4*>(g + (size_t)(r0 + row) * D + 4 * dq)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __device__ void store(float* lds, int tid) const {
#pragma unroll
        for (int c = 0; c < (CH + NT - 1) / NT; ++c) {
            const int f = tid + c * NT;
            if (f < CH) *reinterpret_cast<f32x4*>(&lds[(f / (D / 4)) * LS + 4 * (f % (D / 4))]) = v[c];
        }
    }
};

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
bwd_dkdv_f32_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                    const float* __restrict__ K, const float* __restrict__ V,
                    const float* __restrict__ dO, const float* __restrict__ LSE,
                    const float* __restrict__ Dv, float* __restrict__ dK,
                    float* __restrict__ dV, int accumulate) {
    using Tl = Tile32<D>;
    constexpr int ND = D / 32, NDQ = D / 4;
    extern __shared__ __attribute__((aligned(16))) float fsm[];
    __shared__ __attribute__((aligned(16))) float s_lse[2][RB], s_dv[2][RB];

    const int bh = blockIdx.x % BH;
    const int kt = blockIdx.x / BH;
    const int kbase = kt * 128;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int k0 = kbase + 32 * wave;
    const int j = k0 + l32;

    float kf[NDQ][2], vf[NDQ][2];
#pragma unroll
    for (int u = 0; u < NDQ; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const size_t off = base + (size_t)j * D + 4 * u + 2 * h + s;
            kf[u][s] = j < S ? K[off] : 0.f;
            vf[u][s] = j < S ? V[off] : 0.f;
        }
    f32x16 dkacc[ND], dvacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dkacc[d][r] = dvacc[d][r] = 0.f;

    const int qstart = CAUSAL ? kbase : 0;
    const int nst = qstart < S ? (S - qstart + RB - 1) / RB : 0;
    Tl tq, tg;
    float pre_lse = 0.f, pre_dv = 0.f;
    auto fetch = [&](int st) {
        const int r0 = qstart + st * RB;
        tq.fetch(Q + base, r0, S, tid);
        tg.fetch(dO + base, r0, S, tid);
        if (tid < RB) {
            const int row = r0 + tid;
            pre_lse = row < S ? LSE[(size_t)bh * S + row] * 1.4426950408889634f : 0.f;
            pre_dv = row < S ? Dv[(size_t)bh * S + row] : 0.f;
        }
    };
    auto store = [&](int buf) {
        float* sb = fsm + buf * 2 * Tl::ELEMS;
        tq.store(sb, tid);
        tg.store(sb + Tl::ELEMS, tid);
        if (tid < RB) {
            s_lse[buf][tid] = pre_lse;
            s_dv[buf][tid] = pre_dv;
        }
    };
    if (nst > 0) {
        fetch(0);
        store(0);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) fetch(st + 1);
        const int i0 = qstart + st * RB;
        if (!(CAUSAL && i0 + RB - 1 < k0)) {
            const float* qs = fsm + cur * 2 * Tl::ELEMS;
            const float* gs = qs + Tl::ELEMS;
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
            for (int u = 0; u < NDQ; ++u)
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int c = 4 * u + 2 * h + e;
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(qs[l32 * Tl::LS + c], kf[u][e], s, 0, 0, 0);
                    dp = __builtin_amdgcn_mfma_f32_32x32x2f32(gs[l32 * Tl::LS + c], vf[u][e], dp, 0, 0, 0);
                }
            float p[16], ds[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int il = 8 * (r >> 2) + 4 * h + (r & 3);
                const int i = i0 + il;
                const bool ok = i < S && j < S && (!CAUSAL || j <= i);
                p[r] = ok ? fast_exp2(s[r] * sl2 - s_lse[cur][il]) : 0.f;
                ds[r] = p[r] * (dp[r] - s_dv[cur][il]);
            }
            // dV^T[d][j] += sum_i dO[i][d] P[i][j]; MFMA r pairs query 8(r/4)+4h+r%4 per half
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int il = 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
                for (int d = 0; d < ND; ++d) {
                    dvacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(gs[il * Tl::LS + 32 * d + l32],
                                                                    p[r], dvacc[d], 0, 0, 0);
                    dkacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(qs[il * Tl::LS + 32 * d + l32],
                                                                    ds[r], dkacc[d], 0, 0, 0);
                }
            }
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    if (j >= S) return;
    float* dkr = dK + base + (size_t)j * D;
    float* dvr = dV + base + (size_t)j * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = 32 * d + 8 * q + 4 * h;
            f32x4 a = {dkacc[d][4 * q] * scale, dkacc[d][4 * q + 1] * scale,
                       dkacc[d][4 * q + 2] * scale, dkacc[d][4 * q + 3] * scale};
            f32x4 b = {dvacc[d][4 * q], dvacc[d][4 * q + 1], dvacc[d][4 * q + 2],
                       dvacc[d][4 * q + 3]};
            if (accumulate) {
                a += *reinterpret_cast<const f32x4*>(dkr + col);
                b += *reinterpret_cast<const f32x4*>(dvr + col);
            }
            *reinterpret_cast<f32x4*>(dkr + col) = a;
            *reinterpret_cast<f32x4*>(dvr + col) = b;
        }
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
bwd_dq_f32_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                  const float* __restrict__ K, const float* __restrict__ V,
                  const float* __restrict__ dO, const float* __restrict__ LSE,
                  const float* __restrict__ Dv, float* __restrict__ dQ, int accumulate) {
    using Tl = Tile32<D>;
    constexpr int ND = D / 32, NDQ = D / 4;
    extern __shared__ __attribute__((aligned(16))) float fsm[];

    const int n_qt = (S + 127) / 128;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int qbase = qt * 128;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = qbase + 32 * wave;
    const int i = r0 + l32;

    float qf[NDQ][2], gf[NDQ][2];
#pragma unroll
    for (int u = 0; u < NDQ; ++u)
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const size_t off = base + (size_t)i * D + 4 * u + 2 * h + s;
            qf[u][s] = i < S ? Q[off] : 0.f;
            gf[u][s] = i < S ? dO[off] : 0.f;
        }
    const float lse2 = i < S ? LSE[(size_t)bh * S + i] * 1.4426950408889634f : 0.f;
    const float dvi = i < S ? Dv[(size_t)bh * S + i] : 0.f;
    f32x16 dqacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqacc[d][r] = 0.f;

    const int kend = CAUSAL ? min(S, qbase + 128) : S;
    const int nst = (kend + RB - 1) / RB;
    Tl tk, tv;
    auto fetch = [&](int st) {
        tk.fetch(K + base, st * RB, S, tid);
        tv.fetch(V + base, st * RB, S, tid);
    };
    auto store = [&](int buf) {
        float* sb = fsm + buf * 2 * Tl::ELEMS;
        tk.store(sb, tid);
        tv.store(sb + Tl::ELEMS, tid);
    };
    if (nst > 0) {
        fetch(0);
        store(0);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) fetch(st + 1);
        const int j0 = st * RB;
        if (!(CAUSAL && j0 > r0 + 31)) {
            const float* ks = fsm + cur * 2 * Tl::ELEMS;
            const float* vs = ks + Tl::ELEMS;
            f32x16 s, dp;
#pragma unroll
            for (int r = 0; r < 16; ++r) s[r] = dp[r] = 0.f;
#pragma unroll
            for (int u = 0; u < NDQ; ++u)
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int c = 4 * u + 2 * h + e;
                    s = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[l32 * Tl::LS + c], qf[u][e], s, 0, 0, 0);
                    dp = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[l32 * Tl::LS + c], gf[u][e], dp, 0, 0, 0);
                }
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int jl = 8 * (r >> 2) + 4 * h + (r & 3);
                const int jj = j0 + jl;
                const bool ok = i < S && jj < S && (!CAUSAL || jj <= i);
                const float p = ok ? fast_exp2(s[r] * sl2 - lse2) : 0.f;
                const float ds = p * (dp[r] - dvi);
#pragma unroll
                for (int d = 0; d < ND; ++d)
                    dqacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(ks[jl * Tl::LS + 32 * d + l32],
                                                                    ds, dqacc[d], 0, 0, 0);
            }
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    if (i >= S) return;
    float* dqr = dQ + base + (size_t)i * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = 32 * d + 8 * q + 4 * h;
            f32x4 a = {dqacc[d][4 * q] * scale, dqacc[d][4 * q + 1] * scale,
                       dqacc[d][4 * q + 2] * scale, dqacc[d][4 * q + 3] * scale};
            if (accumulate) a += *reinterpret_cast<const f32x4*>(dqr + col);
            *reinterpret_cast<f32x4*>(dqr + col) = a;
        }
}

// ---------------------------------------------------------------------------------
// launch
// ---------------------------------------------------------------------------------
template <typename Kern>
int set_lds(Kern kern, size_t bytes, bool& done) {
    if (done) return DH_OK;
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess)
        return set_error(DH_ERR_HIP, "dh_flash_bwd: LDS attribute: %s", hipGetErrorString(e));
    done = true;
    return DH_OK;
}

template <int D, bool CAUSAL>
int run_bf16(int BH, int S, float scale, const void* Q, const void* K, const void* V,
             const void* dO, const float* LSE, const float* Dv, float* dQ, float* dK, float* dV,
             int acc) {
    using Tl = Tile16<D>;
    const float sl2 = scale * 1.4426950408889634f;
    const int tiles = (S + 127) / 128;
    {
        auto kern = bwd_dkdv_bf16_kernel<D, CAUSAL>;
        const size_t lds = 2 * (2 * Tl::NAT + 2 * Tl::TRN) * sizeof(uint16_t);
        static bool done = false;
        DH_TRY(set_lds(kern, lds, done));
        kern<<<BH * tiles, NT, lds, stream()>>>(BH, S, scale, sl2, (const uint16_t*)Q,
                                                (const uint16_t*)K, (const uint16_t*)V,
                                                (const uint16_t*)dO, LSE, Dv, dK, dV, acc);
        DH_TRY(check_launch("dh_flash_bwd(dK,dV bf16)"));
    }
    {
        auto kern = bwd_dq_bf16_kernel<D, CAUSAL>;
        const size_t lds = 2 * (2 * Tl::NAT + Tl::TRN) * sizeof(uint16_t);
        static bool done = false;
        DH_TRY(set_lds(kern, lds, done));
        kern<<<BH * tiles, NT, lds, stream()>>>(BH, S, scale, sl2, (const uint16_t*)Q,
                                                (const uint16_t*)K, (const uint16_t*)V,
                                                (const uint16_t*)dO, LSE, Dv, dQ, acc);
        DH_TRY(check_launch("dh_flash_bwd(dQ bf16)"));
    }
    return DH_OK;
}

template <int D, bool CAUSAL>
int run_f32(int BH, int S, float scale, const void* Q, const void* K, const void* V,
            const void* dO, const float* LSE, const float* Dv, float* dQ, float* dK, float* dV,
            int acc) {
    using Tl = Tile32<D>;
    const float sl2 = scale * 1.4426950408889634f;
    const int tiles = (S + 127) / 128;
    const size_t lds = 2 * 2 * Tl::ELEMS * sizeof(float);
    {
        auto kern = bwd_dkdv_f32_kernel<D, CAUSAL>;
        static bool done = false;
        DH_TRY(set_lds(kern, lds, done));
        kern<<<BH * tiles, NT, lds, stream()>>>(BH, S, scale, sl2, (const float*)Q,
                                                (const float*)K, (const float*)V,
                                                (const float*)dO, LSE, Dv, dK, dV, acc);
        DH_TRY(check_launch("dh_flash_bwd(dK,dV f32)"));
    }
    {
        auto kern = bwd_dq_f32_kernel<D, CAUSAL>;
        static bool done = false;
        DH_TRY(set_lds(kern, lds, done));
        kern<<<BH * tiles, NT, lds, stream()>>>(BH, S, scale, sl2, (const float*)Q,
                                                (const float*)K, (const float*)V,
                                                (const float*)dO, LSE, Dv, dQ, acc);
        DH_TRY(check_launch("dh_flash_bwd(dQ f32)"));
    }
    return DH_OK;
}

template <typename T, int D>
int run_dvec(int rows, const void* O, const void* dO, float* Dv) {
    dvec_kernel<T, D><<<(rows + 15) / 16, NT, 0, stream()>>>(rows, (const T*)O, (const T*)dO, Dv);
    return check_launch("dh_flash_bwd(Dvec)");
}

template <int D>
int dispatch(int dtype, int causal, int BH, int S, float scale, const void* Q, const void* K,
             const void* V, const void* O, const void* dO, const float* LSE, float* Dv,
             float* dQ, float* dK, float* dV, int acc) {
    const int rows = BH * S;
    if (dtype == DH_BF16) {
        DH_TRY((run_dvec<uint16_t, D>(rows, O, dO, Dv)));
        return causal ? run_bf16<D, true>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc)
                      : run_bf16<D, false>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc);
    }
    DH_TRY((run_dvec<float, D>(rows, O, dO, Dv)));
    return causal ? run_f32<D, true>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc)
                  : run_f32<D, false>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc);
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" int dh_flash_bwd(int dtype, int BH, int S, int D, float scale, int causal,
                            const void* Q, const void* K, const void* V, const void* O,
                            const void* dO, const float* LSE, float* dQ, float* dK, float* dV,
                            int accumulate) {
    DH_TRY(ensure_init());
    if (BH < 0 || S < 0) return set_error(DH_ERR_INVALID, "dh_flash_bwd: negative shape");
    if (BH == 0 || S == 0) return DH_OK;
    if (!Q || !K || !V || !O || !dO || !LSE || !dQ || !dK || !dV)
        return set_error(DH_ERR_INVALID, "dh_flash_bwd: null pointer");
    if (D != 32 && D != 64 && D != 128)
        return set_error(DH_ERR_UNSUPPORTED, "dh_flash_bwd: head dim %d (supported: 32, 64, 128)", D);
    if (dtype != DH_BF16 && dtype != DH_F32)
        return set_error(DH_ERR_UNSUPPORTED, "dh_flash_bwd: dtype %d", dtype);
    for (const void* p : {Q, K, V, O, dO, (const void*)dQ, (const void*)dK, (const void*)dV})
        if ((uintptr_t)p % 16) return set_error(DH_ERR_INVALID, "dh_flash_bwd: 16-byte alignment");
    // Dvec scratch (BH*S floats) from the pool; returned to it once the work is queued
    // (later users of the buffer are ordered after these kernels on the same stream).
    float* Dv = (float*)dh_malloc((size_t)BH * S * sizeof(float));
    if (!Dv) return DH_ERR_OOM;
    int st;
    if (D == 128) st = dispatch<128>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV, accumulate);
    else if (D == 64) st = dispatch<64>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV, accumulate);
    else st = dispatch<32>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV, accumulate);
    dh_free(Dv);
    return st;
}
