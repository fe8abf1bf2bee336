// dh_flash_fwd.hip -- FlashAttention forward on gfx950 matrix cores.
//
// O = softmax(Q K^T * scale [causal mask j <= i]) V per (batch x head) slice, in the
// reference layout (B, S*D): slice b at b*S*D, rows of D contiguous.  Replaces the
// reference's CPU online-softmax loop and its one-work-item-per-row OpenCL kernel
// (runtime/nn/training.inc:284-401).  LSE = m + ln(l) per row is saved for the backward.
//
// Layout trick: the kernels compute S^T = K Q^T and O^T = V^T P^T, so in every MFMA
// result the lane index is the query row.  The online-softmax state (running max m,
// normaliser l) and the rescaling of the output accumulator are then lane-local; the
// only cross-lane step is one v_permlane32_swap per reduction (the two 32-lane halves
// hold the two interleaved halves of each key block).
//
// bf16 kernel (v_mfma_f32_32x32x16_bf16): work-group = 4 waves, 256 query rows; each
//   wave owns 64 rows (two 32-row sub-blocks) so every K/V fragment read from LDS feeds
//   two MFMAs.  Keys stream in stages of 64 (two 32-key sub-blocks), double-buffered in
//   LDS: K as [key][d] and V transposed to [d][key] (register transpose with v_perm_b32
//   on the way in).  Q fragments live in registers for the whole kernel.
// fp32 kernel (v_mfma_f32_32x32x2_f32): same structure with 32 rows per wave and K, V
//   both [key][d] in LDS.
// Causal work-groups are launched heaviest-first (longest key range) and all
//   q-tiles of one slice land on the same XCD, which shares that slice's K/V in L2.
#include <cmath>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int NT = 256;            // threads per work-group (4 waves)
constexpr int BN = 64;             // keys per LDS stage
constexpr float NEG = -1.0e30f;    // masked score (log2 domain); exp2 of it is 0

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------
// bf16
// ---------------------------------------------------------------------------------
template <int D>
struct Bf16Stage {
    static constexpr int KS = D + 8;        // K row stride in LDS (bf16)
    static constexpr int VS = BN + 4;       // V^T row stride in LDS (bf16)
    static constexpr int K_ELEMS = BN * KS;
    static constexpr int V_ELEMS = D * VS;
    static constexpr int KCH = BN * D / 8 / NT;          // 16-byte K chunks per thread
    static constexpr int VBLK = (BN / 4) * (D / 8);      // 4 key x 8 d blocks per stage
    u32x4 k[KCH];
    u32x4 v[4];

    // Rows at or beyond S read row S - 1 instead: finite data for keys that are masked
    // out, and no divergent branches around the loads.
    __device__ void fetch(const uint16_t* __restrict__ Kg, const uint16_t* __restrict__ Vg,
                          int j0, int S, int tid) {
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
            const int f = tid + c * NT;
            const int key = f / (D / 8), dq = f % (D / 8);
            const int j = min(j0 + key, S - 1);
            k[c] = *reinterpret_cast<const u32x4*>(Kg + (size_t)j * D + 8 * dq);
        }
        if (tid < VBLK) {
            const int kq = tid % (BN / 4), db = tid / (BN / 4);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = min(j0 + 4 * kq + r, S - 1);
                v[r] = *reinterpret_cast<const u32x4*>(Vg + (size_t)j * D + 8 * db);
            }
        }
    }
    __device__ void store(uint16_t* ks, uint16_t* vt, int tid) const {
#pragma unroll
        for (int c = 0; c < KCH; ++c) {
            const int f = tid + c * NT;
            const int key = f / (D / 8), dq = f % (D / 8);
            *reinterpret_cast<u32x4*>(&ks[key * KS + 8 * dq]) = k[c];
        }
        if (tid < VBLK) {
            const int kq = tid % (BN / 4), db = tid / (BN / 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x2 lo = {pack_lo16(v[0][q], v[1][q]), pack_lo16(v[2][q], v[3][q])};
                u32x2 hi = {pack_hi16(v[0][q], v[1][q]), pack_hi16(v[2][q], v[3][q])};
                *reinterpret_cast<u32x2*>(&vt[(8 * db + 2 * q) * VS + 4 * kq]) = lo;
                *reinterpret_cast<u32x2*>(&vt[(8 * db + 2 * q + 1) * VS + 4 * kq]) = hi;
            }
        }
    }
};

__device__ inline uint32_t cvt_pk_bf16(float a, float b) {
    return (uint32_t)__builtin_bit_cast(uint16_t, (__bf16)a) |
           ((uint32_t)__builtin_bit_cast(uint16_t, (__bf16)b) << 16);
}

// Lazy rescaling: a row keeps exponentiating against the max it already uses (m) until a
// block's max exceeds it by more than RESCALE_TH (log2 units).  Then p <= 2^RESCALE_TH,
// harmless for fp32 sums and bf16 P, and the 128-register output accumulator is rescaled
// only when some row of the wave actually needs it -- after the first blocks, almost never.
constexpr float RESCALE_TH = 8.0f;

// Scores S^T of one 64-key stage for one 32-row sub-block: sacc[kb] = K[32 kb ..] Q^T.
template <int D>
__device__ inline void scores(const uint16_t* ks, const bf16x8 (&qf)[D / 16], int l32, int h,
                              f32x16 (&sacc)[2]) {
    using St = Bf16Stage<D>;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
            const bf16x8 kf = *reinterpret_cast<const bf16x8*>(
                &ks[(32 * kb + l32) * St::KS + 16 * t + 8 * h]);
            sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[t], sacc[kb], 0, 0, 0);
        }
    }
}

// Online-softmax update of one 32-row sub-block for one stage, then O^T += V^T P^T.
// Keys j > lim (this lane's causal diagonal / the end of the sequence) are masked.
template <int D>
__device__ inline void softmax_pv(const uint16_t* vt, f32x16 (&sacc)[2], float scale_log2,
                                  int j0, int lim, int l32, int h, float& m, float& l,
                                  f32x16 (&oacc)[D / 32]) {
    using St = Bf16Stage<D>;
    constexpr int ND = D / 32;
    float mx = NEG;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int j = j0 + 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
            const float s = j > lim ? NEG : sacc[kb][r] * scale_log2;
            sacc[kb][r] = s;
            mx = fmaxf(mx, s);
        }
    mx = fmaxf(mx, xor32(mx));
    if (__any(mx > m + RESCALE_TH)) {      // wave-uniform: rare after the first blocks
        const float m_new = fmaxf(m, mx);
        const float corr = fast_exp2(m - m_new);
        m = m_new;
        l *= corr;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[d][r] *= corr;
    }
    float sum = 0.f;
    uint32_t pk[2][8];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int r = 0; r < 16; r += 2) {
            const float p0 = fast_exp2(sacc[kb][r] - m);
            const float p1 = fast_exp2(sacc[kb][r + 1] - m);
            sum += p0 + p1;
            pk[kb][r >> 1] = cvt_pk_bf16(p0, p1);
        }
    l += sum + xor32(sum);
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const bf16x8 pf = __builtin_bit_cast(
                bf16x8, u32x4{pk[kb][4 * kk], pk[kb][4 * kk + 1], pk[kb][4 * kk + 2],
                              pk[kb][4 * kk + 3]});
            const int key = 32 * kb + 16 * kk + 4 * h;
#pragma unroll
            for (int d = 0; d < ND; ++d) {
                const uint16_t* row = &vt[(32 * d + l32) * St::VS + key];
                const u32x2 a = *reinterpret_cast<const u32x2*>(row);
                const u32x2 b = *reinterpret_cast<const u32x2*>(row + 8);
                oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, u32x4{a[0], a[1], b[0], b[1]}), pf, oacc[d], 0, 0,
                    0);
            }
        }
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
flash_fwd_bf16_kernel(int BH, int S, float scale_log2, const uint16_t* __restrict__ Q,
                      const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                      uint16_t* __restrict__ O, float* __restrict__ LSE) {
    using St = Bf16Stage<D>;
    constexpr int ROWS_WG = 256, ND = D / 32, NTK = D / 16;
    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    uint16_t* const kbuf = smem;                       // 2 stages of K
    uint16_t* const vbuf = smem + 2 * St::K_ELEMS;     // 2 stages of V^T

    const int n_qt = (S + ROWS_WG - 1) / ROWS_WG;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int q0 = qt * ROWS_WG;
    const size_t base = (size_t)bh * S * D;
    const uint16_t* Qg = Q + base;
    const uint16_t* Kg = K + base;
    const uint16_t* Vg = V + base;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int wrow = q0 + 64 * wave;               // first row of this wave

    // Q fragments (B operand of S^T = K Q^T): lane (i, h) holds Q[i][16t + 8h .. +7].
    bf16x8 qf[2][NTK];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
        const int i = min(wrow + 32 * rs + l32, S - 1);
#pragma unroll
        for (int t = 0; t < NTK; ++t)
            qf[rs][t] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(Qg + (size_t)i * D + 16 * t + 8 * h));
    }

    f32x16 oacc[2][ND];
#pragma unroll
    for (int rs = 0; rs < 2; ++rs)
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[rs][d][r] = 0.f;
    float m[2] = {NEG, NEG}, l[2] = {0.f, 0.f};

    const int kend = CAUSAL ? min(S, q0 + ROWS_WG) : S;
    const int nst = (kend + BN - 1) / BN;
    St stage;
    if (nst > 0) {
        stage.fetch(Kg, Vg, 0, S, tid);
        stage.store(kbuf, vbuf, tid);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) stage.fetch(Kg, Vg, (st + 1) * BN, S, tid);
        const uint16_t* ks = kbuf + cur * St::K_ELEMS;
        const uint16_t* vt = vbuf + cur * St::V_ELEMS;
        const int j0 = st * BN;
#pragma unroll
        for (int rs = 0; rs < 2; ++rs) {
            const int r0 = wrow + 32 * rs;
            // causal: a sub-block whose rows all precede this stage has nothing to add
            if (CAUSAL && j0 > r0 + 31) continue;
            // keys above lim are masked: the causal diagonal and the end of the sequence
            const int lim = CAUSAL ? min(r0 + l32, S - 1) : S - 1;
            f32x16 sacc[2];
            scores<D>(ks, qf[rs], l32, h, sacc);
            softmax_pv<D>(vt, sacc, scale_log2, j0, lim, l32, h, m[rs], l[rs], oacc[rs]);
        }
        if (more) stage.store(kbuf + (cur ^ 1) * St::K_ELEMS, vbuf + (cur ^ 1) * St::V_ELEMS, tid);
        __syncthreads();
    }

    // Epilogue: lane (i, h) holds O^T[d][i] for d = 32*db + 8q + 4h + (0..3).
#pragma unroll
    for (int rs = 0; rs < 2; ++rs) {
        const int i = wrow + 32 * rs + l32;
        if (i >= S) continue;
        const float inv = l[rs] > 0.f ? 1.f / l[rs] : 0.f;
        uint16_t* orow = O + base + (size_t)i * D;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x2 w = {cvt_pk_bf16(oacc[rs][d][4 * q] * inv, oacc[rs][d][4 * q + 1] * inv),
                           cvt_pk_bf16(oacc[rs][d][4 * q + 2] * inv, oacc[rs][d][4 * q + 3] * inv)};
                *reinterpret_cast<u32x2*>(orow + 32 * d + 8 * q + 4 * h) = w;
            }
        if (h == 0) LSE[(size_t)bh * S + i] = (m[rs] + __log2f(l[rs])) * 0.69314718055994531f;
    }
}

// ---------------------------------------------------------------------------------
// fp32
// ---------------------------------------------------------------------------------
template <int D>
struct F32Stage {
    static constexpr int LS = D + 4;                  // row stride (floats)
    static constexpr int ELEMS = BN * LS;
    static constexpr int CH = BN * D / 4 / NT;        // float4 chunks per thread per tensor
    f32x4 k[CH], v[CH];

    __device__ void fetch(const float* __restrict__ Kg, const float* __restrict__ Vg, int j0,
                          int S, int tid) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int f = tid + c * NT;
            const int key = f / (D / 4), dq = f % (D / 4);
            const int j = j0 + key;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            k[c] = j < S ? *reinterpret_cast<const f32x4*>(Kg + (size_t)j * D + 4 * dq) : z;
            v[c] = j < S ? *reinterpret_cast<const f32x4*>(Vg + (size_t)j * D + 4 * dq) : z;
        }
    }
    __device__ void store(float* ks, float* vs, int tid) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int f = tid + c * NT;
            const int key = f / (D / 4), dq = f % (D / 4);
            *reinterpret_cast<f32x4*>(&ks[key * LS + 4 * dq]) = k[c];
            *reinterpret_cast<f32x4*>(&vs[key * LS + 4 * dq]) = v[c];
        }
    }
};

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(NT)
flash_fwd_f32_kernel(int BH, int S, float scale_log2, const float* __restrict__ Q,
                     const float* __restrict__ K, const float* __restrict__ V,
                     float* __restrict__ O, float* __restrict__ LSE) {
    using St = F32Stage<D>;
    constexpr int ROWS_WG = 128, ND = D / 32, NDQ = D / 4;
    extern __shared__ __attribute__((aligned(16))) float fsm[];
    float* const kbuf = fsm;
    float* const vbuf = fsm + 2 * St::ELEMS;

    const int n_qt = (S + ROWS_WG - 1) / ROWS_WG;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int q0 = qt * ROWS_WG;
    const size_t base = (size_t)bh * S * D;
    const float* Qg = Q + base;
    const float* Kg = K + base;
    const float* Vg = V + base;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = q0 + 32 * wave;
    const int i = r0 + l32;

    // Q fragment: for d-group u, lane (i, h) holds Q[i][4u + 2h], Q[i][4u + 2h + 1].
    float qf[NDQ][2];
#pragma unroll
    for (int u = 0; u < NDQ; ++u) {
        const float* q = Qg + (size_t)i * D + 4 * u + 2 * h;
        qf[u][0] = i < S ? q[0] : 0.f;
        qf[u][1] = i < S ? q[1] : 0.f;
    }
    f32x16 oacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[d][r] = 0.f;
    float m = NEG, l = 0.f;

    const int kend = CAUSAL ? min(S, q0 + ROWS_WG) : S;
    const int nst = (kend + BN - 1) / BN;
    St stage;
    if (nst > 0) {
        stage.fetch(Kg, Vg, 0, S, tid);
        stage.store(kbuf, vbuf, tid);
        __syncthreads();
    }
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) stage.fetch(Kg, Vg, (st + 1) * BN, S, tid);
        const float* ks = kbuf + cur * St::ELEMS;
        const float* vs = vbuf + cur * St::ELEMS;
        const int j0 = st * BN;

        f32x16 sacc[2];
        bool act[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            const int kb0 = j0 + 32 * kb;
            act[kb] = kb0 < S && (!CAUSAL || kb0 <= r0 + 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
            if (act[kb]) {
#pragma unroll
                for (int u = 0; u < NDQ; ++u) {
                    const float* kr = &ks[(32 * kb + l32) * St::LS + 4 * u + 2 * h];
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[0], qf[u][0], sacc[kb], 0, 0, 0);
                    sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x2f32(kr[1], qf[u][1], sacc[kb], 0, 0, 0);
                }
            }
        }
        float mx = NEG;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int j = j0 + 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
                float s = sacc[kb][r] * scale_log2;
                if (!act[kb] || j >= S || (CAUSAL && j > i)) s = NEG;
                sacc[kb][r] = s;
                mx = fmaxf(mx, s);
            }
        mx = fmaxf(mx, xor32(mx));
        const float m_new = fmaxf(m, mx);
        const float corr = fast_exp2(m - m_new);
        m = m_new;
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(sacc[kb][r] - m_new);
                sacc[kb][r] = p;
                sum += p;
            }
        sum += xor32(sum);
        l = l * corr + sum;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) oacc[d][r] *= corr;
        // O^T[d][i] += sum_j V[j][d] P[i][j]; MFMA r pairs key 8(r/4) + 4h + r%4 per half.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
            if (!act[kb]) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
#pragma unroll
                for (int d = 0; d < ND; ++d)
                    oacc[d] = __builtin_amdgcn_mfma_f32_32x32x2f32(
                        vs[key * St::LS + 32 * d + l32], sacc[kb][r], oacc[d], 0, 0, 0);
            }
        }
        if (more) stage.store(kbuf + (cur ^ 1) * St::ELEMS, vbuf + (cur ^ 1) * St::ELEMS, tid);
        __syncthreads();
    }

    if (i < S) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        float* orow = O + base + (size_t)i * D;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                f32x4 w = {oacc[d][4 * q] * inv, oacc[d][4 * q + 1] * inv,
                           oacc[d][4 * q + 2] * inv, oacc[d][4 * q + 3] * inv};
                *reinterpret_cast<f32x4*>(orow + 32 * d + 8 * q + 4 * h) = w;
            }
        if (h == 0) LSE[(size_t)bh * S + i] = (m + __log2f(l)) * 0.69314718055994531f;
    }
}

template <typename Kern>
int set_lds(Kern kern, size_t bytes, bool& done) {
    if (done) return DH_OK;
    hipError_t e = hipFuncSetAttribute((const void*)kern,
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
    if (e != hipSuccess)
        return set_error(DH_ERR_HIP, "dh_flash_fwd: LDS attribute: %s", hipGetErrorString(e));
    done = true;
    return DH_OK;
}

template <int D, bool CAUSAL>
int launch_bf16(int BH, int S, float sl2, const void* Q, const void* K, const void* V, void* O,
                float* LSE) {
    auto kern = flash_fwd_bf16_kernel<D, CAUSAL>;
    const size_t lds = 2 * (Bf16Stage<D>::K_ELEMS + Bf16Stage<D>::V_ELEMS) * sizeof(uint16_t);
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    const int grid = BH * ((S + 255) / 256);
    kern<<<grid, NT, lds, stream()>>>(BH, S, sl2, (const uint16_t*)Q, (const uint16_t*)K,
                                      (const uint16_t*)V, (uint16_t*)O, LSE);
    return check_launch("dh_flash_fwd(bf16)");
}

template <int D, bool CAUSAL>
int launch_f32(int BH, int S, float sl2, const void* Q, const void* K, const void* V, void* O,
               float* LSE) {
    auto kern = flash_fwd_f32_kernel<D, CAUSAL>;
    const size_t lds = 4 * F32Stage<D>::ELEMS * sizeof(float);
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    const int grid = BH * ((S + 127) / 128);
    kern<<<grid, NT, lds, stream()>>>(BH, S, sl2, (const float*)Q, (const float*)K,
                                      (const float*)V, (float*)O, LSE);
    return check_launch("dh_flash_fwd(f32)");
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" int dh_flash_fwd(int dtype, int BH, int S, int D, float scale, int causal,
                            const void* Q, const void* K, const void* V, void* O, float* LSE) {
    DH_TRY(ensure_init());
    if (BH < 0 || S < 0) return set_error(DH_ERR_INVALID, "dh_flash_fwd: negative shape");
    if (BH == 0 || S == 0) return DH_OK;
    if (!Q || !K || !V || !O || !LSE) return set_error(DH_ERR_INVALID, "dh_flash_fwd: null pointer");
    if (D != 32 && D != 64 && D != 128)
        return set_error(DH_ERR_UNSUPPORTED, "dh_flash_fwd: head dim %d (supported: 32, 64, 128)", D);
    if ((uintptr_t)Q % 16 || (uintptr_t)K % 16 || (uintptr_t)V % 16 || (uintptr_t)O % 16)
        return set_error(DH_ERR_INVALID, "dh_flash_fwd: Q/K/V/O must be 16-byte aligned");
    const float sl2 = scale * 1.4426950408889634f;
    if (dtype == DH_BF16) {
        if (D == 128) return causal ? launch_bf16<128, true>(BH, S, sl2, Q, K, V, O, LSE)
                                    : launch_bf16<128, false>(BH, S, sl2, Q, K, V, O, LSE);
        if (D == 64) return causal ? launch_bf16<64, true>(BH, S, sl2, Q, K, V, O, LSE)
                                   : launch_bf16<64, false>(BH, S, sl2, Q, K, V, O, LSE);
        return causal ? launch_bf16<32, true>(BH, S, sl2, Q, K, V, O, LSE)
                      : launch_bf16<32, false>(BH, S, sl2, Q, K, V, O, LSE);
    }
    if (dtype == DH_F32) {
        if (D == 128) return causal ? launch_f32<128, true>(BH, S, sl2, Q, K, V, O, LSE)
                                    : launch_f32<128, false>(BH, S, sl2, Q, K, V, O, LSE);
        if (D == 64) return causal ? launch_f32<64, true>(BH, S, sl2, Q, K, V, O, LSE)
                                   : launch_f32<64, false>(BH, S, sl2, Q, K, V, O, LSE);
        return causal ? launch_f32<32, true>(BH, S, sl2, Q, K, V, O, LSE)
                      : launch_f32<32, false>(BH, S, sl2, Q, K, V, O, LSE);
    }
    return set_error(DH_ERR_UNSUPPORTED, "dh_flash_fwd: dtype %d", dtype);
}
