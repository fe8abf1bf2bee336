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
// bf16 kernel (v_mfma_f32_32x32x16_bf16): work-group = 8 waves (two per SIMD), 32 query
//   rows per wave, 256 per work-group.  K and V stream in stages of 64 keys through a
//   4-deep LDS ring filled by direct-to-LDS DMA (no staging registers); both stay
//   row-major, V being read with the transposing ds_read_b64_tr_b16.  Q fragments live in
//   registers for the whole kernel.
// fp32 kernel (v_mfma_f32_32x32x2_f32): same structure with 32 rows per wave and K, V
//   both [key][d] in LDS.
// Causal work-groups are launched heaviest-first (longest key range) and all
//   q-tiles of one slice land on the same XCD, which shares that slice's K/V in L2.
#include <cmath>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int NT = 256;            // threads per work-group of the fp32 kernel (4 waves)
constexpr int BN = 64;             // keys per LDS stage
constexpr float NEG = -1.0e30f;    // masked score (log2 domain); exp2 of it is 0

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// ---------------------------------------------------------------------------------
// bf16
// ---------------------------------------------------------------------------------
constexpr int BF_WAVES = 8;                 // two waves per SIMD
constexpr int BF_NT = 64 * BF_WAVES;
constexpr int BF_ROWS = 32 * BF_WAVES;      // query rows per work-group (32 per wave)
constexpr int BF_NSTAGE = 4;                // LDS ring depth, in stages of BN keys

// One stage = a K tile then a V tile, each BN key rows of D bf16 kept row-major, moved
// by direct-to-LDS DMA in 1 KB blocks (64 lanes x 16 bytes).  The 16-byte chunk c of key
// row j sits at position c ^ swz(j) of its row:
//  K is read with b128 (16 consecutive rows of one chunk per LDS pass): kswz spreads those
//    rows over all 64 banks;
//  V is read with ds_read_b64_tr_b16 (4 consecutive rows x 64 bytes per pass): vswz
//    spreads those 4 rows over all 64 banks.
template <int D>
struct BfTile {
    static constexpr int CH = D / 8;                  // 16-byte chunks per key row
    static constexpr int ROWB = 2 * D;                // bytes per key row
    static constexpr int TILE = BN * ROWB;            // bytes of one K (or V) tile
    static constexpr int STAGE = 2 * TILE;
    static constexpr int NBLK = TILE / 1024;          // DMA blocks per tile
    static constexpr int RPB = 1024 / ROWB;           // key rows per DMA block
    static constexpr int PER = 2 * NBLK / BF_WAVES;   // DMA blocks per wave per stage
    static constexpr int RW = 256 / ROWB;             // key rows per 256-byte bank sweep
    static_assert(PER >= 1 && 2 * NBLK == PER * BF_WAVES, "stage must split over the waves");
    __device__ static int kswz(int j) { return (j * CH / 16) % CH; }
    __device__ static int vswz(int j) { return 4 * ((j / RW) % (4 / RW)); }
};

// Lazy rescaling: a row keeps exponentiating against the max it already uses (m) until a
// block's max exceeds it by more than RESCALE_TH (log2 units).  Then p <= 2^RESCALE_TH,
// harmless for fp32 sums and bf16 P, and the output accumulator is rescaled only when
// some row of the wave actually needs it -- after the first blocks, almost never.
constexpr float RESCALE_TH = 8.0f;

__device__ inline uint32_t cvt_pk_bf16(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));   // RNE
}

__device__ inline float dot2_bf16(uint32_t p, uint32_t q, float acc) {
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(b2, p), __builtin_bit_cast(b2, q),
                                           acc, false);
}

// One work-group = 8 waves x 32 query rows.  Per stage of 64 keys a wave computes
// S^T = K Q^T (2 x D/16 MFMAs, K from LDS, Q from registers), the online softmax on its
// 32 scores per lane, and O^T += V^T P^T (2 x 2 x D/32 MFMAs, V through transpose reads,
// P straight from the score registers).  The running max m is kept on raw scores (scale
// > 0), so p = exp2(s * sl2 - m * sl2) is one FMA and one exp; the row sum l is taken
// over the bf16-rounded p that the PV product uses (v_dot2_f32_bf16 with (1, 1)), per
// lane half, and combined once at the end.
template <int D, bool CAUSAL>
__global__ void __launch_bounds__(BF_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
flash_fwd_bf16_kernel(int BH, int S, float sl2, const uint16_t* __restrict__ Q,
                      const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                      uint16_t* __restrict__ O, float* __restrict__ LSE) {
    using T = BfTile<D>;
    constexpr int NTK = D / 16, ND = D / 32;
    extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];

    const int n_qt = (S + BF_ROWS - 1) / BF_ROWS;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int q0 = qt * BF_ROWS;
    const size_t base = (size_t)bh * S * D;
    const uint16_t* Qg = Q + base;
    const uint16_t* Kg = K + base;
    const uint16_t* Vg = V + base;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = q0 + 32 * wave;                 // first query row of this wave
    const uint32_t ring_lds = lds_addr(ring);

    // DMA work of this wave: blocks wave, wave + 8, ... of the stage (K tile first).
    uint32_t dlds[T::PER];
    int drow[T::PER], dcol[T::PER];
    bool dk[T::PER];
#pragma unroll
    for (int q = 0; q < T::PER; ++q) {
        const int gb = wave + BF_WAVES * q;
        const int tile = gb / T::NBLK, b = gb % T::NBLK;
        const int row = b * T::RPB + lane / T::CH, pos = lane % T::CH;
        dk[q] = tile == 0;
        dlds[q] = tile * T::TILE + b * 1024;
        drow[q] = row;
        dcol[q] = 8 * (pos ^ (tile == 0 ? T::kswz(row) : T::vswz(row)));
    }
    auto issue = [&](int st) {
        const int j0 = st * BN;
        const uint32_t sb = ring_lds + (st % BF_NSTAGE) * T::STAGE;
#pragma unroll
        for (int q = 0; q < T::PER; ++q) {
            const size_t off = (size_t)min(j0 + drow[q], S - 1) * D + dcol[q];
            lds_dma16((dk[q] ? Kg : Vg) + off, __builtin_amdgcn_readfirstlane(sb + dlds[q]));
        }
    };

    // Q fragments (B operand of S^T = K Q^T): lane (i, h) holds Q[i][16t + 8h .. +7].
    bf16x8 qf[NTK];
    {
        const int i = min(r0 + l32, S - 1);
#pragma unroll
        for (int t = 0; t < NTK; ++t)
            qf[t] = __builtin_bit_cast(
                bf16x8, *reinterpret_cast<const u32x4*>(Qg + (size_t)i * D + 16 * t + 8 * h));
        // Consume Q here: the compiler's own wait for these loads then sits before the
        // loop instead of inside it, where it would also drain the prefetched stages.
#pragma unroll
        for (int t = 0; t < NTK; ++t) asm volatile("" ::"v"(__builtin_bit_cast(u32x4, qf[t])));
    }
    // Byte offsets of this lane's fragment reads inside a K / V tile.
    uint32_t kofs[NTK], vofs[ND];
#pragma unroll
    for (int t = 0; t < NTK; ++t) kofs[t] = l32 * T::ROWB + 16 * ((2 * t + h) ^ T::kswz(l32));
    {
        const int i = lane & 15, g = (lane >> 4) & 1;
        const int vr = 4 * h + (i >> 2);           // key row within a 16-key step
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
            const int n = 32 * dt + 16 * g + 4 * (i & 3);
            vofs[dt] = vr * T::ROWB + 16 * ((n >> 3) ^ T::vswz(vr)) + 8 * ((n >> 2) & 1);
        }
    }

    f32x16 oacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) oacc[d][r] = 0.f;
    float m = -INFINITY, l = 0.f;
    const int lim = CAUSAL ? min(r0 + l32, S - 1) : S - 1;   // last key this row sees

    const int kend = CAUSAL ? min(S, q0 + BF_ROWS) : S;
    const int nst = (kend + BN - 1) / BN;
    // stages this wave computes: none if all its rows are padding, else up to its diagonal
    const int wlast = r0 >= S ? 0 : CAUSAL ? min(S - 1, r0 + 31) / BN + 1 : nst;

#pragma unroll
    for (int st = 0; st < BF_NSTAGE - 1; ++st)
        if (st < nst) issue(st);
    for (int st = 0; st < nst; ++st) {
        // stage st has landed once at most (stages issued after it) x PER loads remain
        const int ahead = min(nst - 1 - st, BF_NSTAGE - 2);
        if (ahead >= 2) wait_vmcnt<2 * T::PER>();
        else if (ahead == 1) wait_vmcnt<T::PER>();
        else wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (st + BF_NSTAGE - 1 < nst) issue(st + BF_NSTAGE - 1);
        if (st >= wlast) continue;

        const uint8_t* kt = ring + (st % BF_NSTAGE) * T::STAGE;
        const uint8_t* vt = kt + T::TILE;
        const int j0 = st * BN;
        // All K fragments of the stage are read up front so that the LDS latency overlaps
        // the MFMAs; the two 32-key chains alternate.
        bf16x8 kf[2][NTK];
#pragma unroll
        for (int t = 0; t < NTK; ++t)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                kf[kb][t] = *reinterpret_cast<const bf16x8*>(kt + kofs[t] + 32 * kb * T::ROWB);
        __builtin_amdgcn_sched_barrier(0);
        f32x16 sacc[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
        for (int t = 0; t < NTK; ++t)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[kb][t], qf[t], sacc[kb], 0, 0, 0);
        // sacc[kb][r] = S^T[key j0 + 32 kb + 8 (r / 4) + 4 h + r % 4][row r0 + l32]
        if (j0 + BN - 1 > (CAUSAL ? r0 : S - 1)) {        // wave-uniform: diagonal or tail
            const int rel = lim - j0 - 4 * h;             // mask offsets above rel
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) sacc[kb][r] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sacc[kb][r]);
        if (__any((mx - m) * sl2 > RESCALE_TH)) {      // wave-uniform: rare after the start
            mx = fmaxf(mx, xor32(mx));
            const float m_new = fmaxf(m, mx);
            const float corr = fast_exp2((m - m_new) * sl2);
            m = m_new;
            l *= corr;
#pragma unroll
            for (int d = 0; d < ND; ++d)
#pragma unroll
                for (int r = 0; r < 16; ++r) oacc[d][r] *= corr;
        }
        const float mb = m * sl2;
        uint32_t pk[2][8];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; r += 2) {
                const float p0 = fast_exp2(__builtin_fmaf(sacc[kb][r], sl2, -mb));
                const float p1 = fast_exp2(__builtin_fmaf(sacc[kb][r + 1], sl2, -mb));
                pk[kb][r >> 1] = cvt_pk_bf16(p0, p1);
                l = dot2_bf16(pk[kb][r >> 1], 0x3F803F80u, l);
            }
        // O^T += V^T P^T.  k-step kk of key block kb pairs keys 16 kk + 4 h + (0..3) and
        // 16 kk + 8 + 4 h + (0..3): the score registers 8 kk .. 8 kk + 7 of this lane.
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const bf16x8 pf = __builtin_bit_cast(
                    bf16x8, u32x4{pk[kb][4 * kk], pk[kb][4 * kk + 1], pk[kb][4 * kk + 2],
                                  pk[kb][4 * kk + 3]});
                const uint8_t* vk = vt + (32 * kb + 16 * kk) * T::ROWB;
#pragma unroll
                for (int d = 0; d < ND; ++d) {
                    const s16x4 a0 = ds_read_tr(reinterpret_cast<const uint16_t*>(vk + vofs[d]));
                    const s16x4 a1 = ds_read_tr(
                        reinterpret_cast<const uint16_t*>(vk + vofs[d] + 8 * T::ROWB));
                    const bf16x8 vf = __builtin_bit_cast(
                        bf16x8, s16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]});
                    oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[d], 0, 0, 0);
                }
            }
    }

    // Epilogue: lane (i, h) holds O^T[d][i] for d = 32 dt + 8 q + 4 h + (0..3).
    const int i = r0 + l32;
    l += xor32(l);
    if (i < S) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        uint16_t* orow = O + base + (size_t)i * D;
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u32x2 w = {cvt_pk_bf16(oacc[d][4 * q] * inv, oacc[d][4 * q + 1] * inv),
                           cvt_pk_bf16(oacc[d][4 * q + 2] * inv, oacc[d][4 * q + 3] * inv)};
                *reinterpret_cast<u32x2*>(orow + 32 * d + 8 * q + 4 * h) = w;
            }
        if (h == 0) LSE[(size_t)bh * S + i] = m * sl2 * 0.69314718055994531f + __logf(l);
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
    const size_t lds = (size_t)BF_NSTAGE * BfTile<D>::STAGE;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    const int grid = BH * ((S + BF_ROWS - 1) / BF_ROWS);
    kern<<<grid, BF_NT, lds, stream()>>>(BH, S, sl2, (const uint16_t*)Q, (const uint16_t*)K,
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
    if (!(scale > 0.f) || !std::isfinite(scale))
        return set_error(DH_ERR_INVALID, "dh_flash_fwd: scale must be finite and > 0");
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
