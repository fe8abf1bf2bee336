// dh_flash_bwd.hip -- FlashAttention backward on gfx950 matrix cores.
//
// Gradients of O = softmax(Q K^T * scale) V (causal or not) given O and the row LSE
// saved by the forward: P is recomputed as exp(S * scale - LSE) instead of the
// reference's two extra recompute passes for (m, l) and D_i
// (runtime/ops/autograd.inc:779-840).  No floating-point atomics, so every run gives
// bit-identical gradients.  fp32, three launches:
//   1. Dvec_i = dO_i . O_i                                   (one pass over O, dO)
//   2. per key tile:   dV += P^T dO,  dK += scale * dS^T Q    (dS = P o (dP - Dvec))
//   3. per query tile: dQ += scale * dS K                     (S and dP recomputed)
// or, at D = 128 and 64 where launch 2's 128-key work-groups fill the CUs, launch 2 also stores
// scale * dS and dQ is one GEMM launch over every 128-row query tile on it.
// bf16, two: the per-query-tile launch runs first and forms Dvec_i (and LSE_i log2 e) from
// the dO row it holds anyway and the O row, stores -Dvec_i and LSE_i log2 e, and the
// per-key-tile launch reads them.
// MFMA layouts: in launch 2 the scores are formed as S = Q K^T so the lane index is the
// key (the row of dK / dV); in launch 3 as S^T = K Q^T so the lane index is the query.
// Either way the product that consumes P or dS takes it straight from the score
// registers (the same interleaved-key trick as the forward).  bf16: the streamed tiles
// (Q, dO in launch 2; K, V in launch 3) arrive by direct-to-LDS DMA in 4-deep rings and
// the transposed operands come from the same tiles through transpose reads; fp32: tiles
// are staged through registers into row-major LDS.
#include <mutex>

#include <cstdlib>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int NT = 256;
constexpr int RB = 32;   // rows (queries or keys) per LDS stage

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ inline uint32_t cvt_pk_bf16(float a, float b) {
    typedef float f2 __attribute__((ext_vector_type(2)));
    typedef __bf16 b2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f2{a, b}, b2));   // RNE
}

// dK/dV epilogue store of one lane's 4 columns; acc_k / acc_v: add to the buffer's contents.
// kv_alias: dK and dV are the same buffer (K and V are one tensor, e.g. attention(q, q, q));
// it then receives dK + dV (+ its contents with acc_k), the sum the reference's per-input
// "+=" leaves there (autograd.inc:693-728).
__device__ inline void store_dkdv(float* dk, float* dv, f32x4 a, f32x4 b, int acc_k, int acc_v,
                                  int kv_alias) {
    if (kv_alias) {
        a += b;
        if (acc_k) a += *reinterpret_cast<const f32x4*>(dk);
        *reinterpret_cast<f32x4*>(dk) = a;
        return;
    }
    if (acc_k) a += *reinterpret_cast<const f32x4*>(dk);
    if (acc_v) b += *reinterpret_cast<const f32x4*>(dv);
    *reinterpret_cast<f32x4*>(dk) = a;
    *reinterpret_cast<f32x4*>(dv) = b;
}

// ---------------------------------------------------------------------------------
// 1. Dvec = rowsum(dO * O) (fp32; the bf16 dQ launch forms it itself).  16 lanes per row,
//    each reading its D / 16 consecutive elements of O and of dO as one vector (4 to 32
//    bytes; the entry point requires 16-byte aligned tensors and D is a multiple of 32);
//    work-groups stride over the 16-row groups so that a large BH * S does not launch one
//    tiny work-group per group.
// ---------------------------------------------------------------------------------
template <int NDW>
__device__ inline void load_dw(const uint32_t* __restrict__ p, uint32_t (&w)[NDW]) {
    if constexpr (NDW % 4 == 0) {
#pragma unroll
        for (int q = 0; q < NDW / 4; ++q) {
            const u32x4 v = *reinterpret_cast<const u32x4*>(p + 4 * q);
#pragma unroll
            for (int e = 0; e < 4; ++e) w[4 * q + e] = v[e];
        }
    } else if constexpr (NDW == 2) {
        const u32x2 v = *reinterpret_cast<const u32x2*>(p);
        w[0] = v[0];
        w[1] = v[1];
    } else {
        w[0] = *p;
    }
}

template <typename T, int D>
__global__ void __launch_bounds__(NT)
dvec_kernel(int rows, const T* __restrict__ O, const T* __restrict__ dO, float* __restrict__ Dv) {
    constexpr int NDW = D * (int)sizeof(T) / 4 / 16;   // dwords per lane
    static_assert(NDW == 1 || NDW == 2 || NDW % 4 == 0, "lane chunk of 4, 8 or 16n bytes");
    const int sub = threadIdx.x & 15;
    // row0 depends on the work-group only: every lane runs every iteration (DPP below)
    for (int row0 = blockIdx.x * (NT / 16); row0 < rows; row0 += gridDim.x * (NT / 16)) {
        const int row = row0 + (threadIdx.x >> 4);
        float acc = 0.f;
        if (row < rows) {
            uint32_t a[NDW], b[NDW];
            load_dw<NDW>(reinterpret_cast<const uint32_t*>(O + (size_t)row * D) + NDW * sub, a);
            load_dw<NDW>(reinterpret_cast<const uint32_t*>(dO + (size_t)row * D) + NDW * sub, b);
#pragma unroll
            for (int q = 0; q < NDW; ++q) {
                if constexpr (sizeof(T) == 2) {   // two bf16 per dword
                    acc += __uint_as_float(a[q] << 16) * __uint_as_float(b[q] << 16);
                    acc += __uint_as_float(a[q] & 0xffff0000u) * __uint_as_float(b[q] & 0xffff0000u);
                } else {
                    acc += __uint_as_float(a[q]) * __uint_as_float(b[q]);
                }
            }
        }
        // reduce over the 16 lanes of a DPP row
        acc += dpp_quad_xor1(acc);
        acc += dpp_quad_xor2(acc);
        acc += dpp_half_mirror(acc);
        acc += dpp_row_mirror(acc);
        if (row < rows && sub == 0) Dv[row] = acc;
    }
}

// ---------------------------------------------------------------------------------
// bf16 kernels.  Tiles stream through LDS rings filled by direct-to-LDS buffer loads
// (rows at or past S arrive as zeros).  A tile read both as b128 row fragments (MFMA A
// operand, one row per lane) and through ds_read_b64_tr_b16 (the transposed operand)
// keeps the 16-byte chunk c of row r at position c ^ dswz(r), conflict-free for both
// access patterns; a tile read only as rows uses kswz.
// ---------------------------------------------------------------------------------
template <int D, int ROWS>
struct BwTile {
    static constexpr int CH = D / 8;              // 16-byte chunks per row
    static constexpr int ROWB = 2 * D;            // bytes per row
    static constexpr int TILE = ROWS * ROWB;      // bytes per tile
    static constexpr int NBLK = TILE / 1024;      // 1 KB DMA blocks per tile
    static constexpr int RPB = 1024 / ROWB;       // rows per DMA block
    static constexpr int RW = 256 / ROWB;         // rows per 256-byte bank sweep
    __device__ static int kswz(int r) { return (r * CH / 16) % CH; }
    __device__ static int dswz(int r) { return 4 * ((r / RW) % (4 / RW)) + ((r >> 2) & 3); }
    __device__ static uint32_t rowfrag(int r, int c, bool dual) {
        return r * ROWB + 16 * (c ^ (dual ? dswz(r) : kswz(r)));
    }
    // Transpose-read address of row r, columns n .. n + 3 (n a multiple of 4).
    __device__ static uint32_t trfrag(int r, int n) {
        return r * ROWB + 16 * ((n >> 3) ^ dswz(r)) + 8 * ((n >> 2) & 1);
    }
    // DMA lane mapping: lane l of block b carries row b RPB + l / CH, stored at position
    // l % CH of that row, so it loads chunk (l % CH) ^ swz(row) of the row.
    __device__ static uint32_t dma_voff(int b, int lane, bool dual) {
        const int row = b * RPB + lane / CH, pos = lane % CH;
        return row * ROWB + 16 * (pos ^ (dual ? dswz(row) : kswz(row)));
    }
};

// Transposed MFMA A operand: 8 rows (r0 + 4h + i/4 and + 8, through the two offsets)
// by 32 columns, see the ds_read_tr lane rule.
__device__ inline bf16x8 tr_operand(const uint8_t* p, uint32_t o0, uint32_t o1) {
    const s16x4 a0 = ds_read_tr(reinterpret_cast<const uint16_t*>(p + o0));
    const s16x4 a1 = ds_read_tr(reinterpret_cast<const uint16_t*>(p + o1));
    return __builtin_bit_cast(bf16x8, s16x8{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]});
}

template <int PER>
__device__ inline void wait_dma(int ahead) {     // at most `ahead` stages of PER loads in flight
    if (ahead >= 2) wait_vmcnt<2 * PER>();
    else if (ahead == 1) wait_vmcnt<PER>();
    else wait_vmcnt<0>();
}

// ---------------------------------------------------------------------------------
// 2. dK, dV (bf16).  Work-group: 128 keys, 8 waves (two per SIMD).  Waves w and w + 4 own
//    the same 32 keys (group w % 4) and take alternate 32-query stages (parity w / 4): each
//    step of the loop consumes two stages, and at the end the odd-stage waves hand their
//    partial dK, dV to their partner through LDS, which adds and stores them (a fixed
//    order: results stay bit-identical run to run).  K and V of the 128 keys stay in LDS;
//    Q, dO and each step's LSE*log2(e) and Dvec stream through a 4-stage ring (two steps),
//    all of a step's DMA issued by the even-stage waves so that the odd-stage ones start
//    computing right after the step barrier (when both waves of a SIMD stalled on their
//    issue at once, the backward took 1.2-1.6% longer in a same-box A/B).
//    S = Q K^T and dP = dO V^T come out with lane = key j and register r = query
//    8 (r / 4) + 4 h + r % 4; P and dS feed dV^T += dO^T P and dK^T += Q^T dS straight from
//    those registers.
// ---------------------------------------------------------------------------------
constexpr int KV_WAVES = 8;
constexpr int KV_NT = 64 * KV_WAVES;
constexpr int KV_KEYS = 128;
constexpr int KV_BQ = 32;
constexpr int KV_NSTAGE = 4;

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(KV_NT) __attribute__((amdgpu_waves_per_eu(2, 2)))
bwd_dkdv_bf16_kernel(int BH, int S, float scale, float sl2, const uint16_t* __restrict__ Q,
                     const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                     const uint16_t* __restrict__ dO, const float* __restrict__ L2,
                     const float* __restrict__ Dv, float* __restrict__ dK,
                     float* __restrict__ dV, int acc_k, int acc_v, int kv_alias, int group) {
    using T = BwTile<D, KV_BQ>;
    using R = BwTile<D, KV_KEYS>;                    // resident K, V of the work-group's keys
    constexpr int ND = D / 32, NTK = D / 16;
    constexpr int VEC = 2 * T::TILE;                 // 1 KB of LSE*log2(e), then 1 KB of Dvec
                                                     // (a step's, in its first stage's slot)
    constexpr int STAGE = VEC + 2048;
    constexpr int KVRES = KV_NSTAGE * STAGE;         // K tile, then V tile, after the ring
    constexpr int PERR = 2 * R::NBLK / KV_WAVES;     // resident blocks per wave
    constexpr int PER = 4 * T::NBLK / 4;             // tile blocks per even-stage wave per step
    static_assert(PERR >= 1 && PERR * KV_WAVES == 2 * R::NBLK, "resident tiles must split");
    static_assert(PER >= 1 && PER * 4 == 4 * T::NBLK, "a step must split over the waves");
    static_assert(KV_WAVES * 64 * 32 * ND * 4 / 2 <= KVRES + 2 * R::TILE, "reduction fits LDS");
    extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];

    int bh, kt;                          // causal: small kt = longest query range, first
    slice_group_order(blockIdx.x, BH, (S + KV_KEYS - 1) / KV_KEYS, group, bh, kt);
    if (bh < 0) return;                  // padding of an XCD with one slice fewer
    const int kbase = kt * KV_KEYS;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int grp = wave & 3, par = wave >> 2;
    const int l32 = lane & 31, h = lane >> 5;
    const int k0 = kbase + 32 * grp;
    const int j = k0 + l32;
    const uint32_t ring_lds = lds_addr(ring);

    const int qstart = CAUSAL ? kbase : 0;
    const int nst = qstart < S ? (S - qstart + KV_BQ - 1) / KV_BQ : 0;
    const int nsteps = (nst + 1) / 2;
    // first stage with a query at or after this group's first key; none if no valid key
    const int wfirst = k0 >= S ? nst : CAUSAL ? (k0 - qstart) / KV_BQ : 0;
    // steps whose stage of this wave's parity lies in [wfirst, nst)
    const int s_end = (nst - par + 1) >> 1;
    const int s_first = min((wfirst - par + 1) >> 1, s_end);

    // DMA share per step of the even-stage waves w < 4: tile blocks w + 4 q over (stage in
    // step, tile, block), plus one vector block for waves 0 (LSE) and 1 (Dvec).
    uint32_t dlds[PER], dvoff[PER];
    int dsis[PER];
    bool dq_[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int gb = (wave & 3) + 4 * q;
        const int sis = gb / (2 * T::NBLK), rem = gb % (2 * T::NBLK);
        const int tile = rem / T::NBLK, b = rem % T::NBLK;
        dsis[q] = sis;
        dq_[q] = tile == 0;
        dlds[q] = sis * STAGE + tile * T::TILE + b * 1024;
        dvoff[q] = T::dma_voff(b, lane, true);
    }
    auto issue_step = [&](int sp) {
        const uint32_t sb = ring_lds + ((2 * sp) % KV_NSTAGE) * STAGE;
        if (wave < 4) {
#pragma unroll
            for (int q = 0; q < PER; ++q) {
                const int i0 = qstart + (2 * sp + dsis[q]) * KV_BQ;
                const u32x4 rs = make_rsrc((dq_[q] ? Q : dO) + base + (size_t)min(i0, S) * D,
                                           (uint32_t)max(S - i0, 0) * T::ROWB);
                lds_dma16_buf(dvoff[q], rs, __builtin_amdgcn_readfirstlane(sb + dlds[q]));
            }
        }
        // 256 floats of LSE*log2(e) (wave 0) or Dvec (wave 1) from the step's first query
        if (wave < 2) {
            const int i0 = qstart + 2 * sp * KV_BQ;
            const u32x4 rv = make_rsrc((wave == 0 ? L2 : Dv) + (size_t)bh * S + min(i0, S),
                                       (uint32_t)max(S - i0, 0) * 4);
            lds_dma16_buf(16 * lane, rv, __builtin_amdgcn_readfirstlane(sb + VEC + 1024 * wave));
        }
    };

    // K and V of the work-group's keys stay in LDS for the whole kernel (loaded first, so
    // the first step's wait also covers them); lane (j, h) reads K[j][16t + 8h .. +7] as
    // the B operand.
#pragma unroll
    for (int q = 0; q < PERR; ++q) {
        const int gb = wave + KV_WAVES * q;
        const int tile = gb / R::NBLK, b = gb % R::NBLK;
        const u32x4 rs = make_rsrc((tile == 0 ? K : V) + base + (size_t)kbase * D,
                                   (uint32_t)max(S - kbase, 0) * R::ROWB);
        lds_dma16_buf(R::dma_voff(b, lane, false), rs,
                      __builtin_amdgcn_readfirstlane(ring_lds + KVRES + tile * R::TILE + b * 1024));
    }
    uint32_t rofs[NTK], kofs[NTK];
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
        rofs[t] = T::rowfrag(l32, 2 * t + h, true);
        kofs[t] = KVRES + R::rowfrag(32 * grp + l32, 2 * t + h, false);
    }
    uint32_t tofs0[ND], tofs1[ND];
    {
        const int ii = lane & 15, g = (lane >> 4) & 1, vr = 4 * h + (ii >> 2);
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
            const int n = 32 * dt + 16 * g + 4 * (ii & 3);
            tofs0[dt] = T::trfrag(vr, n);
            tofs1[dt] = T::trfrag(vr + 8, n);
        }
    }
    f32x16 dkacc[ND], dvacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dkacc[d][r] = dvacc[d][r] = 0.f;

    if (nsteps > 0) issue_step(0);
    auto sync = [&](int sp) {
        wait_vmcnt<0>();                             // this step's stages (issued a step ago)
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (sp + 1 < nsteps) issue_step(sp + 1);     // into the slots of step sp - 1
    };
    // One stage, one MFMA per chunk, chunks fenced by sched_barrier(0) and operands read
    // one chunk ahead:
    //   S = Q K^T (NTK MFMAs);
    //   dP - Dvec = dO V^T - Dvec (NTK MFMAs whose chain starts from -Dvec), each chunk also
    //     exponentiating 16 / NTK scores of S, so the exponentials run while the matrix
    //     cores work;
    //   the mask (a branch, taken on diagonal and tail stages only);
    //   dS = P o (dP - Dvec) (one multiply) and the bf16 packing of P, dS for k-step 0;
    //   dV^T += dO^T P, dK^T += Q^T dS for k-step 0 (2 ND MFMAs), the chunks also packing
    //     k-step 1; then the same MFMAs for k-step 1.
    // k-step kk pairs queries 16 kk + 4 h + (0..3) and + 8: score registers 8 kk .. + 7.
    auto compute = [&](int st) {
        const uint8_t* qt = ring + (st % KV_NSTAGE) * STAGE;
        const uint8_t* gt = qt + T::TILE;
        const float* vec =   // the step's vectors, this stage's 32 queries
            reinterpret_cast<const float*>(ring + ((st & ~1) % KV_NSTAGE) * STAGE + VEC) + 32 * (st & 1);
        const int i0 = qstart + st * KV_BQ;
        constexpr int EPC = 16 / NTK;                // exponentials per dP chunk
        constexpr int NP = 2 * ND;                   // dV, dK MFMAs per k-step
        auto rowf = [&](const uint8_t* tile, int t) {
            return *reinterpret_cast<const bf16x8*>(tile + rofs[t]);
        };
        auto keyf = [&](int t, int v) {
            return *reinterpret_cast<const bf16x8*>(ring + kofs[t] + v * R::TILE);
        };
        // transposed operand of P2 slot s of k-step kk: dO^T (even s) or Q^T (odd s), d = s / 2
        auto trf = [&](int kk, int s) {
            return tr_operand((s & 1 ? qt : gt) + 16 * kk * T::ROWB, tofs0[s >> 1], tofs1[s >> 1]);
        };
        // dP's chain starts from -Dvec (stored negated), so it ends as dP - Dvec.
        f32x16 sc, dp;
        f32x4 l4[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            l4[q] = *reinterpret_cast<const f32x4*>(vec + 8 * q + 4 * h);
            const f32x4 d4 = *reinterpret_cast<const f32x4*>(vec + 256 + 8 * q + 4 * h);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                sc[4 * q + e] = 0.f;
                dp[4 * q + e] = d4[e];
            }
        }
        // operands of S/dP MFMA i (i < NTK: S, else dP), read two chunks ahead
        auto opa = [&](int i) { return rowf(i < NTK ? qt : gt, i % NTK); };
        auto opb = [&](int i) { return keyf(i % NTK, i < NTK ? 0 : 1); };
        bf16x8 fa[2] = {opa(0), opa(1)}, fb[2] = {opb(0), opb(1)};
#pragma unroll
        for (int t = 0; t < NTK; ++t) {
            const bf16x8 a = fa[t & 1], b = fb[t & 1];
            fa[t & 1] = opa(t + 2);
            fb[t & 1] = opb(t + 2);
            sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, sc, 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        float p[16];
        bf16x8 ta[2];                                // P2 operands, two MFMAs ahead
#pragma unroll
        for (int t = 0; t < NTK; ++t) {
            const bf16x8 a = fa[t & 1], b = fb[t & 1];
            if (t + 2 < NTK) {
                fa[t & 1] = opa(NTK + t + 2);
                fb[t & 1] = opb(NTK + t + 2);
            }
            if (t + 1 == NTK) {
                ta[0] = trf(0, 0);
                ta[1] = trf(0, 1);
            }
            dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, dp, 0, 0, 0);
#pragma unroll
            for (int e = EPC * t; e < EPC * (t + 1); ++e) {
                p[e] = fast_exp2(__builtin_fmaf(sc[e], sl2, -l4[e >> 2][e & 3]));
                asm volatile("" : "+v"(p[e]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // Queries past S and (causal) keys after the query are dropped.  Register r holds
        // query i0 + 4 h + o(r), o(r) = 8 (r / 4) + r % 4.
        if (i0 + KV_BQ > S || (CAUSAL && i0 < k0 + 31)) {   // wave-uniform: tail or diagonal
            const int lo = CAUSAL ? j - i0 - 4 * h : -KV_BQ;   // keep o >= lo (key <= query)
            const int hi = S - i0 - 4 * h;                      // keep o < hi (query < S)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int o = 8 * (r >> 2) + (r & 3);
                if (o < lo || o >= hi) p[r] = 0.f;
            }
        }
        // unit u: P and dS of registers 2u, 2u + 1 packed to bf16 pairs
        uint32_t pk[8], pd[8];
        auto pack = [&](int u) {
            const int r = 2 * u;
            const float ds0 = p[r] * dp[r];
            const float ds1 = p[r + 1] * dp[r + 1];
            pk[u] = cvt_pk_bf16(p[r], p[r + 1]);
            pd[u] = cvt_pk_bf16(ds0, ds1);
            asm volatile("" : "+v"(pk[u]), "+v"(pd[u]));
        };
#pragma unroll
        for (int u = 0; u < 4; ++u) pack(u);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[4 * kk], pk[4 * kk + 1], pk[4 * kk + 2], pk[4 * kk + 3]});
            const bf16x8 sf = __builtin_bit_cast(bf16x8, u32x4{pd[4 * kk], pd[4 * kk + 1], pd[4 * kk + 2], pd[4 * kk + 3]});
#pragma unroll
            for (int sl = 0; sl < NP; ++sl) {
                const int g = kk * NP + sl;
                const bf16x8 a = ta[g & 1];
                if (g + 2 < 2 * NP) ta[g & 1] = trf((g + 2) / NP, (g + 2) % NP);
                if (sl & 1) dkacc[sl >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, sf, dkacc[sl >> 1], 0, 0, 0);
                else dvacc[sl >> 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, pf, dvacc[sl >> 1], 0, 0, 0);
                if (kk == 0) {
#pragma unroll
                    for (int u = 4 + 4 * sl / NP; u < 4 + 4 * (sl + 1) / NP; ++u) pack(u);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        }
    };
    // Three loops (steps before this wave's first stage, steps with a stage, the rest) keep
    // the compute loop free of branches around the accumulators.
    for (int sp = 0; sp < s_first; ++sp) sync(sp);
    for (int sp = s_first; sp < s_end; ++sp) {
        sync(sp);
        compute(2 * sp + par);
    }
    for (int sp = s_end; sp < nsteps; ++sp) sync(sp);

    // Odd-stage partials to LDS (lane-major, conflict free), then the partner adds them.
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();
    float* red = reinterpret_cast<float*>(ring) + grp * (64 * 32 * ND);
    if (par == 1) {
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                red[((2 * d) * 16 + r) * 64 + lane] = dkacc[d][r];
                red[((2 * d + 1) * 16 + r) * 64 + lane] = dvacc[d][r];
            }
    }
    __syncthreads();
    if (par == 1 || j >= S) return;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            dkacc[d][r] += red[((2 * d) * 16 + r) * 64 + lane];
            dvacc[d][r] += red[((2 * d + 1) * 16 + r) * 64 + lane];
        }
    // lane (j, h) holds dK^T[d][j], dV^T[d][j] for d = 32 dt + 8 q + 4 h + (0..3)
    float* dkr = dK + base + (size_t)j * D;
    float* dvr = dV + base + (size_t)j * D;
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int col = 32 * d + 8 * q + 4 * h;
            f32x4 a = {dkacc[d][4 * q] * scale, dkacc[d][4 * q + 1] * scale,
                       dkacc[d][4 * q + 2] * scale, dkacc[d][4 * q + 3] * scale};
            f32x4 b = {dvacc[d][4 * q], dvacc[d][4 * q + 1], dvacc[d][4 * q + 2], dvacc[d][4 * q + 3]};
            store_dkdv(dkr + col, dvr + col, a, b, acc_k, acc_v, kv_alias);
        }
}

// ---------------------------------------------------------------------------------
// 3. dQ (bf16).  Work-group: W waves x 32 queries; 64-key stages of K and V through a
//    4-deep LDS ring on 8 waves (two per SIMD), a 2-deep one (64 KB at D = 128, two
//    work-groups per CU) on 4: stage st + 1 is issued after barrier st into the slot stage
//    st - 1 left, and each barrier waits for all.  S^T = K Q^T and dP^T = V dO^T come out with
//    lane = query; dS^T feeds dQ^T += K^T dS^T straight from the registers, K^T through
//    transpose reads of the same K tile.
// ---------------------------------------------------------------------------------
constexpr int DQ_BN = 64;

template <int W>
constexpr int dq_nstage() { return W == 8 ? 4 : 2; }

template <int D, bool CAUSAL, int W>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2)))
bwd_dq_bf16_kernel(int BH, int S, float scale, float sl2, const uint16_t* __restrict__ Q,
                   const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                   const uint16_t* __restrict__ O, const uint16_t* __restrict__ dO,
                   const float* __restrict__ LSE, float* __restrict__ L2,
                   float* __restrict__ Dv, float* __restrict__ dQ, int accumulate, int group) {
    using T = BwTile<D, DQ_BN>;
    constexpr int ND = D / 32, NTK = D / 16;
    constexpr int STAGE = 2 * T::TILE;               // K tile, then V tile
    constexpr int DQ_WAVES = W, DQ_ROWS = 32 * W, DQ_NSTAGE = dq_nstage<W>();
    constexpr int PER = 2 * T::NBLK / DQ_WAVES;
    static_assert(PER >= 1 && PER * DQ_WAVES == 2 * T::NBLK, "stage must split over the waves");
    extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];

    const int n_qt = (S + DQ_ROWS - 1) / DQ_ROWS;
    int bh, rr;
    slice_group_order(blockIdx.x, BH, n_qt, group, bh, rr);
    if (bh < 0) return;                  // padding of an XCD with one slice fewer
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int q0 = qt * DQ_ROWS;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = q0 + 32 * wave;
    const int i = r0 + l32;
    const uint32_t ring_lds = lds_addr(ring);
    const int kend = CAUSAL ? min(S, q0 + DQ_ROWS) : S;
    const int nst = (kend + DQ_BN - 1) / DQ_BN;
    const int wlast = r0 >= S ? 0 : CAUSAL ? min(S - 1, r0 + 31) / DQ_BN + 1 : nst;

    uint32_t dlds[PER], dvoff[PER];
    bool dk_[PER];
#pragma unroll
    for (int q = 0; q < PER; ++q) {
        const int gb = wave + DQ_WAVES * q;
        const int tile = gb / T::NBLK, b = gb % T::NBLK;
        dk_[q] = tile == 0;
        dlds[q] = tile * T::TILE + b * 1024;
        dvoff[q] = T::dma_voff(b, lane, tile == 0);
    }
    auto issue = [&](int st) {
        const int j0 = st * DQ_BN;
        const uint32_t sb = ring_lds + (st % DQ_NSTAGE) * STAGE;
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const u32x4 rs = make_rsrc((dk_[q] ? K : V) + base + (size_t)j0 * D,
                                       (uint32_t)(S - j0) * T::ROWB);
            lds_dma16_buf(dvoff[q], rs, __builtin_amdgcn_readfirstlane(sb + dlds[q]));
        }
    };

    // The first stages' DMA goes out before the row loads below, so that the two fetches
    // overlap (the compiler's wait for the rows is a full vmcnt(0): it cannot count the DMA,
    // so these stages have landed by the loop).
#pragma unroll
    for (int st = 0; st < DQ_NSTAGE - 1; ++st)
        if (st < nst) issue(st);

    // Q and dO rows of this lane's query as B operands: Q[i][16t + 8h .. +7].  The same
    // elements of O give the lane half of Dvec_i = dO_i . O_i; the two halves (lanes l and
    // l ^ 32) are added, and -Dvec_i and LSE_i log2(e) are stored for the dK/dV launch.
    bf16x8 qf[NTK], gf[NTK];
    float lse2, dvi;
    {
        const int ic = min(i, S - 1);
        float part = 0.f;
#pragma unroll
        for (int t = 0; t < NTK; ++t) {
            const size_t off = base + (size_t)ic * D + 16 * t + 8 * h;
            const u32x4 g4 = *reinterpret_cast<const u32x4*>(dO + off);
            const u32x4 o4 = *reinterpret_cast<const u32x4*>(O + off);
            qf[t] = __builtin_bit_cast(bf16x8, *reinterpret_cast<const u32x4*>(Q + off));
            gf[t] = __builtin_bit_cast(bf16x8, g4);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                part += __uint_as_float(o4[e] << 16) * __uint_as_float(g4[e] << 16);
                part += __uint_as_float(o4[e] & 0xffff0000u) * __uint_as_float(g4[e] & 0xffff0000u);
            }
        }
        dvi = part + xor32(part);
        lse2 = LSE[(size_t)bh * S + ic] * 1.4426950408889634f;
        if (h == 0 && i < S) {
            Dv[(size_t)bh * S + i] = -dvi;       // negated: the dK/dV launch's dP chain starts from it
            L2[(size_t)bh * S + i] = lse2;
        }
#pragma unroll
        for (int t = 0; t < NTK; ++t)
            asm volatile("" ::"v"(__builtin_bit_cast(u32x4, qf[t])), "v"(__builtin_bit_cast(u32x4, gf[t])));
        asm volatile("" ::"v"(lse2), "v"(dvi));
    }
    uint32_t kofs[NTK], vofs[NTK], tofs0[ND], tofs1[ND];
#pragma unroll
    for (int t = 0; t < NTK; ++t) {
        kofs[t] = T::rowfrag(l32, 2 * t + h, true);
        vofs[t] = T::rowfrag(l32, 2 * t + h, false);
    }
    {
        const int ii = lane & 15, g = (lane >> 4) & 1, vr = 4 * h + (ii >> 2);
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
            const int n = 32 * dt + 16 * g + 4 * (ii & 3);
            tofs0[dt] = T::trfrag(vr, n);
            tofs1[dt] = T::trfrag(vr + 8, n);
        }
    }
    f32x16 dqacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int r = 0; r < 16; ++r) dqacc[d][r] = 0.f;
    const int lim = CAUSAL ? min(i, S - 1) : S - 1;   // last key this query sees

    for (int st = 0; st < nst; ++st) {
        wait_dma<PER>(min(nst - 1 - st, DQ_NSTAGE - 2));
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
        if (st + DQ_NSTAGE - 1 < nst) issue(st + DQ_NSTAGE - 1);
        if (st >= wlast) continue;

        // One MFMA per chunk, chunks fenced by sched_barrier(0), operands read two chunks
        // ahead: S^T (2 NTK MFMAs, two chains), dP^T (2 NTK MFMAs) with two exponentials of
        // P per chunk, the mask, dS^T of group 0, then dQ^T += K^T dS^T by groups g =
        // (key block kb, k-step kk) of ND MFMAs, each chunk also packing part of group g + 1.
        const uint8_t* kt = ring + (st % DQ_NSTAGE) * STAGE;
        const uint8_t* vt = kt + T::TILE;
        const int j0 = st * DQ_BN;
        constexpr int NSD = 2 * NTK;                 // S^T (and dP^T) MFMAs per stage
        constexpr int NOP = 2 * NSD + 4 * ND;        // MFMAs per stage
        auto opnd = [&](int c) -> bf16x8 {          // A operand of MFMA c
            if (c < 2 * NSD) {
                const int t = (c % NSD) >> 1, kb = c & 1;
                return *reinterpret_cast<const bf16x8*>((c < NSD ? kt + kofs[t] : vt + vofs[t]) + 32 * kb * T::ROWB);
            }
            const int g = (c - 2 * NSD) / ND, d = (c - 2 * NSD) % ND;
            return tr_operand(kt + (32 * (g >> 1) + 16 * (g & 1)) * T::ROWB, tofs0[d], tofs1[d]);
        };
        f32x16 sc[2], dp[2];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sc[kb][r] = dp[kb][r] = 0.f;
        bf16x8 fa[2] = {opnd(0), opnd(1)};
#pragma unroll
        for (int c = 0; c < NSD; ++c) {
            const bf16x8 a = fa[c & 1];
            fa[c & 1] = opnd(c + 2);
            sc[c & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qf[c >> 1], sc[c & 1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
        float p[2][16];                              // P in the score layout
#pragma unroll
        for (int c = 0; c < NSD; ++c) {
            const bf16x8 a = fa[c & 1];
            fa[c & 1] = opnd(NSD + c + 2);
            dp[c & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, gf[c >> 1], dp[c & 1], 0, 0, 0);
#pragma unroll
            for (int e = 32 * c / NSD; e < 32 * (c + 1) / NSD; ++e) {
                p[e >> 4][e & 15] = fast_exp2(__builtin_fmaf(sc[e >> 4][e & 15], sl2, -lse2));
                asm volatile("" : "+v"(p[e >> 4][e & 15]));
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        // On the diagonal or tail stages (wave-uniform) keys after the query (causal) or past
        // S are dropped.  The empty volatile asm keeps the mask a real branch: the compiler
        // otherwise if-converts its 32 compares and selects into every stage.
        if (j0 + DQ_BN - 1 > (CAUSAL ? r0 : S - 1)) {
            asm volatile("" ::: "memory");
            const int rel = lim - j0 - 4 * h;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) p[kb][r] = 0.f;
        }
        uint32_t pd[16];   // dS^T[key][i] as bf16 pairs; pd[4 g + u] belongs to group g
        auto pack = [&](int q) {
            const int kb = q >> 3, r = 2 * (q & 7);
            pd[q] = cvt_pk_bf16(p[kb][r] * (dp[kb][r] - dvi), p[kb][r + 1] * (dp[kb][r + 1] - dvi));
            asm volatile("" : "+v"(pd[q]));
        };
#pragma unroll
        for (int u = 0; u < 4; ++u) pack(u);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int c = 2 * NSD; c < NOP; ++c) {
            const int g = (c - 2 * NSD) / ND, d = (c - 2 * NSD) % ND;
            const bf16x8 a = fa[c & 1];
            if (c + 2 < NOP) fa[c & 1] = opnd(c + 2);
            const bf16x8 sf = __builtin_bit_cast(bf16x8, u32x4{pd[4 * g], pd[4 * g + 1], pd[4 * g + 2], pd[4 * g + 3]});
            dqacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, sf, dqacc[d], 0, 0, 0);
            if (g < 3) {
#pragma unroll
                for (int u = 4 * d / ND; u < 4 * (d + 1) / ND; ++u) pack(4 * (g + 1) + u);
            }
            __builtin_amdgcn_sched_barrier(0);
        }
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
// fp32 variants (v_mfma_f32_16x16x4_f32 for dK/dV, v_mfma_f32_32x32x2_f32 for dQ).  All
// LDS tiles row-major [row][d] (stride D + 4): the per-key / per-query operands of the fp32
// MFMAs are single floats, so a row-major tile read at a column already yields the
// "transposed" operand.
// ---------------------------------------------------------------------------------
template <int D, int THREADS = NT>
struct Tile32 {
    static constexpr int LS = D + 4;
    static constexpr int ELEMS = RB * LS;
    static constexpr int CH = RB * D / 4;           // float4 chunks per tile
    f32x4 v[(CH + THREADS - 1) / THREADS];
    // The stage's base (uniform) plus a 32-bit unsigned offset per thread, so that the loads
    // take the scalar-base form instead of a 64-bit address per thread kept across stages (the
    // empty asm keeps the compiler from hoisting base + offset out of the stage loop as one).
    __device__ void fetch(const float* __restrict__ g, int r0, int S, int tid) {
        const float* gs = g + (size_t)r0 * D;
#pragma unroll
        for (int c = 0; c < (CH + THREADS - 1) / THREADS; ++c) {
            const int f = tid + c * THREADS;
            const int row = f / (D / 4), dq = f % (D / 4);
            uint32_t ob = 4u * (row * D + 4 * dq);   // bytes
            asm volatile("" : "+v"(ob));
            v[c] = (f < CH && r0 + row < S)
                       ? *reinterpret_cast<const f32x4*>(reinterpret_cast<const char*>(gs) + ob)
                       : f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    __device__ void store(float* lds, int tid) const {
#pragma unroll
        for (int c = 0; c < (CH + THREADS - 1) / THREADS; ++c) {
            const int f = tid + c * THREADS;
            if (f < CH) *reinterpret_cast<f32x4*>(&lds[(f / (D / 4)) * LS + 4 * (f % (D / 4))]) = v[c];
        }
    }
};

// fp32 dK/dV.  Work-group: 128 keys, 8 waves of 16 keys, each wave's K and V rows in
// registers (D / 2 floats per lane each) and its dK/dV accumulators too (D / 2 each); Q, dO
// and each stage's LSE*log2(e) and Dvec stream through a register-staged LDS double buffer
// of 32-query stages, one barrier per stage.  16 keys per wave (v_mfma_f32_16x16x4_f32 rather
// than 32 on 32x32x2) halve the per-wave registers, so two waves share each SIMD at
// D = 128 (234 VGPRs) and four at D <= 64 (two work-groups per CU).  Grids short of a round
// of the CUs take W = 4, 2 or 1 waves (64, 32, 16 keys) per work-group instead; with fewer
// threads staging each tile, the 1- and 2-wave forms get the whole register file.
// MFMA layouts (lane l: l16 = l % 16, g = l / 16): operands A[m = l16][k = g] and
// B[k = g][n = l16]; result register i of lane l is row 4 g + i, column l16.  S = Q K^T and
// dP = dO V^T per 16-query block qb come out with lane = key j and register i = query
// 16 qb + 4 g + i, and P, dS feed dV^T += dO^T P, dK^T += Q^T dS straight from those
// registers: k-step (qb, i) pairs lane group g with query 16 qb + 4 g + i.
template <int D, int W>
constexpr int dkdv_f32_wpe() { return W == 8 ? (D == 128 ? 2 : 4) : W == 4 ? 2 : 1; }

template <int D, bool CAUSAL, int W, bool DS = false>
__global__ void __launch_bounds__(64 * W)
__attribute__((amdgpu_waves_per_eu(dkdv_f32_wpe<D, W>(), dkdv_f32_wpe<D, W>())))
bwd_dkdv_f32_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                       const float* __restrict__ K, const float* __restrict__ V,
                       const float* __restrict__ dO, const float* __restrict__ LSE,
                       const float* __restrict__ Dv, float* __restrict__ dK,
                       float* __restrict__ dV, int accumulate, int kv_alias,
                       float* __restrict__ dS_out, long long ds_slice) {
    using Tl = Tile32<D, 64 * W>;
    constexpr int NB = D / 16, NDQ = D / 4, QB = RB / 16;
    extern __shared__ __attribute__((aligned(16))) float fsm[];
    __shared__ __attribute__((aligned(16))) float s_lse[2][RB], s_dv[2][RB];

    const int bh = blockIdx.x % BH;
    const int kt = blockIdx.x / BH;
    const int kbase = kt * 16 * W;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l16 = lane & 15, g = lane >> 4;
    const int k0 = kbase + 16 * wave;
    const int j = k0 + l16;

    // B operand of d-step u: K[j][4u + g], V[j][4u + g]
    float kf[NDQ], vf[NDQ];
#pragma unroll
    for (int u = 0; u < NDQ; ++u) {
        const size_t off = base + (size_t)j * D + 4 * u + g;
        kf[u] = j < S ? K[off] : 0.f;
        vf[u] = j < S ? V[off] : 0.f;
    }
    f32x4 dkacc[NB], dvacc[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) dkacc[b] = dvacc[b] = f32x4{0.f, 0.f, 0.f, 0.f};

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
            pre_lse = row < S ? LSE[(size_t)bh * S + row] : 0.f;   // scaled in store()
            pre_dv = row < S ? Dv[(size_t)bh * S + row] : 0.f;
        }
    };
    auto store = [&](int buf) {
        float* sb = fsm + buf * 2 * Tl::ELEMS;
        tq.store(sb, tid);
        tg.store(sb + Tl::ELEMS, tid);
        if (tid < RB) {
            // the log2(e) scaling here rather than at the load, so that no instruction waits
            // for the load (and, in order, for the Q/dO loads before it) until this store
            s_lse[buf][tid] = pre_lse * 1.4426950408889634f;
            s_dv[buf][tid] = pre_dv;
        }
    };
    // DS (128-key work-groups): scale dS of each stage goes to an LDS tile [RB queries][128
    // keys] (two, alternating by stage), and the work-group writes the previous stage's tile
    // out as whole 512-byte row pieces: row i of 128-row tile t lies at t (t + 1) 8192 +
    // (i - 128 t)(t + 1) 128 of the slice (causal: keys up to the tile's end) or at i 128 T
    // (all T tiles of keys), and this work-group's keys are the 128 from kbase.
    constexpr int DSS = 128 + 4;                                    // LDS tile row stride
    float* const dst = fsm + 4 * Tl::ELEMS;                         // [2][RB][DSS] with DS
    auto flush = [&](int stp) {
        static_assert(!DS || W == 8, "dS tiles need 128-key work-groups");
        const int row = tid >> 4, c0 = 8 * (tid & 15);              // 32 rows x 16 x 8 keys
        const int i = qstart + stp * RB + row;
        if (i >= S) return;
        const int t = i >> 7;
        const long long off = CAUSAL ? 8192LL * t * (t + 1) + (long long)(i - 128 * t) * (t + 1) * 128
                                     : (long long)i * (((S + 127) >> 7) << 7);
        const float* src = dst + (stp & 1) * RB * DSS + row * DSS + c0;
        float* out = dS_out + bh * ds_slice + off + kbase + c0;
        *reinterpret_cast<f32x4*>(out) = *reinterpret_cast<const f32x4*>(src);
        *reinterpret_cast<f32x4*>(out + 4) = *reinterpret_cast<const f32x4*>(src + 4);
    };
    if (nst > 0) {
        fetch(0);
        store(0);
        __syncthreads();
    }
    // K and V (kf, vf) have landed on every path into the stage loop.  store(0)'s wait covers
    // them only where a stage exists, and without this wait the compiler's wait insertion
    // cannot tell them from the loop's own loads: it made each stage's first MFMA wait for the
    // next stage's prefetch.  The builtin (vmcnt(0), expcnt and lgkmcnt untouched), unlike
    // inline assembly, is seen by that pass.
    __builtin_amdgcn_s_waitcnt(0x0F70);
    for (int st = 0; st < nst; ++st) {
        const int cur = st & 1;
        const bool more = st + 1 < nst;
        if (more) fetch(st + 1);
        // the previous stage's tile, complete since the barrier that ended that stage; the
        // next write to its buffer comes after this stage's barrier
        if (DS && st > 0) flush(st - 1);
        const int i0 = qstart + st * RB;
        if (CAUSAL && i0 + RB - 1 < k0) {
            // no key of this wave is visible to these queries: their dS entries are zeros
            if (DS) {
#pragma unroll
                for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        dst[cur * RB * DSS + (16 * qb + 4 * g + r) * DSS + 16 * wave + l16] = 0.f;
            }
        } else {
            const float* qs = fsm + cur * 2 * Tl::ELEMS;
            const float* gs = qs + Tl::ELEMS;
            f32x4 s[QB], dp[QB];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb) s[qb] = dp[qb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int u = 0; u < NDQ; ++u)
#pragma unroll
                for (int qb = 0; qb < QB; ++qb) {
                    const int a = (16 * qb + l16) * Tl::LS + 4 * u + g;
                    s[qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[a], kf[u], s[qb], 0, 0, 0);
                    dp[qb] = __builtin_amdgcn_mfma_f32_16x16x4f32(gs[a], vf[u], dp[qb], 0, 0, 0);
                }
            float p[QB][4], ds[QB][4];
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int il = 16 * qb + 4 * g + r;
                    const int i = i0 + il;
                    const bool ok = i < S && j < S && (!CAUSAL || j <= i);
                    p[qb][r] = ok ? fast_exp2(s[qb][r] * sl2 - s_lse[cur][il]) : 0.f;
                    ds[qb][r] = p[qb][r] * (dp[qb][r] - s_dv[cur][il]);
                    if (DS) dst[cur * RB * DSS + il * DSS + 16 * wave + l16] = ds[qb][r] * scale;
                }
            // dV^T[d][j] += sum_i dO[i][d] P[i][j], d = 16 b + (row of the result)
#pragma unroll
            for (int qb = 0; qb < QB; ++qb)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int row = (16 * qb + 4 * g + r) * Tl::LS + l16;
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        dvacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(gs[row + 16 * b], p[qb][r],
                                                                        dvacc[b], 0, 0, 0);
                        dkacc[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(qs[row + 16 * b], ds[qb][r],
                                                                        dkacc[b], 0, 0, 0);
                    }
                }
        }
        if (more) store(cur ^ 1);
        __syncthreads();
    }
    if (DS && nst > 0) flush(nst - 1);
    if (j >= S) return;
    float* dkr = dK + base + (size_t)j * D;
    float* dvr = dV + base + (size_t)j * D;
    // lane (j, g) holds dK^T[d][j], dV^T[d][j] for d = 16 b + 4 g + (0..3)
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int col = 16 * b + 4 * g;
        store_dkdv(dkr + col, dvr + col, dkacc[b] * scale, dvacc[b], accumulate, accumulate,
                   kv_alias);
    }
}

template <int D, bool CAUSAL, int WAVES>
__global__ void __launch_bounds__(64 * WAVES)
__attribute__((amdgpu_waves_per_eu(WAVES >= 4 ? WAVES / 4 : 1, WAVES >= 4 ? WAVES / 4 : 1)))
bwd_dq_f32_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                  const float* __restrict__ K, const float* __restrict__ V,
                  const float* __restrict__ dO, const float* __restrict__ LSE,
                  const float* __restrict__ Dv, float* __restrict__ dQ, int accumulate) {
    using Tl = Tile32<D, 64 * WAVES>;
    constexpr int ND = D / 32, NDQ = D / 4, ROWS = 32 * WAVES;
    extern __shared__ __attribute__((aligned(16))) float fsm[];

    const int n_qt = (S + ROWS - 1) / ROWS;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int qbase = qt * ROWS;
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

    const int kend = CAUSAL ? min(S, qbase + ROWS) : S;
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

// fp32, small grids, D <= 64 (config 3's 24 slices of 256 rows): the kernels above give a
// work-group of one wave 16 keys (or 32 queries) and walk the other dimension in series, one
// register-staged LDS stage after another -- at config 3 a 35 us chain each.  Here a work-group
// owns 16 keys (dK/dV) or 16 queries (dQ) and its 8 waves take 16-query (16-key) chunks of the
// other dimension round-robin, all operands loaded straight from global memory into the MFMA
// registers (no LDS staging, no barrier in the loop); the waves' partial sums meet in LDS and
// are added in wave order (bit-identical reruns).  v_mfma_f32_16x16x4_f32 layouts (lane l
// supplies A[l % 16][l / 16] and B[l / 16][l % 16]; result register r is D[4 (l / 16) + r]
// [l % 16]); c = l % 16, g = l / 16, DQ = D / 4, DV = D / 16:
//  dK/dV: S = Q K^T and dP = dO V^T pair Q[i0 + c][DQ g + u] with K[k0 + c][DQ g + u] at
//    k-step u (the order of d in the contraction is free as long as both operands agree);
//    result register r holds query i0 + 4 g + r, key k0 + c.  dV^T += dO^T P and
//    dK^T += Q^T dS take that query at k-step r, so P and dS feed the products in place; the A
//    operand of d-block b is dO[query][DV c + b] (Q for dK), read through a buffer resource
//    that returns zeros for rows past S; result register r' of d-block b is d = DV (4 g + r')
//    + b for key k0 + c.
//  dQ: S^T = K Q^T and dP^T = V dO^T (result register r: key k0 + 4 g + r, query q0 + c), then
//    dQ^T += K^T dS^T with the A operand K[key][DV c + e] of d-block e.
constexpr int S16_W = 8;

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(64 * S16_W)
bwd_dkdv_f32_s16_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                        const float* __restrict__ K, const float* __restrict__ V,
                        const float* __restrict__ dO, const float* __restrict__ LSE,
                        const float* __restrict__ Dv, float* __restrict__ dK,
                        float* __restrict__ dV, int accumulate, int kv_alias) {
    constexpr int W = S16_W, DQ = D / 4, DV = D / 16, RS = D + 4, PART = 2 * 16 * RS;
    extern __shared__ __attribute__((aligned(16))) float fsm[];   // per wave: dK rows, dV rows

    const int bh = blockIdx.x % BH;
    const int k0 = (blockIdx.x / BH) * 16;
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int j = k0 + c;                                  // this lane's key
    const __amdgpu_buffer_rsrc_t rq = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(Q + base), 0, 4 * S * D, 0x00020000);
    const __amdgpu_buffer_rsrc_t rg = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(dO + base), 0, 4 * S * D, 0x00020000);

    float kf[DQ], vf[DQ];
    load_floats(K + base + (size_t)min(j, S - 1) * D + DQ * g, kf);
    load_floats(V + base + (size_t)min(j, S - 1) * D + DQ * g, vf);
    f32x4 dk[DV], dv[DV];
#pragma unroll
    for (int b = 0; b < DV; ++b) dk[b] = dv[b] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int qstart = CAUSAL ? k0 : 0;                   // k0 < S: the grid covers S's keys
    const int nch = (S - qstart + 15) / 16;
    for (int ch = wave; ch < nch; ch += W) {
        const int i0 = qstart + 16 * ch;
        const int ia = min(i0 + c, S - 1);
        float qa[DQ], ga[DQ], qt[4][DV], gt[4][DV], l2[4], dvr[4];
        load_floats(Q + base + (size_t)ia * D + DQ * g, qa);
        load_floats(dO + base + (size_t)ia * D + DQ * g, ga);
        const int off = 4 * (i0 + 4 * g) * D + 4 * DV * c;   // row i0 + 4 g, this lane's columns
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i0 + 4 * g + r;
            buf_load_floats(rq, off + 4 * D * r, qt[r]);
            buf_load_floats(rg, off + 4 * D * r, gt[r]);
            const int ir = min(i, S - 1);
            l2[r] = LSE[(size_t)bh * S + ir] * 1.4426950408889634f;
            dvr[r] = Dv[(size_t)bh * S + ir];
        }
        f32x4 sa[2], pa[2];
        sa[0] = sa[1] = pa[0] = pa[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < DQ; ++u) {
            sa[u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(qa[u], kf[u], sa[u & 1], 0, 0, 0);
            pa[u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(ga[u], vf[u], pa[u & 1], 0, 0, 0);
        }
        float p[4], ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int i = i0 + 4 * g + r;
            const bool ok = i < S && j < S && (!CAUSAL || j <= i);
            p[r] = ok ? fast_exp2((sa[0][r] + sa[1][r]) * sl2 - l2[r]) : 0.f;
            ds[r] = ok ? p[r] * ((pa[0][r] + pa[1][r]) - dvr[r]) : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int b = 0; b < DV; ++b) {
                dv[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(gt[r][b], p[r], dv[b], 0, 0, 0);
                dk[b] = __builtin_amdgcn_mfma_f32_16x16x4f32(qt[r][b], ds[r], dk[b], 0, 0, 0);
            }
    }

    float* const part = fsm + wave * PART;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int b = 0; b < DV; ++b) {
            part[c * RS + DV * (4 * g + r) + b] = dk[b][r];
            part[16 * RS + c * RS + DV * (4 * g + r) + b] = dv[b][r];
        }
    __syncthreads();
    constexpr int QPR = D / 4;                             // 4-column groups per key row
    if (tid >= 16 * QPR) return;
    const int row = tid / QPR, col = 4 * (tid % QPR);
    const int jj = k0 + row;
    if (jj >= S) return;
    f32x4 a = {0.f, 0.f, 0.f, 0.f}, v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) {
        a += *reinterpret_cast<const f32x4*>(fsm + w * PART + row * RS + col);
        v += *reinterpret_cast<const f32x4*>(fsm + w * PART + 16 * RS + row * RS + col);
    }
    store_dkdv(dK + base + (size_t)jj * D + col, dV + base + (size_t)jj * D + col, a * scale, v,
               accumulate, accumulate, kv_alias);
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(64 * S16_W)
bwd_dq_f32_s16_kernel(int BH, int S, float scale, float sl2, const float* __restrict__ Q,
                      const float* __restrict__ K, const float* __restrict__ V,
                      const float* __restrict__ dO, const float* __restrict__ LSE,
                      const float* __restrict__ Dv, float* __restrict__ dQ, int accumulate) {
    constexpr int W = S16_W, DQ = D / 4, DV = D / 16, RS = D + 4, PART = 16 * RS;
    extern __shared__ __attribute__((aligned(16))) float fsm[];   // per wave: dQ rows

    const int n_qb = (S + 15) / 16;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int q0 = (CAUSAL ? n_qb - 1 - rr : rr) * 16;   // longest key range first
    const size_t base = (size_t)bh * S * D;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int qi = q0 + c;                                 // this lane's query
    const int qr = min(qi, S - 1);
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(K + base), 0, 4 * S * D, 0x00020000);

    float qf[DQ], gf[DQ];
    load_floats(Q + base + (size_t)qr * D + DQ * g, qf);
    load_floats(dO + base + (size_t)qr * D + DQ * g, gf);
    const float l2 = LSE[(size_t)bh * S + qr] * 1.4426950408889634f;
    const float dvi = Dv[(size_t)bh * S + qr];
    f32x4 dq[DV];
#pragma unroll
    for (int e = 0; e < DV; ++e) dq[e] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int kend = CAUSAL ? min(S, q0 + 16) : S;
    const int nch = (kend + 15) / 16;
    for (int ch = wave; ch < nch; ch += W) {
        const int k0 = 16 * ch;
        const int kr = min(k0 + c, S - 1);
        float ka[DQ], va[DQ], kt[4][DV];
        load_floats(K + base + (size_t)kr * D + DQ * g, ka);
        load_floats(V + base + (size_t)kr * D + DQ * g, va);
        int off = 4 * (k0 + 4 * g) * D + 4 * DV * c;   // row k0 + 4 g, this lane's columns
        asm volatile("" : "+v"(off));   // one base register per chunk, constants as immediates
#pragma unroll
        for (int r = 0; r < 4; ++r) buf_load_floats(rk, off + 4 * D * r, kt[r]);
        f32x4 sa[2], pa[2];
        sa[0] = sa[1] = pa[0] = pa[1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < DQ; ++u) {
            sa[u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(ka[u], qf[u], sa[u & 1], 0, 0, 0);
            pa[u & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(va[u], gf[u], pa[u & 1], 0, 0, 0);
        }
        float ds[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int key = k0 + 4 * g + r;
            const bool ok = qi < S && key < S && (!CAUSAL || key <= qi);
            const float p = ok ? fast_exp2((sa[0][r] + sa[1][r]) * sl2 - l2) : 0.f;
            ds[r] = ok ? p * ((pa[0][r] + pa[1][r]) - dvi) : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int e = 0; e < DV; ++e)
                dq[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(kt[r][e], ds[r], dq[e], 0, 0, 0);
    }

    float* const part = fsm + wave * PART;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < DV; ++e) part[c * RS + DV * (4 * g + r) + e] = dq[e][r];
    __syncthreads();
    constexpr int QPR = D / 4;
    if (tid >= 16 * QPR) return;
    const int row = tid / QPR, col = 4 * (tid % QPR);
    const int i = q0 + row;
    if (i >= S) return;
    f32x4 a = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int w = 0; w < W; ++w) a += *reinterpret_cast<const f32x4*>(fsm + w * PART + row * RS + col);
    float* dqr = dQ + base + (size_t)i * D + col;
    a *= scale;
    if (accumulate) a += *reinterpret_cast<const f32x4*>(dqr);
    *reinterpret_cast<f32x4*>(dqr) = a;
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

template <int D, bool CAUSAL, int W>
int launch_dq_bf16(int BH, int S, float scale, float sl2, const void* Q, const void* K,
                   const void* V, const void* O, const void* dO, const float* LSE, float* L2,
                   float* Dv, float* dQ, int acc, int group) {
    auto kern = bwd_dq_bf16_kernel<D, CAUSAL, W>;
    const size_t lds = (size_t)dq_nstage<W>() * 2 * BwTile<D, DQ_BN>::TILE;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    const int n_qt = (S + 32 * W - 1) / (32 * W);
    if (!slice_grouping(BH)) group = 0;
    const long long grid = group > 0 ? slice_grid(BH, n_qt) : (long long)BH * n_qt;
    kern<<<(unsigned)grid, 64 * W, lds, stream()>>>(BH, S, scale, sl2, (const uint16_t*)Q,
                                                   (const uint16_t*)K, (const uint16_t*)V,
                                                   (const uint16_t*)O, (const uint16_t*)dO, LSE,
                                                   L2, Dv, dQ, acc, group);
    return check_launch("dh_flash_bwd(dQ bf16)");
}

// dQ launch first (it also stores Dvec and LSE log2 e into Dv and L2), then dK/dV.  A gradient
// buffer shared with dQ is added to by the dK/dV launch, so shared buffers receive the sum.
template <int D, bool CAUSAL>
int run_bf16(int BH, int S, float scale, const void* Q, const void* K, const void* V,
             const void* O, const void* dO, const float* LSE, float* L2, float* Dv, float* dQ,
             float* dK, float* dV, int acc) {
    const int kv_alias = dK == dV;
    const int acc_k = acc || dK == dQ, acc_v = acc || dV == dQ;
    const float sl2 = scale * 1.4426950408889634f;
    // Each XCD walks its slices 4 at a time, heaviest tile first (slice_group_order): the Q, dO
    // (dK/dV launch) and K, V (dQ launch) streams of a few slices stay in the XCD's L2.
    // Config 4, same-box A/B (ms for the backward): rank-major over all slices 1.97; groups of
    // 1 slice 1.99, 2: 1.91, 4: 1.89-1.91, 8: 1.91, 16: 1.97.  Tuning knobs override.
    static const int group_kv = [] {
        const char* e = std::getenv("DH_FLASH_BWD_GROUP_KV");
        return e ? std::atoi(e) : 4;
    }();
    static const int group_q = [] {
        const char* e = std::getenv("DH_FLASH_BWD_GROUP_Q");
        return e ? std::atoi(e) : 4;
    }();
    // dQ on 4-wave work-groups (128 queries, two per CU, a two-stage ring) except D = 128 grids
    // of between one and four rounds of the 256-query tiles.  Same box, 8-wave / 4-wave time:
    // config 4 1.007-1.009, (16, 4096, 128) causal 1.072, (16, 2048, 64) causal 1.233,
    // (128, 2048, 64) 1.024; (32, 4096, 128) causal 0.980-0.985, (64, 2048, 128) 1.002.
    const long long grid8 = (long long)BH * ((S + 255) / 256);
    if (D == 128 && grid8 > num_cus() && grid8 < 4LL * num_cus())
        DH_TRY((launch_dq_bf16<D, CAUSAL, 8>(BH, S, scale, sl2, Q, K, V, O, dO, LSE, L2, Dv, dQ, acc, group_q)));
    else
        DH_TRY((launch_dq_bf16<D, CAUSAL, 4>(BH, S, scale, sl2, Q, K, V, O, dO, LSE, L2, Dv, dQ, acc, group_q)));
    {
        auto kern = bwd_dkdv_bf16_kernel<D, CAUSAL>;
        const size_t lds = (size_t)KV_NSTAGE * (2 * BwTile<D, KV_BQ>::TILE + 2048) +
                           2 * BwTile<D, KV_KEYS>::TILE;
        static bool done = false;
        DH_TRY(set_lds(kern, lds, done));
        const int n_kt = (S + KV_KEYS - 1) / KV_KEYS;
        const int gkv = slice_grouping(BH) ? group_kv : 0;
        const long long grid = gkv > 0 ? slice_grid(BH, n_kt) : (long long)BH * n_kt;
        kern<<<(unsigned)grid, KV_NT, lds, stream()>>>(BH, S, scale, sl2, (const uint16_t*)Q,
                                                       (const uint16_t*)K, (const uint16_t*)V,
                                                       (const uint16_t*)dO, L2, Dv, dK, dV,
                                                       acc_k, acc_v, kv_alias, gkv);
        DH_TRY(check_launch("dh_flash_bwd(dK,dV bf16)"));
    }
    return DH_OK;
}

template <int D, bool CAUSAL, int W, bool DS = false>
int launch_dkdv_f32(int BH, int S, float scale, float sl2, const void* Q, const void* K,
                    const void* V, const void* dO, const float* LSE, const float* Dv, float* dK,
                    float* dV, int acc, int kv_alias, size_t lds, float* dS_out = nullptr,
                    long long ds_slice = 0) {
    auto kern = bwd_dkdv_f32_kernel<D, CAUSAL, W, DS>;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    kern<<<BH * ((S + 16 * W - 1) / (16 * W)), 64 * W, lds, stream()>>>(
        BH, S, scale, sl2, (const float*)Q, (const float*)K, (const float*)V, (const float*)dO,
        LSE, Dv, dK, dV, acc, kv_alias, dS_out, ds_slice);
    return check_launch("dh_flash_bwd(dK,dV f32)");
}

template <int D, bool CAUSAL, int W>
int launch_dq_f32(int BH, int S, float scale, float sl2, const void* Q, const void* K,
                  const void* V, const void* dO, const float* LSE, const float* Dv, float* dQ,
                  int acc_q, size_t lds) {
    auto kern = bwd_dq_f32_kernel<D, CAUSAL, W>;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    kern<<<BH * ((S + 32 * W - 1) / (32 * W)), 64 * W, lds, stream()>>>(
        BH, S, scale, sl2, (const float*)Q, (const float*)K, (const float*)V, (const float*)dO,
        LSE, Dv, dQ, acc_q);
    return check_launch("dh_flash_bwd(dQ f32)");
}

// Waves per work-group: the most (8 at most) whose grid of `rows`-per-wave tiles still fills
// one round of the CUs, else 1.
inline int f32_waves(int BH, int S, int rows) {
    int w = 8;
    while (w > 1 && (long long)BH * ((S + rows * w - 1) / (rows * w)) < num_cus()) w /= 2;
    return w;
}

template <int D, bool CAUSAL>
int run_f32(int BH, int S, float scale, const void* Q, const void* K, const void* V,
            const void* dO, const float* LSE, const float* Dv, float* dQ, float* dK, float* dV,
            int acc, int kv_alias, int acc_q, int allow_ds) {
    using Tl = Tile32<D>;
    const float sl2 = scale * 1.4426950408889634f;
    // Small and mid grids: the 16-key / 16-query kernels, where the tiled kernels' work-groups
    // walk long serial chains.  D <= 64: grids of under a round of 128-row tiles; causal ones
    // up to a round, or two with S >= 2048, where their uneven key ranges leave CUs waiting.
    // D = 128 (the dK/dV kernel at 238 VGPRs, two waves per SIMD): causal grids under a round,
    // non-causal under half.  Same box, whole backward, these kernels / the tiled ones (us):
    // config 3 26.8 / 75.8, (2, 1040, 64) 56.8 / 281, (8, 1024, 64) causal 73 / 253,
    // non-causal 110 / 259, (16, 2048, 64) causal 400 / 556, (64, 512, 64) causal 141 / 161,
    // (32, 2048, 32) causal 401 / 465, (24, 256, 128) causal 46.7 / 134, (16, 1024, 128)
    // causal 279 / 420, (8, 512, 128) 79 / 252; tiled kept: (32, 1024, 32) non-causal 206 /
    // 184, (64, 1024, 64) causal 429 / 429, (256, 256, 64) causal 182 / 135, (32, 1024, 128)
    // causal 541 / 523, (32, 512, 128) 287 / 231, (128, 256, 128) causal 213 / 168.
    {
        const long long g128 = (long long)BH * ((S + 127) / 128);
        const int cus = num_cus();
        const bool small = D <= 64 ? (CAUSAL ? g128 <= cus || (g128 <= 2LL * cus && S >= 2048)
                                             : g128 < cus)
                                   : (CAUSAL ? g128 < cus : 2 * g128 < cus);
        // buffer offsets (bytes, up to 16 rows past S) fit an int
        if (small && (long long)(S + 32) * D * 4 <= INT32_MAX) {
            auto kdkdv = bwd_dkdv_f32_s16_kernel<D, CAUSAL>;
            const size_t lds_kv = (size_t)S16_W * 2 * 16 * (D + 4) * sizeof(float);
            static bool done_kv = false;
            DH_TRY(set_lds(kdkdv, lds_kv, done_kv));
            kdkdv<<<BH * ((S + 15) / 16), 64 * S16_W, lds_kv, stream()>>>(
                BH, S, scale, sl2, (const float*)Q, (const float*)K, (const float*)V,
                (const float*)dO, LSE, Dv, dK, dV, acc, kv_alias);
            DH_TRY(check_launch("dh_flash_bwd(dK,dV f32, 16-row)"));
            auto kdq = bwd_dq_f32_s16_kernel<D, CAUSAL>;
            const size_t lds_q = (size_t)S16_W * 16 * (D + 4) * sizeof(float);
            static bool done_q = false;
            DH_TRY(set_lds(kdq, lds_q, done_q));
            kdq<<<BH * ((S + 15) / 16), 64 * S16_W, lds_q, stream()>>>(
                BH, S, scale, sl2, (const float*)Q, (const float*)K, (const float*)V,
                (const float*)dO, LSE, Dv, dQ, acc_q);
            return check_launch("dh_flash_bwd(dQ f32, 16-row)");
        }
    }
    const size_t lds = 2 * 2 * Tl::ELEMS * sizeof(float);
    // D = 128 and 64 grids of at least a round of 128-key dK/dV work-groups: that launch stores
    // scale dS (fp32) for every query row and the keys up to the end of its 128-row tile
    // (causal) or all keys, and dQ_tile (+)= (scale dS_tile) K for every 128-row tile of every
    // slice is one GEMM launch (flash_dq_from_ds_f32, heaviest tiles first) -- one S^2 D product
    // instead of the dQ launch's three (S and dP recomputed, then dS K).  Scratch: 128^2 T
    // (T + 1) / 2 floats per slice causal, (128 T)^2 not (T = ceil(S / 128)), from the pool, at
    // most 8 GB: beyond that the slices run in equal chunks (each dK/dV launch and its dQ launch
    // over one chunk, the scratch reused), each chunk still a round of 128-key tiles; without
    // the memory, or where a chunk would be smaller, the dQ launch below.  Per slice the work
    // is the same whichever chunk holds it, so results do not depend on the chunking.  The dS
    // traffic does not shrink with D while the products do, so D = 32 keeps the dQ launch.
    // Same box, whole backward, recomputing dQ launch -> stored dS: config 4's shape 16.85 ->
    // 12.5-12.7 ms, (64, 2048, 128) causal 2.23 -> 1.68 ms, (64, 1024, 128) 1.05 -> 0.85 ms,
    // (32, 4096, 128) causal 4.14 -> 3.11 ms, (8, 4096, 128) non-causal 2.05 -> 1.54 ms,
    // (1, 32768, 128) causal 15.9 -> 11.7 ms; (128, 2048, 64) causal 2.31 -> 1.95 ms,
    // (64, 1024, 64) causal 0.44 -> 0.32 ms, (128, 1024, 64) 1.09 -> 0.93 ms.
    if constexpr (D == 128 || D == 64) {
        static const int ds_knob = [] {
            const char* e = std::getenv("DH_FLASH_BWD_F32_DS");   // tuning knob: 0 or 1
            return e ? std::atoi(e) : 1;
        }();
        static const long long ds_cap = [] {
            const char* e = std::getenv("DH_FLASH_BWD_F32_DS_CAP");   // tuning knob: bytes
            return e ? std::atoll(e) : 8LL << 30;
        }();
        if (allow_ds && ds_knob && f32_waves(BH, S, 16) == 8) {
            const long long T = (S + 127) / 128;
            const long long slice = CAUSAL ? 8192LL * T * (T + 1) : 16384LL * T * T;
            // nch chunks of BH / nch or one more slices (at most `per`, the cap's worth)
            const long long per = ds_cap / (slice * (long long)sizeof(float));
            const int nch = per > 0 ? (int)((BH + per - 1) / per) : 0;
            const int small = nch > 0 ? BH / nch : 0, big = nch > 0 ? (BH + nch - 1) / nch : 0;
            float* dS = nch > 0 && (long long)small * T >= num_cus()
                            ? static_cast<float*>(dh_malloc((size_t)(slice * big) * sizeof(float)))
                            : nullptr;
            if (dS) {
                const size_t lds_ds = lds + (size_t)2 * RB * (128 + 4) * sizeof(float);
                int st = DH_OK;
                for (int c = 0, b0 = 0; st == DH_OK && c < nch; ++c) {
                    const int nb = small + (c < BH % nch ? 1 : 0);
                    const size_t eo = (size_t)b0 * S * D, ro = (size_t)b0 * S;
                    const float* Kc = (const float*)K + eo;
                    st = launch_dkdv_f32<D, CAUSAL, 8, true>(
                        nb, S, scale, sl2, (const float*)Q + eo, Kc, (const float*)V + eo,
                        (const float*)dO + eo, LSE + ro, Dv + ro, dK + eo, dV + eo, acc, kv_alias,
                        lds_ds, dS, slice);
                    if (st == DH_OK)
                        st = flash_dq_from_ds_f32(nb, S, D, CAUSAL, dS, slice, Kc,
                                                  acc_q ? 1.f : 0.f, dQ + eo);
                    b0 += nb;
                }
                dh_free(dS);   // pooled; later users of the buffer are ordered on the stream
                return st;
            }
        }
    }
    // dK/dV: 16 keys per wave (8 waves, 128 keys, when that grid fills the CUs).
    switch (f32_waves(BH, S, 16)) {
    case 8: DH_TRY((launch_dkdv_f32<D, CAUSAL, 8>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dK, dV, acc, kv_alias, lds))); break;
    case 4: DH_TRY((launch_dkdv_f32<D, CAUSAL, 4>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dK, dV, acc, kv_alias, lds))); break;
    case 2: DH_TRY((launch_dkdv_f32<D, CAUSAL, 2>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dK, dV, acc, kv_alias, lds))); break;
    default: DH_TRY((launch_dkdv_f32<D, CAUSAL, 1>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dK, dV, acc, kv_alias, lds)));
    }
    // dQ: 32 queries per wave (8 waves, two per SIMD, on 256-query tiles when that grid fills
    // the CUs, continued down to 1 wave; as in the fp32 forward, non-causal grids take 8 waves
    // from 5/8 of a round: same box, whole backward (48, 1024, 128) 1.052 -> 1.035 ms,
    // (40, 1024, 64) 0.542 -> 0.504, (60, 1024, 32) 0.314 -> 0.283, (40, 1536, 128) 1.540 ->
    // 1.513).
    const bool nc8 = !CAUSAL && 8LL * BH * ((S + 255) / 256) >= 5LL * num_cus();
    switch (nc8 ? 8 : f32_waves(BH, S, 32)) {
    case 8: return launch_dq_f32<D, CAUSAL, 8>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dQ, acc_q, lds);
    case 4: return launch_dq_f32<D, CAUSAL, 4>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dQ, acc_q, lds);
    case 2: return launch_dq_f32<D, CAUSAL, 2>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dQ, acc_q, lds);
    default: return launch_dq_f32<D, CAUSAL, 1>(BH, S, scale, sl2, Q, K, V, dO, LSE, Dv, dQ, acc_q, lds);
    }
}

template <typename T, int D>
int run_dvec(int rows, const void* O, const void* dO, float* Dv) {
    // eight work-groups (32 waves) per CU, each striding over 16-row groups
    const int groups = (rows + NT / 16 - 1) / (NT / 16);
    const int grid = groups < 8 * num_cus() ? groups : 8 * num_cus();
    dvec_kernel<T, D><<<grid, NT, 0, stream()>>>(rows, (const T*)O, (const T*)dO, Dv);
    return check_launch("dh_flash_bwd(Dvec)");
}

template <int D>
int dispatch(int dtype, int causal, int BH, int S, float scale, const void* Q, const void* K,
             const void* V, const void* O, const void* dO, const float* LSE, float* Dv,
             float* dQ, float* dK, float* dV, int acc, int kv_alias, int acc_q, int allow_ds) {
    const int rows = BH * S;
    if (dtype == DH_BF16) {
        float* L2 = Dv + rows;                       // second half of the scratch
        return causal ? run_bf16<D, true>(BH, S, scale, Q, K, V, O, dO, LSE, L2, Dv, dQ, dK, dV, acc)
                      : run_bf16<D, false>(BH, S, scale, Q, K, V, O, dO, LSE, L2, Dv, dQ, dK, dV, acc);
    }
    DH_TRY((run_dvec<float, D>(rows, O, dO, Dv)));
    return causal ? run_f32<D, true>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc, kv_alias, acc_q, allow_ds)
                  : run_f32<D, false>(BH, S, scale, Q, K, V, dO, LSE, Dv, dQ, dK, dV, acc, kv_alias, acc_q, allow_ds);
}

}  // namespace
}  // namespace dh

using namespace dh;

namespace {

// Argument checks shared by the entry points.  Any two of dQ, dK, dV may be the same buffer
// (one tensor passed as two or three of Q, K, V); buffers that overlap without being equal are
// rejected.
int check_bwd_args(int dtype, int BH, int S, int D, const void* Q, const void* K,
                   const void* V, const void* O, const void* dO, const float* LSE,
                   const float* dQ, const float* dK, const float* dV) {
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
    const uintptr_t bytes = (uintptr_t)BH * S * D * sizeof(float);
    const float* g[3] = {dQ, dK, dV};
    for (int a = 0; a < 3; ++a)
        for (int b = a + 1; b < 3; ++b) {
            const uintptr_t x = (uintptr_t)g[a], y = (uintptr_t)g[b];
            if (x != y && x < y + bytes && y < x + bytes)
                return set_error(DH_ERR_INVALID,
                                 "dh_flash_bwd: gradient buffers overlap without being equal");
        }
    return DH_OK;
}

// The launches over caller-supplied scratch Dv (BH*S floats, twice that for bf16).  fp32: the
// dK/dV launch runs before the dQ launch on the same stream, so a dQ buffer shared with dK or
// dV accumulates onto what that launch stored; bf16: the other way round (run_bf16).
int run_bwd(int dtype, int BH, int S, int D, float scale, int causal, const void* Q,
            const void* K, const void* V, const void* O, const void* dO, const float* LSE,
            float* dQ, float* dK, float* dV, int accumulate, float* Dv, int allow_ds) {
    const int kv_alias = dK == dV;
    const int acc_q = accumulate || dQ == dK || dQ == dV;
    if (D == 128)
        return dispatch<128>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV,
                             accumulate, kv_alias, acc_q, allow_ds);
    if (D == 64)
        return dispatch<64>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV,
                            accumulate, kv_alias, acc_q, allow_ds);
    return dispatch<32>(dtype, causal, BH, S, scale, Q, K, V, O, dO, LSE, Dv, dQ, dK, dV,
                        accumulate, kv_alias, acc_q, allow_ds);
}

}  // namespace

extern "C" int dh_flash_bwd(int dtype, int BH, int S, int D, float scale, int causal,
                            const void* Q, const void* K, const void* V, const void* O,
                            const void* dO, const float* LSE, float* dQ, float* dK, float* dV,
                            int accumulate) {
    DH_TRY(ensure_init());
    DH_TRY(check_bwd_args(dtype, BH, S, D, Q, K, V, O, dO, LSE, dQ, dK, dV));
    if (BH == 0 || S == 0) return DH_OK;
    // Scratch from the pool: Dvec (BH*S floats) and, for bf16, LSE*log2(e) (BH*S floats);
    // returned to the pool once the work is queued (later users of the buffer are ordered
    // after these kernels on the same stream).
    float* Dv = (float*)dh_malloc((size_t)BH * S * sizeof(float) * (dtype == DH_BF16 ? 2 : 1));
    if (!Dv) return DH_ERR_OOM;
    const int st = run_bwd(dtype, BH, S, D, scale, causal, Q, K, V, O, dO, LSE, dQ, dK, dV,
                           accumulate, Dv, 1);
    dh_free(Dv);
    return st;
}

// ---------------------------------------------------------------------------------
// dh_flash_bwd_noalloc: the same launches over a fixed device array instead of pool
// memory, for callers that cannot allocate (code under graph capture, serving loops).
// ---------------------------------------------------------------------------------
namespace {

// Dvec (BH*S floats) and, for bf16, LSE*log2(e) (BH*S more) of one call: 8 MB, held by every
// device the library runs on until the process ends.
constexpr size_t kNoAllocRows = size_t(1) << 20;
static __device__ __align__(256) float scratch[2 * kNoAllocRows];

// Device address of `scratch`, looked up once per device with that device current.  The
// host-side name `scratch` is only a stand-in for the symbol and is never passed to a kernel.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_addr[kMaxDevices] = {};

int scratch_address(float** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess)
        return set_error(DH_ERR_HIP, "dh_flash_bwd_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(DH_ERR_UNSUPPORTED, "dh_flash_bwd_noalloc: device %d", dev);
    std::lock_guard<std::mutex> g(g_scratch_mu);
    if (!g_scratch_addr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(DH_ERR_HIP, "dh_flash_bwd_noalloc: hipGetSymbolAddress: %s",
                             hipGetErrorString(e));
        g_scratch_addr[dev] = static_cast<float*>(p);
    }
    *out = g_scratch_addr[dev];
    return DH_OK;
}

}  // namespace

extern "C" int dh_flash_bwd_noalloc(int dtype, int BH, int S, int D, float scale, int causal,
                                    const void* Q, const void* K, const void* V, const void* O,
                                    const void* dO, const float* LSE, float* dQ, float* dK,
                                    float* dV, int accumulate) {
    DH_TRY(ensure_init());
    if (BH > 0 && S > 0 && (size_t)BH * (size_t)S > kNoAllocRows)
        return set_error(DH_ERR_INVALID,
                         "dh_flash_bwd_noalloc: BH*S = %zu rows exceeds the %zu-row scratch",
                         (size_t)BH * (size_t)S, kNoAllocRows);
    DH_TRY(check_bwd_args(dtype, BH, S, D, Q, K, V, O, dO, LSE, dQ, dK, dV));
    if (BH == 0 || S == 0) return DH_OK;
    float* Dv = nullptr;
    DH_TRY(scratch_address(&Dv));
    // Every Dvec / LSE*log2(e) entry the later launches read is written earlier in this call
    // (by the Dvec launch, or for bf16 by the dQ launch), so nothing is cleared.
    // (no pool memory here: the fp32 dQ launch recomputes dS instead of storing it)
    return run_bwd(dtype, BH, S, D, scale, causal, Q, K, V, O, dO, LSE, dQ, dK, dV, accumulate,
                   Dv, 0);
}
