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
//   registers for the whole kernel.  All grids but non-causal ones past six rounds of the
//   CUs take 4-wave work-groups (128 rows, two per CU) with two-slot K and V rings instead.
// fp32 kernel (v_mfma_f32_32x32x2_f32): 32 rows per wave, K and V both [key][d] in a
//   two-stage LDS ring filled through registers; 8 waves (two per SIMD, 256 rows) when that
//   grid fills the chip (non-causal: 5/8 of it), else 4 (128 rows); small grids take
//   16-row work-groups whose 8 waves split the key range, on v_mfma_f32_16x16x4_f32 with K
//   and V read straight into registers.
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
constexpr int BF_NSTAGE = 4;                // 8-wave LDS ring depth, in stages of BN keys

// One stage = a K tile then a V tile, each BN key rows of D bf16 kept row-major, moved
// by direct-to-LDS DMA in 1 KB blocks (64 lanes x 16 bytes).  The 16-byte chunk c of key
// row j sits at position c ^ swz(j) of its row:
//  K is read with b128 (16 consecutive rows of one chunk per LDS pass): kswz spreads those
//    rows over all 64 banks;
//  V is read with ds_read_b64_tr_b16 (4 consecutive rows x 64 bytes per pass): vswz
//    spreads those 4 rows over all 64 banks.
template <int D, int W>
struct BfTile {
    static constexpr int CH = D / 8;                  // 16-byte chunks per key row
    static constexpr int ROWB = 2 * D;                // bytes per key row
    static constexpr int TILE = BN * ROWB;            // bytes of one K (or V) tile
    static constexpr int STAGE = 2 * TILE;
    static constexpr int NBLK = TILE / 1024;          // DMA blocks per tile
    static constexpr int RPB = 1024 / ROWB;           // key rows per DMA block
    static constexpr int PER = 2 * NBLK / W;          // DMA blocks per wave per stage
    static constexpr int RW = 256 / ROWB;             // key rows per 256-byte bank sweep
    static_assert(PER >= 1 && 2 * NBLK == PER * W, "stage must split over the waves");
    // Ring layout.  8 waves: BF_NSTAGE slots of one K and one V tile, refilled 3 stages
    // ahead.  4 waves (two work-groups per CU, 64 KB each): two K slots, then two V slots;
    // after barrier st the waves refill K(st + 2) into K(st)'s slot (last read by step
    // st - 1, which formed the scores of st) and V(st + 1) into V(st - 1)'s slot.
    static constexpr int LDS = W == 8 ? BF_NSTAGE * STAGE : 4 * TILE;
    __device__ static uint32_t kslot(int st) {
        return W == 8 ? (st % BF_NSTAGE) * STAGE : (st & 1) * TILE;
    }
    __device__ static uint32_t vslot(int st) {
        return W == 8 ? (st % BF_NSTAGE) * STAGE + TILE : (2 + (st & 1)) * TILE;
    }
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

// Work-group -> (slice bh, q-tile rank rr; rank 0 = longest causal key range), by
// slice_group_order: each XCD walks its slices G at a time (G = 4 causal slices hold enough
// work that the last, longest tiles of a group do not trail), heaviest q-tile first within a
// group, so the slices in flight keep their K and V in the XCD's L2.  A grid of exactly
// BH n_qt work-groups with 8 not dividing BH is the rank-major fallback (slice_grouping).
template <bool CAUSAL>
__device__ inline void bf_order(int BH, int n_qt, int& bh, int& rr) {
    const int bid = blockIdx.x;
    if ((BH & 7) && (long long)gridDim.x == (long long)BH * n_qt) {
        bh = bid % BH;
        rr = bid / BH;
        return;
    }
    slice_group_order(bid, BH, n_qt, CAUSAL ? 4 : 1, bh, rr);
}

// One work-group = W waves x 32 query rows.  Per stage of 64 keys a wave computes
// S^T = K Q^T (2 x D/16 MFMAs, K from LDS, Q from registers), the online softmax on its
// 32 scores per lane, and O^T += V^T P^T (2 x 2 x D/32 MFMAs, V through transpose reads,
// P straight from the score registers).  The running max m is kept on raw scores (scale
// > 0), so p = exp2(s * sl2 - m * sl2) is one FMA and one exp; the row sum l is taken
// over the bf16-rounded p that the PV product uses (v_dot2_f32_bf16 with (1, 1)), per
// lane half, and combined once at the end.
template <int D, bool CAUSAL, int W>
__global__ void __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(2, 2)))
flash_fwd_bf16_kernel(int BH, int S, float sl2, const uint16_t* __restrict__ Q,
                      const uint16_t* __restrict__ K, const uint16_t* __restrict__ V,
                      uint16_t* __restrict__ O, float* __restrict__ LSE) {
    using T = BfTile<D, W>;
    constexpr int NTK = D / 16, ND = D / 32, ROWS = 32 * W;
    extern __shared__ __attribute__((aligned(1024))) uint8_t ring[];

    const int n_qt = (S + ROWS - 1) / ROWS;
    int bh, rr;
    bf_order<CAUSAL>(BH, n_qt, bh, rr);
    if (bh < 0) return;                  // padding of an XCD with one slice fewer
    const int qt = CAUSAL ? n_qt - 1 - rr : rr;
    const int q0 = qt * ROWS;
    const size_t base = (size_t)bh * S * D;
    const uint16_t* Qg = Q + base;
    const uint16_t* Kg = K + base;
    const uint16_t* Vg = V + base;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int r0 = q0 + 32 * wave;                 // first query row of this wave
    const uint32_t ring_lds = lds_addr(ring);

    const int kend = CAUSAL ? min(S, q0 + ROWS) : S;
    const int nst = (kend + BN - 1) / BN;
    // DMA work of this wave: blocks wave, wave + W, ... of the stage (K tile first).
    // Loads go through a buffer resource per stage (base = key row j0, range = the rows
    // left in the slice), so each lane's byte offset is loop-invariant and rows at or past
    // S arrive as zeros (masked keys; zero V rows meet p = 0).
    uint32_t dlds[T::PER], dvoff[T::PER];
    bool dk[T::PER];
#pragma unroll
    for (int q = 0; q < T::PER; ++q) {
        const int gb = wave + W * q;
        const int tile = gb / T::NBLK, b = gb % T::NBLK;
        const int row = b * T::RPB + lane / T::CH, pos = lane % T::CH;
        dk[q] = tile == 0;
        dlds[q] = b * 1024;
        dvoff[q] = row * T::ROWB + 16 * (pos ^ (tile == 0 ? T::kswz(row) : T::vswz(row)));
    }
    // DMA block q (of K stage sk or V stage sv) into its ring slot.  A stage at or past nst
    // is never computed: its slot is free, and the load re-reads key rows from 0 (in bounds,
    // cached) so that callers need no branch.
    auto issue_one = [&](int sk, int sv, int q) {
        const int st = dk[q] ? sk : sv;
        const int j0 = st < nst ? st * BN : 0;
        const uint32_t sb = ring_lds + (dk[q] ? T::kslot(st) : T::vslot(st));
        const u32x4 rs = make_rsrc((dk[q] ? Kg : Vg) + (size_t)j0 * D, (uint32_t)(S - j0) * T::ROWB);
        lds_dma16_buf(dvoff[q], rs, __builtin_amdgcn_readfirstlane(sb + dlds[q]));
    };
    auto issue = [&](int sk, int sv) {
#pragma unroll
        for (int q = 0; q < T::PER; ++q) issue_one(sk, sv, q);
    };
    // stages refilled after barrier st
    auto ahead_k = [](int st) { return W == 8 ? st + BF_NSTAGE - 1 : st + 2; };
    auto ahead_v = [](int st) { return W == 8 ? st + BF_NSTAGE - 1 : st + 1; };

    // Q fragments (B operand of S^T = K Q^T): lane (i, h) holds Q[i][16t + 8h .. +7]; loaded
    // in the prologue below.
    bf16x8 qf[NTK];
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

    // stages this wave computes: none if all its rows are padding, else up to its diagonal
    const int wlast = r0 >= S ? 0 : CAUSAL ? min(S - 1, r0 + 31) / BN + 1 : nst;

    // Software pipeline, per wave and stage st (scores of st already in `cur`, masked,
    // with their row max):
    //   A  lazy-rescale decision for st (rarely taken branch);
    //   B  S(st+1) = K(st+1) Q^T on the matrix cores while the VALU exponentiates st;
    //   C  O^T += V^T P^T for st, then the mask and row max of st+1 (whose VALU work
    //      overlaps the last PV MFMAs in flight).  B and C form one basic block.
    // Stage st+1 must therefore be in LDS at barrier st; the DMA stays 3 stages ahead in
    // the 4-slot ring (the slot refilled after barrier st last held stage st-1).  B and C
    // run unconditionally: past the last stage they read a stale, in-bounds ring slot and
    // the result is discarded.
    auto sync = [&](int st) {
        // stages <= st + 1 must have landed; st + 2 may still be in flight (8 waves; with
        // 4, everything issued a step ago is needed now)
        if (W == 8 && st + 2 < nst) wait_vmcnt<T::PER>();
        else wait_vmcnt<0>();
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        __builtin_amdgcn_s_barrier();
    };
    auto scores = [&](int st, f32x16 (&sacc)[2]) {
        const uint8_t* kt = ring + T::kslot(st);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) sacc[kb][r] = 0.f;
#pragma unroll
        for (int t = 0; t < NTK; ++t)
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(kt + kofs[t] + 32 * kb * T::ROWB);
                sacc[kb] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[t], sacc[kb], 0, 0, 0);
            }
    };
    // sacc[kb][r] = S^T[key st*BN + 32 kb + 8 (r / 4) + 4 h + r % 4][row r0 + l32]
    auto mask = [&](int st, f32x16 (&sacc)[2]) {
        const int j0 = st * BN;
        if (j0 + BN - 1 > (CAUSAL ? r0 : S - 1)) {        // wave-uniform: diagonal or tail
            const int rel = lim - j0 - 4 * h;             // mask offsets above rel
#pragma unroll
            for (int kb = 0; kb < 2; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (32 * kb + 8 * (r >> 2) + (r & 3) > rel) sacc[kb][r] = -INFINITY;
        }
    };
    auto rowmax = [&](const f32x16 (&sacc)[2]) {      // max over this lane's 32 scores
        float t8[8];
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const f32x16& a = sacc[q >> 2];
            const int o = 4 * (q & 3);
            t8[q] = fmaxf(fmaxf(a[o], a[o + 1]), fmaxf(a[o + 2], a[o + 3]));
        }
        return fmaxf(fmaxf(fmaxf(t8[0], t8[1]), fmaxf(t8[2], t8[3])),
                     fmaxf(fmaxf(t8[4], t8[5]), fmaxf(t8[6], t8[7])));
    };
    auto rescale = [&](float mx) {
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
    };
    // B and C for stage st, interleaved by hand: sched_barrier(0) between chunks fixes
    // the issue order, and fragment reads are issued ahead of their MFMA by hand.  An MFMA
    // holds the SIMD's issue port about as long as two VALU ops and an exponential as
    // long as two, so the VALU work is spread to keep each chunk near one MFMA's time:
    //   B: chunk i issues score MFMA i of stage st+1 (i = 2 t + kb), the exponentials of
    //      pairs [QB i / NS, QB (i+1) / NS) of stage st, and this wave's DMA share of stage
    //      st+3 (one block every other chunk);
    //   C: chunk j issues PV MFMA j of stage st (j = (2 kb + kk) ND + d); its first chunks
    //      exponentiate the remaining pairs (each before the PV MFMA that consumes it), the
    //      later ones take the bf16 row sums (dot2) and, after the mask of st+1, the row max
    //      of st+1, which is returned.
    auto overlap = [&](int st, const f32x16 (&cur)[2], f32x16 (&nxt)[2]) -> float {
        constexpr int NS = 2 * NTK;            // score MFMAs per stage
        constexpr int NP = 4 * ND;             // PV MFMAs per stage
        constexpr int QB = D == 128 ? 10 : D == 64 ? 12 : 16;   // pairs exponentiated in B
        constexpr int J0 = 16 - QB;            // first C chunk free of exponentials
        constexpr int KPF = 4;                 // K fragments in flight
        const uint8_t* kt = ring + T::kslot(st + 1);
        const uint8_t* vt = ring + T::vslot(st);
        auto kfrag = [&](int i) {
            return *reinterpret_cast<const bf16x8*>(kt + kofs[i >> 1] + 32 * (i & 1) * T::ROWB);
        };
        // V fragment of PV MFMA j: keys 32 kb + 16 kk + 4 h + (0..3) and + 8 (see vofs).
        auto vread = [&](int j, s16x4 (&a)[2]) {
            const int d = j % ND, kk = (j / ND) & 1, kb = j / (2 * ND);
            const uint8_t* vk = vt + (32 * kb + 16 * kk) * T::ROWB + vofs[d];
            a[0] = ds_read_tr(reinterpret_cast<const uint16_t*>(vk));
            a[1] = ds_read_tr(reinterpret_cast<const uint16_t*>(vk + 8 * T::ROWB));
        };
        const float mb = m * sl2;
        uint32_t pk[16];                       // pk[8 kb + r / 2] = bf16 pair (r, r + 1) of cur[kb]
        auto expo = [&](int q) {
            const f32x16& c = cur[q >> 3];
            const int r = 2 * (q & 7);
            const float p0 = fast_exp2(__builtin_fmaf(c[r], sl2, -mb));
            const float p1 = fast_exp2(__builtin_fmaf(c[r + 1], sl2, -mb));
            pk[q] = cvt_pk_bf16(p0, p1);
            asm volatile("" : "+v"(pk[q]));    // keep it in this chunk (no sinking)
        };
        bf16x8 kf[KPF];
        s16x4 va[3][2];
#pragma unroll
        for (int i = 0; i < KPF; ++i) kf[i] = kfrag(i);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) nxt[kb][r] = 0.f;
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < NS; ++i) {
            nxt[i & 1] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[i % KPF], qf[i >> 1],
                                                                 nxt[i & 1], 0, 0, 0);
            if (i + KPF < NS) kf[i % KPF] = kfrag(i + KPF);
            else if (i + KPF - NS < 2) vread(i + KPF - NS, va[i + KPF - NS]);
#pragma unroll
            for (int q = QB * i / NS; q < QB * (i + 1) / NS; ++q) expo(q);
            if ((i & 1) && (i >> 1) < T::PER) issue_one(ahead_k(st), ahead_v(st), i >> 1);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int q = NS / 2; q < T::PER; ++q) issue_one(ahead_k(st), ahead_v(st), q);
        float tmax[8];
#pragma unroll
        for (int j = 0; j < NP; ++j) {
            if (j == NP / 2) {
                mask(st + 1, nxt);
                __builtin_amdgcn_sched_barrier(0);
            }
            const int d = j % ND, q0 = 4 * (j / ND);
            const bf16x8 pf = __builtin_bit_cast(bf16x8, u32x4{pk[q0], pk[q0 + 1], pk[q0 + 2], pk[q0 + 3]});
            const s16x4(&a)[2] = va[j % 3];
            const bf16x8 vf = __builtin_bit_cast(
                bf16x8, s16x8{a[0][0], a[0][1], a[0][2], a[0][3], a[1][0], a[1][1], a[1][2], a[1][3]});
            oacc[d] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf, oacc[d], 0, 0, 0);
            if (j + 2 < NP) vread(j + 2, va[(j + 2) % 3]);
            if (j < J0) expo(QB + j);
            if (j >= J0) {
#pragma unroll
                for (int q = 16 * (j - J0) / (NP - J0); q < 16 * (j - J0 + 1) / (NP - J0); ++q)
                    l = dot2_bf16(pk[q], 0x3F803F80u, l);
                asm volatile("" : "+v"(l));
            }
            if (j >= NP / 2) {
                constexpr int MPC = 8 / (NP / 2);     // partial maxima per chunk
#pragma unroll
                for (int u = 0; u < MPC; ++u) {
                    const int q = (j - NP / 2) * MPC + u;
                    const f32x16& a4 = nxt[q >> 2];
                    const int o = 4 * (q & 3);
                    tmax[q] = fmaxf(fmaxf(a4[o], a4[o + 1]), fmaxf(a4[o + 2], a4[o + 3]));
                    asm volatile("" : "+v"(tmax[q]));
                }
            }
            __builtin_amdgcn_sched_barrier(0);
        }
        return fmaxf(fmaxf(fmaxf(tmax[0], tmax[1]), fmaxf(tmax[2], tmax[3])),
                     fmaxf(fmaxf(tmax[4], tmax[5]), fmaxf(tmax[6], tmax[7])));
    };
    auto step = [&](int st, f32x16 (&cur)[2], f32x16 (&nxt)[2], float mx_cur) -> float {
        sync(st);
        if (st >= wlast) {                     // no rows left here: only the DMA share
            issue(ahead_k(st), ahead_v(st));
            return 0.f;
        }
        rescale(mx_cur);
        return overlap(st, cur, nxt);
    };

    // Prologue: the first stages' DMA, then the Q rows, so that the two fetches overlap (Q
    // comes from HBM; with the Q wait first, a work-group spent both latencies in series).
    if constexpr (W == 8) {
#pragma unroll
        for (int st = 0; st < BF_NSTAGE - 1; ++st)
            if (st < nst) issue(st, st);
    } else {
        static_assert(W == 8 || T::NBLK % 4 == 0, "4 waves: blocks q < PER / 2 are K's");
        issue(0, 0);                                    // K(0), V(0)
#pragma unroll
        for (int q = 0; q < T::PER / 2; ++q) issue_one(1, 0, q);   // K(1)
    }
    {   // the Q fragments
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
    // (The compiler's wait for Q above is a full vmcnt(0): it cannot count the DMA, so the
    // stages issued before the Q loads have landed too.)
    wait_vmcnt<0>();
    __builtin_amdgcn_s_barrier();
    f32x16 sa[2], sb[2];
    float mx = 0.f;
    if (wlast > 0) {
        scores(0, sa);
        mask(0, sa);
        mx = rowmax(sa);
    }
    for (int st = 0; st < nst; st += 2) {
        mx = step(st, sa, sb, mx);
        if (st + 1 < nst) mx = step(st + 1, sb, sa, mx);
    }
    // The last steps' look-ahead blocks (re-reads past the last stage) land before the
    // work-group can end and its LDS go to another one; issued a stage ago, they have.
    wait_vmcnt<0>();

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
template <int D, int THREADS = NT>
struct F32Stage {
    static constexpr int LS = D + 4;                  // row stride (floats)
    static constexpr int ELEMS = BN * LS;
    static constexpr int CH = BN * D / 4 / THREADS;   // float4 chunks per thread per tensor
    f32x4 k[CH], v[CH];

    // The stage's base (uniform) plus a 32-bit unsigned offset per thread: scalar-base loads
    // instead of a 64-bit address per thread kept across stages.
    __device__ void fetch(const float* __restrict__ Kg, const float* __restrict__ Vg, int j0,
                          int S, int tid) {
        const float* ks = Kg + (size_t)j0 * D;
        const float* vs = Vg + (size_t)j0 * D;
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int f = tid + c * THREADS;
            const int key = f / (D / 4), dq = f % (D / 4);
            const uint32_t o = key * D + 4 * dq;
            const f32x4 z = {0.f, 0.f, 0.f, 0.f};
            k[c] = j0 + key < S ? *reinterpret_cast<const f32x4*>(ks + o) : z;
            v[c] = j0 + key < S ? *reinterpret_cast<const f32x4*>(vs + o) : z;
        }
    }
    __device__ void store(float* ks, float* vs, int tid) const {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int f = tid + c * THREADS;
            const int key = f / (D / 4), dq = f % (D / 4);
            *reinterpret_cast<f32x4*>(&ks[key * LS + 4 * dq]) = k[c];
            *reinterpret_cast<f32x4*>(&vs[key * LS + 4 * dq]) = v[c];
        }
    }
};

// WAVES = 8: two waves per SIMD on one 256-row tile (the other wave fills each one's
// softmax and barrier gaps; each K/V stage feeds twice the rows; 250 VGPRs at D = 128).
// WAVES = 4: one wave per SIMD on 128 rows, for grids the 256-row tiles would leave short of
// one round of the CUs.
template <int D, bool CAUSAL, int WAVES>
__global__ void __launch_bounds__(64 * WAVES) __attribute__((amdgpu_waves_per_eu(WAVES / 4, WAVES / 4)))
flash_fwd_f32_kernel(int BH, int S, float scale_log2, const float* __restrict__ Q,
                     const float* __restrict__ K, const float* __restrict__ V,
                     float* __restrict__ O, float* __restrict__ LSE) {
    using St = F32Stage<D, 64 * WAVES>;
    constexpr int ROWS_WG = 32 * WAVES, ND = D / 32, NDQ = D / 4;
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
    // The Q rows (qf) have landed on every path into the stage loop.  store(0)'s wait covers
    // them only where a stage exists; without this wait the compiler's wait insertion cannot
    // tell them from the loop's own loads and made each stage's first MFMA wait for the next
    // stage's prefetch.  The builtin (vmcnt(0), expcnt and lgkmcnt untouched), unlike inline
    // assembly, is seen by that pass.
    __builtin_amdgcn_s_waitcnt(0x0F70);
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
        // Lazy rescaling, as in the bf16 kernel: the running max m moves (and O, l are
        // rescaled) only when some row of the wave sees a block max above m + RESCALE_TH;
        // p = exp2(s - m) <= 2^RESCALE_TH otherwise.  The first stage always moves it.
        if (__any(mx > m + RESCALE_TH)) {                // wave-uniform
            mx = fmaxf(mx, xor32(mx));
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
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float p = fast_exp2(sacc[kb][r] - m);
                sacc[kb][r] = p;
                sum += p;
            }
        sum += xor32(sum);
        l += sum;
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

// fp32, small grids on 16-row work-groups (config 3: 24 slices of 256 rows).  A short problem
// is a chain of latencies per work-group (Q rows, K/V, the two products, the merge, the
// stores), so its time is set by the longest chain, not by the matrix cores' throughput.  A
// work-group owns 16 query rows and its 8 waves take 16- or 32-key chunks round-robin (wave
// w: chunks w, w + 8, ...), on v_mfma_f32_16x16x4_f32, with K and V read straight from
// global memory into the operand registers (no LDS staging, no barrier in the loop): the
// heaviest config-3 work-group runs one 32-key chunk per wave, 64 MFMAs of 2048 flops.
// MFMA layouts (16 x 16 x 4: lane l supplies A[l % 16][l / 16] and B[l / 16][l % 16]; result
// register r is D[4 (l / 16) + r][l % 16]); c = l % 16, g = l / 16:
//  S^T = K Q^T: k-step s pairs K[key][d] with Q[query][d] for d = D/4 g + s (the order of d
//    inside the contraction is free as long as both operands agree), so a lane loads D/4
//    consecutive floats of one Q row and of one K row; result register r of key block kb is
//    the score of key k0 + 16 kb + 4 g + r for query q0 + c.
//  O^T += V^T P^T: k-step (kb, r) takes key k0 + 16 kb + 4 g + r at lane group g -- exactly
//    the key whose probability the lane holds in that score register, so P is used in place;
//    the V operand of d-block e at lane (c, g) is V[that key][D/16 c + e], one vector load of
//    D/16 floats per key row.  Result register r of d-block e is O^T[D/16 (4 g + r) + e][q0 + c].
// The row max and sum run over the four lane groups with two lane swaps.  Every chunk a wave
// processes holds a valid key for each of its rows (chunk starts are multiples of the chunk
// width at or below the block's first row), so no running max stays at the mask value; waves
// without a chunk hold m = NEG, l = 0, O = 0 and drop out of the merge (2^(NEG - M) = 0).
// The merge is spread over all 512 threads: 32 per row, each adding the 8 partials of D/32
// columns in wave order.
template <int D>
struct F32S16Cfg {
    static constexpr int W = 8;                        // waves per work-group
    static constexpr int CK = D == 128 ? 16 : 32;      // keys per chunk
    static constexpr int NKB = CK / 16;                // 16-key blocks per chunk
    static constexpr int DQ = D / 4;                   // Q / K floats per lane (k-steps)
    static constexpr int DV = D / 16;                  // V floats per lane per key (d-blocks)
    static constexpr int RS = D + 4;                   // merge row stride (floats)
    static constexpr int PART = 16 * RS + 32;          // one wave's O rows, then m[16], l[16]
    static constexpr int LDS_FLOATS = W * PART;
};

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(64 * F32S16Cfg<D>::W)
flash_fwd_f32_s16_kernel(int BH, int S, float scale_log2, const float* __restrict__ Q,
                         const float* __restrict__ K, const float* __restrict__ V,
                         float* __restrict__ O, float* __restrict__ LSE) {
    using Cfg = F32S16Cfg<D>;
    constexpr int W = Cfg::W, CK = Cfg::CK, NKB = Cfg::NKB, DQ = Cfg::DQ, DV = Cfg::DV;
    constexpr int RS = Cfg::RS, PART = Cfg::PART;
    extern __shared__ __attribute__((aligned(16))) float fsm[];

    const int n_qb = (S + 15) / 16;
    const int bh = blockIdx.x % BH;
    const int rr = blockIdx.x / BH;
    const int qb = CAUSAL ? n_qb - 1 - rr : rr;          // longest key range first
    const int q0 = qb * 16;
    const size_t base = (size_t)bh * S * D;
    const float* Kg = K + base;
    const float* Vg = V + base;

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int c = lane & 15, g = lane >> 4;
    const int qi = q0 + c;                               // this lane's query row

    float qf[DQ];
    load_floats(Q + base + (size_t)min(qi, S - 1) * D + DQ * g, qf);
    f32x4 oacc[DV];
#pragma unroll
    for (int e = 0; e < DV; ++e) oacc[e] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = NEG, l = 0.f;

    const int kend = CAUSAL ? min(S, q0 + 16) : S;
    const int nch = (kend + CK - 1) / CK;
    // K and V of chunk ch into the operand registers.  K rows past S read row S - 1 (their
    // scores are masked); V rows come through a buffer resource over the slice, which returns
    // zeros past it -- no select on the loaded values, so nothing waits for a load before its
    // use.  The next chunk's K is loaded once the score MFMAs have read kf, its V once the PV
    // MFMAs have read vf, so each load overlaps the other half of the chunk.
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(Vg), 0, 4 * S * D, 0x00020000);
    float kf[NKB][DQ], vf[NKB][4][DV];
    auto load_k = [&](int ch) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
            load_floats(Kg + (size_t)min(ch * CK + 16 * kb + c, S - 1) * D + DQ * g, kf[kb]);
    };
    auto load_v = [&](int ch) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
                buf_load_floats(rs, 4 * ((ch * CK + 16 * kb + 4 * g + r) * D + DV * c), vf[kb][r]);
    };
    if (wave < nch) {
        load_k(wave);
        load_v(wave);
    }
    for (int ch = wave; ch < nch; ch += W) {
        const int k0 = ch * CK;
        const bool more = ch + W < nch;
        // two accumulators per key block (even and odd k-steps) halve the dependent chain
        f32x4 sa[NKB][2];
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) sa[kb][0] = sa[kb][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int st = 0; st < DQ; ++st)
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
                sa[kb][st & 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[kb][st], qf[st],
                                                                    sa[kb][st & 1], 0, 0, 0);
        if (more) load_k(ch + W);
        float p[NKB][4];
        float mx = NEG;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int j = k0 + 16 * kb + 4 * g + r;
                float sc = (sa[kb][0][r] + sa[kb][1][r]) * scale_log2;
                if (j >= S || (CAUSAL && j > qi)) sc = NEG;
                p[kb][r] = sc;
                mx = fmaxf(mx, sc);
            }
        float lo, hi;
        halves16(mx, lo, hi);
        mx = fmaxf(lo, hi);
        halves32(mx, lo, hi);
        mx = fmaxf(lo, hi);
        const float m_new = fmaxf(m, mx);
        const float corr = fast_exp2(m - m_new);
        m = m_new;
        float sum = 0.f;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[kb][r] = fast_exp2(p[kb][r] - m_new);
                sum += p[kb][r];
            }
        halves16(sum, lo, hi);
        sum = lo + hi;
        halves32(sum, lo, hi);
        sum = lo + hi;
        l = l * corr + sum;
#pragma unroll
        for (int e = 0; e < DV; ++e) oacc[e] *= corr;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int e = 0; e < DV; ++e)
                    oacc[e] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[kb][r][e], p[kb][r], oacc[e],
                                                                   0, 0, 0);
        if (more) load_v(ch + W);
    }

    // Merge: each wave parks O^T (lane (c, g): columns D/4 g .. D/4 g + D/4 of row c), m, l.
    float* const part = fsm + wave * PART;
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
        for (int e = 0; e < DV; ++e) part[c * RS + DV * (4 * g + r) + e] = oacc[e][r];
    if (g == 0) {
        part[16 * RS + c] = m;
        part[16 * RS + 16 + c] = l;
    }
    __syncthreads();
    constexpr int TPR = 64 * W / 16;                     // threads per row
    constexpr int CPT = D / TPR;                         // columns per thread
    static_assert(CPT >= 1 && D % TPR == 0, "columns per thread");
    const int row = tid / TPR, col = (tid % TPR) * CPT;
    const int i = q0 + row;
    if (i >= S) return;
    float mw[W], M = NEG;
#pragma unroll
    for (int w = 0; w < W; ++w) {
        mw[w] = fsm[w * PART + 16 * RS + row];
        M = fmaxf(M, mw[w]);
    }
    float acc[CPT], L = 0.f;
#pragma unroll
    for (int e = 0; e < CPT; ++e) acc[e] = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
        const float sc = fast_exp2(mw[w] - M);
        L += sc * fsm[w * PART + 16 * RS + 16 + row];
#pragma unroll
        for (int e = 0; e < CPT; ++e) acc[e] += sc * fsm[w * PART + row * RS + col + e];
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    float* orow = O + base + (size_t)i * D + col;
#pragma unroll
    for (int e = 0; e < CPT; ++e) orow[e] = acc[e] * inv;
    if (col == 0) LSE[(size_t)bh * S + i] = (M + __log2f(L)) * 0.69314718055994531f;
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

template <int D, bool CAUSAL, int W>
int launch_bf16_w(int BH, int S, float sl2, const void* Q, const void* K, const void* V, void* O,
                  float* LSE) {
    auto kern = flash_fwd_bf16_kernel<D, CAUSAL, W>;
    const size_t lds = BfTile<D, W>::LDS;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
    const int n_qt = (S + 32 * W - 1) / (32 * W);
    const long long grid = slice_grouping(BH) ? slice_grid(BH, n_qt) : (long long)BH * n_qt;
    kern<<<(unsigned)grid, 64 * W, lds, stream()>>>(BH, S, sl2, (const uint16_t*)Q,
                                                   (const uint16_t*)K, (const uint16_t*)V,
                                                   (uint16_t*)O, LSE);
    return check_launch("dh_flash_fwd(bf16)");
}

template <int D, bool CAUSAL>
int launch_bf16(int BH, int S, float sl2, const void* Q, const void* K, const void* V, void* O,
                float* LSE) {
    // 4-wave work-groups (two per CU): twice the work-groups, and each CU's two run their
    // prologues and epilogues apart.  Same box, 8-wave / 4-wave time: 1.5 to 6 rounds of the
    // CUs 1.00-1.16 (D = 64: 1.09-1.11); at 8 rounds causal 1.003-1.007, non-causal
    // 0.986-0.999, where the doubled K/V staging per row takes back what the overlap gives.
    // So 8-wave work-groups only for non-causal grids past six rounds.
    if (!CAUSAL && (long long)BH * ((S + 255) / 256) > 6LL * num_cus())
        return launch_bf16_w<D, CAUSAL, 8>(BH, S, sl2, Q, K, V, O, LSE);
    return launch_bf16_w<D, CAUSAL, 4>(BH, S, sl2, Q, K, V, O, LSE);
}

template <int D, bool CAUSAL>
int launch_f32(int BH, int S, float sl2, const void* Q, const void* K, const void* V, void* O,
               float* LSE) {
    const int grid = BH * ((S + 127) / 128);
    // Small problems: 16-row work-groups whose 8 waves split the key range (grids of under
    // half a round of 128-row tiles; causal ones under a round, or of one round with S >= 1024,
    // where the 128-row tiles' uneven key ranges leave most CUs waiting on the longest ones).
    // Same box, 16-row kernel against the tiled kernels (us): causal (16, 2048, 64) 120 / 184,
    // (32, 1024, 128) 131 / 168, (8, 4096, 128) 372 / 620, (64, 256, 64) 18.0 / 29.4,
    // (32, 768, 64) 47.6 / 73.7, (40, 512, 128) 54.5 / 88.7; kept tiled: (128, 256, 64) causal
    // 35 / 31, non-causal (32, 1024, 64) 120 / 107, (100, 256, 64) 38.5 / 32.8, and (64, 1024,
    // 64) causal 153 / 154.
    const int cus = num_cus();
    if ((long long)(S + 32) * D * 4 <= INT32_MAX &&   // V's buffer offsets (bytes) fit an int
        (2 * grid < cus || (CAUSAL && (grid < cus || (grid == cus && S >= 1024))))) {
        auto kern = flash_fwd_f32_s16_kernel<D, CAUSAL>;
        const size_t lds = (size_t)F32S16Cfg<D>::LDS_FLOATS * sizeof(float);
        static bool done_s16 = false;
        DH_TRY(set_lds(kern, lds, done_s16));
        kern<<<BH * ((S + 15) / 16), 64 * F32S16Cfg<D>::W, lds, stream()>>>(
            BH, S, sl2, (const float*)Q, (const float*)K, (const float*)V, (float*)O, LSE);
        return check_launch("dh_flash_fwd(f32, 16-row)");
    }
    // 256-row tiles on 8 waves when they fill at least one round of the CUs (config 4's
    // shape: 5.48 -> 4.53 ms, same box), else 128-row tiles on 4 waves.
    const size_t lds = 4 * F32Stage<D>::ELEMS * sizeof(float);
    // 8 waves when their grid fills the CUs, and for non-causal grids from 5/8 of a round
    // (same box, 8-wave against 4-wave at 0.62-0.94 rounds: (48, 1024, 128) 0.290 / 0.343 ms,
    // (40, 1024, 64) 0.160 / 0.196, (60, 1024, 32) 0.101 / 0.131; at half a round, and for
    // causal grids under one round, 4 waves stay faster: (32, 1024, 32) 0.096 / 0.065,
    // (64, 520, 128) causal 0.144 / 0.089).
    const int grid8 = BH * ((S + 255) / 256);
    if (grid8 >= num_cus() || (!CAUSAL && 8 * grid8 >= 5 * num_cus())) {
        auto kern = flash_fwd_f32_kernel<D, CAUSAL, 8>;
        static bool done8 = false;
        DH_TRY(set_lds(kern, lds, done8));
        kern<<<grid8, 512, lds, stream()>>>(BH, S, sl2, (const float*)Q, (const float*)K,
                                            (const float*)V, (float*)O, LSE);
        return check_launch("dh_flash_fwd(f32, 8 waves)");
    }
    auto kern = flash_fwd_f32_kernel<D, CAUSAL, 4>;
    static bool done = false;
    DH_TRY(set_lds(kern, lds, done));
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
