// dh_gemm_f32.hip -- fp32 GEMM on the gfx950 matrix cores (v_mfma_f32_32x32x2_f32).
//
// C[M x N] = op(A) @ op(B) + beta * C for the four storage layouts (NN, NT, TN, TT), optionally
// batched (strided operands, gridDim.y = batch member) and with a bias + ReLU epilogue.
// NN serves tensor_matmul's C = A @ B (runtime/ops/elementwise.inc:971-1213); NT and TN
// with beta = 1 serve the matmul backward dA += dY B^T, dB += A^T dY
// (runtime/ops/autograd.inc:91-125).  NT with the bias (+ ReLU) epilogue is dream_linear /
// linear_relu's Y = X W^T + b (elementwise.inc:1432-1516); batched NN is dream_bmm
// (elementwise.inc:1218-1252).
//
// Work decomposition
//   work-group (256 threads = 4 wave64s) owns a 128 x 128 tile of C (64 x 256 or 256 x 64
//   when M or N is at most 64); each wave owns a 64 x 64 sub-tile: 2 x 2 MFMA blocks of
//   32 x 32, 64 fp32 accumulators per lane.
//   K advances in slices of 16: both operand slices are staged in LDS k-major
//   (As[k][i], Bs[k][j]) and double-buffered; the next slice is fetched from global
//   memory into registers while the matrix cores work on the current one.
// MFMA operand layout (32x32x2): lane l supplies A[i = l % 32][k = l / 32] and
//   B[k = l / 32][j = l % 32]; accumulator register r of lane l holds
//   C[8 * (r / 4) + 4 * (l / 32) + r % 4][l % 32].
// Edges: rows/cols beyond M, N and K are loaded as zeros and never stored, so any
//   shape is exact.  When a matrix's leading dimension and base address allow it the
//   contiguous dimension is fetched with 128-bit loads.
#include <type_traits>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int BK = 16, NTHREADS = 256;

// Four consecutive elements of one row of a row-major matrix:
// row r, columns c..c+3 of a rows x cols matrix with leading dimension ld.
// VEC: 16-byte aligned rows and cols % 4 == 0, so a chunk (c % 4 == 0) is wholly inside or
// outside; an outside chunk then reads 16 zero bytes (g_zero4) instead.  The load is
// branch-free and nothing touches its result before the LDS store, so the wait for it can
// sit there (a select or branch on the value would force the wait right after the load).
__device__ __attribute__((aligned(16))) float g_zero4[4];   // zero-initialised, never written

template <bool VEC>
__device__ inline f32x4 load4(const float* __restrict__ p, int ld, int rows, int cols, int r,
                              int c) {
    f32x4 v = {0.f, 0.f, 0.f, 0.f};
    if (VEC) {
        const bool in = r < rows && c < cols;
        return *reinterpret_cast<const f32x4*>(in ? p + (size_t)r * ld + c : g_zero4);
    }
    if (r >= rows) return v;
    const float* q = p + (size_t)r * ld + c;
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (c + e < cols) v[e] = q[e];
    return v;
}

// Operand slice loader.  "Contiguous-k" operands (A in NN/NT, B in NT/TT) are read
// along k and transposed into the k-major LDS tile; the others are copied row by row.
// TILE = tile extent along the non-k dimension (64, 128 or 256).  The k-major LDS rows are
// padded by 4 floats, which puts the 4 k-rows a transposing store of a 16-wide slice touches
// 16 banks apart (conflict-free); an MFMA operand read (k-rows k and k + 1 in the two lane
// halves) overlaps on 28 banks.  An XOR swizzle like store_swz's for these tiles measured +1%
// at 4096^3 but -3% for 64 x 512^3 batched products: it breaks the paired ds_read2 /
// ds_write2 forms the padded layout gets.
template <bool KCONTIG, bool VEC, int TILE, int BKT = BK, int NT = NTHREADS>
struct Slice {
    static constexpr int CH = TILE * BKT / 4 / NT;   // float4 per thread per slice
    f32x4 v[CH];

    // base/ld describe the stored matrix; t0 = first index along the tile dimension,
    // k0 = first k; extent_t / extent_k bound the valid region.
    __device__ void fetch(const float* __restrict__ base, int ld, int t0, int k0, int extent_t,
                          int extent_k, int tid) {
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int f = tid + r * NT;
            if (KCONTIG) {   // stored [t][k]: 4 k per float4
                const int t = f / (BKT / 4), kq = f % (BKT / 4);
                v[r] = load4<VEC>(base, ld, extent_t, extent_k, t0 + t, k0 + 4 * kq);
            } else {         // stored [k][t]: 4 t per float4
                const int k = f / (TILE / 4), tq = f % (TILE / 4);
                v[r] = load4<VEC>(base, ld, extent_k, extent_t, k0 + k, t0 + 4 * tq);
            }
        }
    }
    __device__ void store(float* lds, int stride, int tid) const {
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int f = tid + r * NT;
            if (KCONTIG) {
                const int t = f / (BKT / 4), kq = f % (BKT / 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) lds[(4 * kq + e) * stride + t] = v[r][e];
            } else {
                const int k = f / (TILE / 4), tq = f % (TILE / 4);
                *reinterpret_cast<f32x4*>(&lds[k * stride + 4 * tq]) = v[r];
            }
        }
    }
    // The same copy into a 64-wide, unpadded k-major tile whose element (k, t) sits at
    // k * 64 + swz64(k, t): for 32-wide slices (8 float4 per row of a k-contiguous operand) the
    // padded layout puts rows kq and kq + 4 of a transposing store on the same banks, and the
    // two k-rows of an MFMA operand read (lanes 0-31 row k, 32-63 row k + 1) on overlapping
    // ones.  swz64 flips bit 5 of t on odd k (the two rows of a read fall in opposite bank
    // halves) and bits 3-5 by (k / 4) % 8 (the 8 k-quads of a store on distinct banks); it
    // keeps runs of 4 aligned t together, so the row copies stay 16-byte stores.
    __device__ static int swz64(int k, int t) { return t ^ (32 * (k & 1)) ^ (8 * ((k >> 2) & 7)); }
    __device__ void store_swz(float* lds, int tid) const {
        static_assert(TILE == 64, "64-wide tiles");
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int f = tid + r * NT;
            if (KCONTIG) {
                const int t = f / (BKT / 4), kq = f % (BKT / 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 4 * kq + e;
                    lds[k * 64 + swz64(k, t)] = v[r][e];
                }
            } else {
                const int k = f / (TILE / 4), tq = f % (TILE / 4);
                *reinterpret_cast<f32x4*>(&lds[k * 64 + swz64(k, 4 * tq)]) = v[r];
            }
        }
    }
};

// One work-group tile TBM x TBN of C (128 x 128, or 64 x 256 / 256 x 64 for products with M
// or N at most 64) at the origin tile_of(m0, n0) sets; the 4 waves tile it in 64 x 64
// sub-tiles.
template <bool TA, bool TB, bool VA, bool VB, int TBM, int TBN, typename TileOf>
__device__ __forceinline__ void gemm_f32_tile(int M, int N, int K, const float* __restrict__ A,
                                              int lda, const float* __restrict__ B, int ldb,
                                              float beta, float* __restrict__ C, int ldc,
                                              const float* __restrict__ bias, int epi,
                                              TileOf tile_of) {
    constexpr int LDS_A = TBM + 4, LDS_B = TBN + 4;   // padded k-major row strides (floats)
    // Wave sub-tile WT x WT: 64 (2 x 2 MFMA blocks) for the 128 x 128 / 64 x 256 / 256 x 64
    // tiles, 32 (one block) for 64 x 64 tiles.
    constexpr int WT = TBM == 64 && TBN == 64 ? 32 : 64, NB = WT / 32;
    constexpr int WN = TBN / WT;                        // waves along N
    static_assert((TBM / WT) * WN == 4, "4 waves");
    __shared__ __attribute__((aligned(16))) float As[2][BK * LDS_A];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDS_B];

    int m0, n0;
    tile_of(m0, n0);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = (wave / WN) * WT, wn = (wave % WN) * WT;

    // A: op(A)[i][k]; stored [i][k] when !TA (k contiguous), [k][i] when TA.
    // B: op(B)[k][j]; stored [k][j] when !TB (j contiguous), [j][k] when TB.
    // Two register sets: slice kt + 2 is fetched while slice kt is computed and slice kt + 1
    // waits in the other set, so a load has two slices' compute to land -- with one or two
    // work-groups per CU (small products, split-K chunks) nothing else hides it.
    Slice<!TA, VA, TBM> sa[2];
    Slice<TB, VB, TBN> sb[2];

    f32x16 acc[NB][NB];
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    // The loop is branch-free so the compiler's wait for a slice's loads can sit at its LDS
    // store, two slices later (with a guarded fetch it waited for every load right away):
    // fetches are unconditional (a slice at or past K reads zeros) and the slice count is
    // taken up to an even number (a zero slice adds nothing).  fp32 4096^3: 1.26 -> 1.15 ms.
    const int nk = (K + BK - 1) / BK;
    if (nk > 0) {
        sa[0].fetch(A, lda, m0, 0, M, K, tid);
        sb[0].fetch(B, ldb, n0, 0, N, K, tid);
        sa[1].fetch(A, lda, m0, BK, M, K, tid);
        sb[1].fetch(B, ldb, n0, BK, N, K, tid);
        sa[0].store(As[0], LDS_A, tid);
        sb[0].store(Bs[0], LDS_B, tid);
        __syncthreads();
    }
    auto mma = [&](const float* as, const float* bs) {   // one k-slice from LDS
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float av[NB], bv[NB];
#pragma unroll
            for (int x = 0; x < NB; ++x) {
                av[x] = as[(kk + h) * LDS_A + wm + 32 * x + l32];
                bv[x] = bs[(kk + h) * LDS_B + wn + 32 * x + l32];
            }
#pragma unroll
            for (int a = 0; a < NB; ++a)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    };
    // One k-slice of the loop; the register set index is a template constant (a runtime
    // index would put both sets in scratch).
    auto step = [&](auto cur_c, int kt) {
        constexpr int cur = decltype(cur_c)::value;
        // set cur held slice kt, already in LDS: refill it with slice kt + 2
        sa[cur].fetch(A, lda, m0, (kt + 2) * BK, M, K, tid);
        sb[cur].fetch(B, ldb, n0, (kt + 2) * BK, N, K, tid);
        mma(As[cur], Bs[cur]);
        // slice kt + 1, fetched an iteration ago (past the last slice: unread zeros)
        sa[cur ^ 1].store(As[cur ^ 1], LDS_A, tid);
        sb[cur ^ 1].store(Bs[cur ^ 1], LDS_B, tid);
        __syncthreads();
    };
    if (nk == 1) {   // one slice (tiny K): no loop, no zero slice
        mma(As[0], Bs[0]);
    } else {
        for (int kt = 0; kt < nk; kt += 2) {
            step(std::integral_constant<int, 0>{}, kt);
            step(std::integral_constant<int, 1>{}, kt + 1);
        }
    }

    // Epilogue: lanes 0..31 of a register cover 32 consecutive columns of one row.
    // C = acc + beta C + bias (bias[col], or bias[row] with DH_EPI_ROW_BIAS), then max(., 0)
    // with DH_EPI_RELU (NaN passes, like `y < 0 ? 0 : y`).
    const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS), relu = epi & DH_EPI_RELU;
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int col = n0 + wn + 32 * b + l32;
            if (col >= N) continue;
            const float bv = bias && !row_bias ? bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < M) {
                    float* c = C + (size_t)row * ldc + col;
                    float v = (beta == 0.f ? acc[a][b][r] : acc[a][b][r] + beta * *c) +
                              (row_bias ? bias[row] : bv);
                    if (relu) v = v < 0.f ? 0.f : v;
                    *c = v;
                }
            }
        }
}

// The kernel body: batch member blockIdx.y (strides in elements; 0 for a single product).  In
// a split-K launch the members are the chunks of K, and the last one takes the ragged rest,
// k_last (= K otherwise).
template <bool TA, bool TB, bool VA, bool VB, int TBM, int TBN>
__device__ __forceinline__ void gemm_f32_grid_tile(int M, int N, int K, const float* __restrict__ A,
                                                   int lda, const float* __restrict__ B, int ldb,
                                                   float beta, float* __restrict__ C, int ldc,
                                                   long long sA, long long sB, long long sC,
                                                   const float* __restrict__ bias, int epi,
                                                   int k_last) {
    if (blockIdx.y == gridDim.y - 1) K = k_last;
    A += blockIdx.y * sA;
    B += blockIdx.y * sB;
    C += blockIdx.y * sC;
    gemm_f32_tile<TA, TB, VA, VB, TBM, TBN>(M, N, K, A, lda, B, ldb, beta, C, ldc, bias, epi,
                                            [&](int& m0, int& n0) {
        const int tiles_m = (M + TBM - 1) / TBM, tiles_n = (N + TBN - 1) / TBN;
        int tm, tn;
        xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 8, tm, tn);
        m0 = tm * TBM;
        n0 = tn * TBN;
    });
}

template <bool TA, bool TB, bool VA, bool VB, int TBM, int TBN>
__global__ void __launch_bounds__(NTHREADS)
gemm_f32_kernel(int M, int N, int K, const float* __restrict__ A, int lda,
                const float* __restrict__ B, int ldb, float beta, float* __restrict__ C, int ldc,
                long long sA, long long sB, long long sC, const float* __restrict__ bias,
                int epi, int k_last) {
    gemm_f32_grid_tile<TA, TB, VA, VB, TBM, TBN>(M, N, K, A, lda, B, ldb, beta, C, ldc, sA, sB, sC,
                                                bias, epi, k_last);
}

// The 128 x 128 tile held to four waves per SIMD (at most 128 registers a lane: the
// accumulators move to arch VGPRs), so that four work-groups share a CU where the default form
// fits three (94 VGPRs + 64 accumulation registers).  For grids of at least four tiles per CU:
// same box, fp32 4096^3 NN 1.080 -> 1.055 ms, TN 1.094-1.099 -> 1.062-1.066, 8192 x 8192 x 2048
// 1-3% faster; with fewer tiles per CU the default form is faster (2048^3, one per CU: 175 ->
// 184 us; 3000^3 NN 520 -> 535-543 us).
template <bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(NTHREADS)
__attribute__((amdgpu_waves_per_eu(4, 4)))
gemm_f32_occ4_kernel(int M, int N, int K, const float* __restrict__ A, int lda,
                     const float* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                     int ldc, long long sA, long long sB, long long sC,
                     const float* __restrict__ bias, int epi, int k_last) {
    gemm_f32_grid_tile<TA, TB, VA, VB, 128, 128>(M, N, K, A, lda, B, ldb, beta, C, ldc, sA, sB, sC,
                                                bias, epi, k_last);
}

// dQ of the fp32 flash backward from stored scale*dS (one launch for all row tiles), head
// dimension D = 128 or 64: query tile t of slice bh is dQ[bh][128 t .. +rows][0..D) (+)= dS_t
// K[bh][0..kk), where dS_t (rows x kk, row stride len) starts at dS + bh slice + off: causal
// len = 128 (t + 1), off = 8192 t (t + 1) (tile t's rows hold the keys up to the tile's end);
// otherwise len = 128 T, off = 128 t len; kk = min(len, S).  A work-group takes a TM x D block
// of it (TM = 128 at D = 128; two 64 x 64 blocks per tile at D = 64); the tiles go heaviest
// first, and consecutive work-groups take consecutive slices, so with BH a multiple of 8 each
// XCD reads the K rows of its own slices.
template <bool VA, bool VB, int D>
__global__ void __launch_bounds__(NTHREADS)
flash_dq_from_ds_kernel(int BH, int S, int T, int causal, const float* __restrict__ dS,
                        long long slice, const float* __restrict__ Kr, float beta,
                        float* __restrict__ dQ) {
    constexpr int TM = D == 128 ? 128 : 64, R = 128 / TM;   // R row blocks per query tile
    const int bh = blockIdx.x % BH, q = blockIdx.x / BH;
    const int t = T - 1 - q / R, r = q % R;
    const int rows = (S - 128 * t < 128 ? S - 128 * t : 128) - TM * r;
    if (rows <= 0) return;   // the second block of a short last tile
    const int len = causal ? 128 * (t + 1) : 128 * T;
    const int kk = len < S ? len : S;
    const long long off = (causal ? 8192LL * t * (t + 1) : 128LL * t * len) + (long long)TM * r * len;
    const size_t sd = (size_t)bh * S * D;
    gemm_f32_tile<false, false, VA, VB, TM, D>(rows < TM ? rows : TM, D, kk, dS + bh * slice + off,
                                               len, Kr + sd, D, beta,
                                               dQ + sd + (size_t)(128 * t + TM * r) * D, D, nullptr, 0,
                                               [](int& m0, int& n0) { m0 = n0 = 0; });
}

// 64 x 64 tiles with two waves per SIMD: for grids of about one work-group per CU (config 1's
// 1024^3, a layer's forward) one wave per SIMD leaves the matrix core idle across each
// slice's LDS stores, barrier and fragment reads.  Here 8 waves share a 64 x 64 tile: 32-wide
// k-slices, waves w and w + 4 own the same 32 x 32 block and take the slice's first and second
// 16 k; at the end waves 4..7 hand their sums to waves 0..3 through LDS (fixed order), which
// run the epilogue.  PF slices are in flight from global memory at a time (register sets):
// 4 for long K (config 1: 1.5-3.5% faster than 2 in two same-box A/Bs), 2 otherwise, since the
// loop runs in groups of PF slices and the zero slices past K in a last group cost products.
constexpr int KS_NT = 512, KS_BK = 32;

template <bool TA, bool TB, bool VA, bool VB, int PF>
__global__ void __launch_bounds__(KS_NT)
gemm_f32_ks_kernel(int M, int N, int K, const float* __restrict__ A, int lda,
                   const float* __restrict__ B, int ldb, float beta, float* __restrict__ C, int ldc,
                   long long sA, long long sB, long long sC, const float* __restrict__ bias,
                   int epi) {
    A += blockIdx.y * sA;
    B += blockIdx.y * sB;
    C += blockIdx.y * sC;
    constexpr int T = 64;   // tiles k-major, 64 floats per k-row, swizzled (Slice::swz64)
    __shared__ __attribute__((aligned(16))) float As[2][KS_BK * T];
    __shared__ __attribute__((aligned(16))) float Bs[2][KS_BK * T];

    const int tiles_m = (M + T - 1) / T, tiles_n = (N + T - 1) / T;
    int tm, tn;
    xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * T, n0 = tn * T;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int blk = wave & 3, kh0 = (wave >> 2) * (KS_BK / 2);
    const int wm = (blk >> 1) * 32, wn = (blk & 1) * 32;

    Slice<!TA, VA, T, KS_BK, KS_NT> sa[PF];
    Slice<TB, VB, T, KS_BK, KS_NT> sb[PF];
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.f;

    const int nk = (K + KS_BK - 1) / KS_BK;
    if (nk > 0) {
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            sa[q].fetch(A, lda, m0, q * KS_BK, M, K, tid);
            sb[q].fetch(B, ldb, n0, q * KS_BK, N, K, tid);
        }
        sa[0].store_swz(As[0], tid);
        sb[0].store_swz(Bs[0], tid);
        __syncthreads();
    }
    using SA = Slice<!TA, VA, T, KS_BK, KS_NT>;
    auto mma = [&](const float* as, const float* bs) {   // this wave's half of a k-slice
#pragma unroll
        for (int kk = 0; kk < KS_BK / 2; kk += 2) {
            const int k = kh0 + kk + h;
            const float av = as[k * T + SA::swz64(k, wm + l32)];
            const float bv = bs[k * T + SA::swz64(k, wn + l32)];
            acc = __builtin_amdgcn_mfma_f32_32x32x2f32(av, bv, acc, 0, 0, 0);
        }
    };
    // slice kt: register set kt % PF (refilled with slice kt + PF once stored), LDS buffer
    // kt % 2; slices past K load as zeros, so a last group's extra steps add nothing
    auto step = [&](auto cur_c, int kt) {
        constexpr int cur = decltype(cur_c)::value, nxt = (cur + 1) % PF, lb = cur & 1;
        sa[cur].fetch(A, lda, m0, (kt + PF) * KS_BK, M, K, tid);
        sb[cur].fetch(B, ldb, n0, (kt + PF) * KS_BK, N, K, tid);
        mma(As[lb], Bs[lb]);
        sa[nxt].store_swz(As[lb ^ 1], tid);
        sb[nxt].store_swz(Bs[lb ^ 1], tid);
        __syncthreads();
    };
    if (nk == 1) {
        mma(As[0], Bs[0]);
        __syncthreads();
    } else {
        for (int kt = 0; kt < nk; kt += PF) {
            step(std::integral_constant<int, 0>{}, kt);
            step(std::integral_constant<int, 1>{}, kt + 1);
            if constexpr (PF == 4) {
                step(std::integral_constant<int, 2>{}, kt + 2);
                step(std::integral_constant<int, 3>{}, kt + 3);
            }
        }
    }
    // waves 4..7 -> LDS (lane-major, conflict free; As is free after the loop's last barrier)
    float* red = &As[0][0];
    if (wave >= 4) {
#pragma unroll
        for (int r = 0; r < 16; ++r) red[(blk * 16 + r) * 64 + lane] = acc[r];
    }
    __syncthreads();
    if (wave >= 4) return;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] += red[(blk * 16 + r) * 64 + lane];

    const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS), relu = epi & DH_EPI_RELU;
    const int col = n0 + wn + l32;
    if (col >= N) return;
    const float bcol = bias && !row_bias ? bias[col] : 0.f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int row = m0 + wm + 8 * (r >> 2) + 4 * h + (r & 3);
        if (row < M) {
            float* c = C + (size_t)row * ldc + col;
            float v = (beta == 0.f ? acc[r] : acc[r] + beta * *c) + (row_bias ? bias[row] : bcol);
            if (relu) v = v < 0.f ? 0.f : v;
            *c = v;
        }
    }
}

// ---- conv2d forward as an implicit GEMM ---------------------------------------------
// Y[n][co][p] = sum_r Kn[co][r] col_n[r][p] + bias[co] with col_n[r][p] = X[n][ci][h][w],
// r = (ci KH + kh) KW + kw, p = oh OW + ow, h = oh stride + kh - pad, w = ow stride + kw - pad
// (zero outside the input): the im2col matrix is gathered by the B loader and never stored.
// Rows and columns have their own padding (the data gradient pads by KH - 1 - pad and
// KW - 1 - pad).
struct ConvGeom {
    int Cin, H, W, KH, KW, padh, padw, stride, OH, OW;
    FastDiv f_ow, f_kw, f_khkw;   // division by OW, KW and KH*KW
};

// B slice of the implicit GEMM: rows k0 .. k0 + BK of col_n, columns t0 .. t0 + TILE, laid out
// like Slice<false, ...> (row k, 4 consecutive columns per chunk).  A thread's chunks all sit
// in the same 4 columns (tq = tid % (TILE / 4)) and in rows RSTEP apart, so the columns'
// window origins are computed once per tile and a slice only decomposes its rows.  Every
// element is one 32-bit-offset buffer load of the image's planes: byte offset = 4 (tap term
// of its row + pixel term of its column); a tap outside the input takes an offset past the
// buffer's range, which reads zero.
constexpr uint32_t CONV_OOB = 0xFFFFFFF0u;   // past every image buffer (entries check the size)

template <int TILE>
struct ConvSlice {
    static constexpr int CH = TILE * BK / 4 / NTHREADS;
    static constexpr int RSTEP = NTHREADS / (TILE / 4);
    f32x4 v[CH];
    int hb[4], wb[4];   // oh * stride - pad, ow * stride - pad of the thread's 4 columns
    int pix[4];         // 4 (hb W + wb): the column's part of the byte offset

    __device__ void init(const ConvGeom& g, int t0, int P, int tid) {
        const int tq = tid % (TILE / 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int p = t0 + 4 * tq + e;
            const int oh = (int)fdiv((uint32_t)p, g.f_ow), ow = p - oh * g.OW;
            const int h0 = oh * g.stride - g.padh;
            wb[e] = ow * g.stride - g.padw;
            pix[e] = 4 * (h0 * g.W + wb[e]);
            hb[e] = p < P ? h0 : -(1 << 30);   // a column past P: h < 0
        }
    }
    __device__ void fetch(__amdgpu_buffer_rsrc_t rs, const ConvGeom& g, int R, int k0, int tid) {
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int k = k0 + tid / (TILE / 4) + RSTEP * r;
            const int q = (int)fdiv((uint32_t)k, g.f_kw), kw = k - q * g.KW;
            const int ci = (int)fdiv((uint32_t)k, g.f_khkw), kh = q - ci * g.KH;
            const int tap = 4 * ((ci * g.H + kh) * g.W + kw);
            const bool kin = k < R;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int h = hb[e] + kh, w = wb[e] + kw;
                const bool in = kin && (unsigned)h < (unsigned)g.H && (unsigned)w < (unsigned)g.W;
                const uint32_t off = in ? (uint32_t)(tap + pix[e]) : CONV_OOB;
                v[r][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
            }
        }
    }
    __device__ void store(float* lds, int stride, int tid) const {
#pragma unroll
        for (int r = 0; r < CH; ++r) {
            const int f = tid + r * NTHREADS;
            *reinterpret_cast<f32x4*>(&lds[(f / (TILE / 4)) * stride + 4 * (f % (TILE / 4))]) = v[r];
        }
    }
};

// Work-group tile TBM (output channels) x TBN (output positions of image z0 + blockIdx.y);
// the k-loop is the GEMM kernel's (two register sets, branch-free), A = the kernel matrix
// Cout x R (k contiguous), epilogue: + bias[co] (+ the old Y with accumulate), stored into
// Y's (N, Cout, OH OW) layout.
template <int TBM, int TBN, bool VA>
__global__ void __launch_bounds__(NTHREADS)
conv_fwd_kernel(int Cout, int P, int R, const float* __restrict__ Kn, const float* __restrict__ X,
                ConvGeom g, float* __restrict__ Y, const float* __restrict__ bias, int z0,
                int accumulate) {
    const int n = z0 + blockIdx.y;
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<float*>(X) + (size_t)n * g.Cin * g.H * g.W, 0, (int)(4u * g.Cin * g.H * g.W),
        0x00020000);
    float* Yn = Y + (size_t)n * Cout * P;
    constexpr int LDS_A = TBM + 4, LDS_B = TBN + 4;
    constexpr int WT = TBM == 64 && TBN == 64 ? 32 : 64, NB = WT / 32;   // wave sub-tile
    constexpr int WN = TBN / WT;
    static_assert((TBM / WT) * WN == 4, "4 waves");
    __shared__ __attribute__((aligned(16))) float As[2][BK * LDS_A];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDS_B];

    const int tiles_m = (Cout + TBM - 1) / TBM, tiles_n = (P + TBN - 1) / TBN;
    int tm, tn;
    xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * TBM, n0 = tn * TBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = (wave / WN) * WT, wn = (wave % WN) * WT;

    Slice<true, VA, TBM> sa[2];
    ConvSlice<TBN> sb[2];
    sb[0].init(g, n0, P, tid);
    sb[1].init(g, n0, P, tid);

    f32x16 acc[NB][NB];
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    const int nk = (R + BK - 1) / BK;   // R >= 1
    sa[0].fetch(Kn, R, m0, 0, Cout, R, tid);
    sb[0].fetch(xr, g, R, 0, tid);
    sa[1].fetch(Kn, R, m0, BK, Cout, R, tid);
    sb[1].fetch(xr, g, R, BK, tid);
    sa[0].store(As[0], LDS_A, tid);
    sb[0].store(Bs[0], LDS_B, tid);
    __syncthreads();
    auto mma = [&](const float* as, const float* bs) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float av[NB], bv[NB];
#pragma unroll
            for (int x = 0; x < NB; ++x) {
                av[x] = as[(kk + h) * LDS_A + wm + 32 * x + l32];
                bv[x] = bs[(kk + h) * LDS_B + wn + 32 * x + l32];
            }
#pragma unroll
            for (int a = 0; a < NB; ++a)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    };
    auto step = [&](auto cur_c, int kt) {
        constexpr int cur = decltype(cur_c)::value;
        sa[cur].fetch(Kn, R, m0, (kt + 2) * BK, Cout, R, tid);
        sb[cur].fetch(xr, g, R, (kt + 2) * BK, tid);
        mma(As[cur], Bs[cur]);
        sa[cur ^ 1].store(As[cur ^ 1], LDS_A, tid);
        sb[cur ^ 1].store(Bs[cur ^ 1], LDS_B, tid);
        __syncthreads();
    };
    if (nk == 1) {
        mma(As[0], Bs[0]);
    } else {
        for (int kt = 0; kt < nk; kt += 2) {
            step(std::integral_constant<int, 0>{}, kt);
            step(std::integral_constant<int, 1>{}, kt + 1);
        }
    }
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int col = n0 + wn + 32 * b + l32;
            if (col >= P) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < Cout) {
                    float* y = Yn + (size_t)row * P + col;
                    const float v = acc[a][b][r] + (bias ? bias[row] : 0.f);
                    *y = accumulate ? *y + v : v;
                }
            }
        }
}

template <int TBM, int TBN>
int launch_conv(int N, int Cout, int P, int R, const float* Kn, const float* X,
                const ConvGeom& g, float* Y, const float* bias, int accumulate) {
    const bool va = ((uintptr_t)Kn % 16 == 0) && (R % 4 == 0);
    const int tiles = ((Cout + TBM - 1) / TBM) * ((P + TBN - 1) / TBN);
    for (int z0 = 0; z0 < N; z0 += 65535) {
        const dim3 grid(tiles, N - z0 < 65535 ? N - z0 : 65535);
        if (va)
            conv_fwd_kernel<TBM, TBN, true><<<grid, NTHREADS, 0, stream()>>>(Cout, P, R, Kn, X, g, Y, bias, z0, accumulate);
        else
            conv_fwd_kernel<TBM, TBN, false><<<grid, NTHREADS, 0, stream()>>>(Cout, P, R, Kn, X, g, Y, bias, z0, accumulate);
        DH_TRY(check_launch("dh_conv2d"));
    }
    return DH_OK;
}

struct Batch {
    long long sA, sB, sC;
    int count;
    const float* bias;
    int epi;                // DH_EPI_* flags
};

// Split-K reduction: C = beta C + sum_s part[s] (fixed order, so reruns are bit-identical)
// + bias, then ReLU (the DH_EPI_* epilogue).
__global__ void __launch_bounds__(256) splitk_reduce(const float* __restrict__ part, int S, int M,
                                                     int N, float beta, float* __restrict__ C,
                                                     int ldc, const float* __restrict__ bias,
                                                     int epi) {
    const size_t MN = (size_t)M * N;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < MN; e += (size_t)gridDim.x * 256) {
        float v = 0.f;
        for (int s = 0; s < S; ++s) v += part[s * MN + e];
        const int r = (int)(e / N), c = (int)(e % N);
        float* o = C + (size_t)r * ldc + c;
        v = (beta == 0.f ? v : v + beta * *o) + (bias ? bias[(epi & DH_EPI_ROW_BIAS) ? r : c] : 0.f);
        if (epi & DH_EPI_RELU) v = v < 0.f ? 0.f : v;
        *o = v;
    }
}

// ---- conv2d weight gradient as an implicit GEMM ---------------------------------------
// gK[co][r] (+)= sum_n sum_p dY[n][co][p] col_n[r][p]: an NT product whose contraction runs
// over (image, output position).  A = dY_n read in place ([co][p], p contiguous); B = col_n^T
// gathered from X by the loader (the im2col matrix is never stored).  The contraction is cut
// per image into BK-wide slices (an image's last slice padded with zeros) and the slices
// into chunks, one per gridDim.y member, each writing an fp32 partial that splitk_reduce adds
// in a fixed order.

// The thread's rows of B (kernel taps r): chunk c covers tap t0 + f / (BK / 4), f = tid +
// c NTHREADS, at output positions p0 + 4 (f % (BK / 4)) + (0..3) -- its tap and hence the
// input plane and window offset stay fixed across slices.
template <int TILE>
struct ColTGeom {
    static constexpr int CH = TILE * BK / 4 / NTHREADS;
    int tap[CH], dh[CH], dw[CH];    // 4 (ci H W + dh W + dw); kh - padh (-2^30 past R); kw - padw
    __device__ void init(const ConvGeom& g, int R, int t0, int tid) {
#pragma unroll
        for (int c = 0; c < CH; ++c) {
            const int r = t0 + (tid + c * NTHREADS) / (BK / 4);
            const int q = (int)fdiv((uint32_t)r, g.f_kw), kw = r - q * g.KW;
            const int ci = (int)fdiv((uint32_t)r, g.f_khkw), kh = q - ci * g.KH;
            dw[c] = kw - g.padw;
            tap[c] = 4 * ((ci * g.H + kh - g.padh) * g.W + dw[c]);
            dh[c] = r < R ? kh - g.padh : -(1 << 30);
        }
    }
};

// A thread's chunks share their 4 positions (f % (BK / 4) = tid % (BK / 4)), so a slice
// decomposes them once; each element is then one 32-bit-offset buffer load (tap term + pixel
// term; taps outside the input read zero through an offset past the buffer).
template <int TILE>
struct ColTSlice {
    static constexpr int CH = TILE * BK / 4 / NTHREADS;
    f32x4 v[CH];
    // positions p0 .. p0 + BK of the image behind rs; np = number of valid positions (0: zeros)
    __device__ void fetch(__amdgpu_buffer_rsrc_t rs, const ConvGeom& g, const ColTGeom<TILE>& c,
                          int p0, int np, int tid) {
        const int pq = 4 * (tid % (BK / 4));
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const int p = p0 + pq + e;
            const int oh = (int)fdiv((uint32_t)p, g.f_ow), ow = p - oh * g.OW;
            const int hs = oh * g.stride, ws = ow * g.stride;
            const int pix = 4 * (hs * g.W + ws);
            const bool pin = pq + e < np;
#pragma unroll
            for (int k = 0; k < CH; ++k) {
                const int h = hs + c.dh[k], w = ws + c.dw[k];
                const bool in = pin && (unsigned)h < (unsigned)g.H && (unsigned)w < (unsigned)g.W;
                const uint32_t off = in ? (uint32_t)(c.tap[k] + pix) : CONV_OOB;
                v[k][e] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0));
            }
        }
    }
    __device__ void store(float* lds, int stride, int tid) const {   // transposing, as Slice<true>
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int f = tid + k * NTHREADS;
            const int t = f / (BK / 4), kq = f % (BK / 4);
#pragma unroll
            for (int e = 0; e < 4; ++e) lds[(4 * kq + e) * stride + t] = v[k][e];
        }
    }
};

// Work-group: tile TBM (output channels) x TBN (taps) of chunk blockIdx.y, i.e. the slices
// [y chunk, min((y + 1) chunk, total)) of the flattened (image, slice) contraction, nkp
// slices per image.  Writes its partial to part + y Cout R.
template <int TBM, int TBN, bool VA>
__global__ void __launch_bounds__(NTHREADS)
conv_wgrad_kernel(int Cout, int P, int R, const float* __restrict__ dY, const float* __restrict__ X,
                  ConvGeom g, int nkp, int total, int chunk, float* __restrict__ part) {
    const int sbeg = blockIdx.y * chunk;
    const int ns = min(total - sbeg, chunk);          // slices of this chunk (>= 1)
    float* C = part + (size_t)blockIdx.y * Cout * R;
    constexpr int LDS_A = TBM + 4, LDS_B = TBN + 4;
    constexpr int WT = TBM == 64 && TBN == 64 ? 32 : 64, NB = WT / 32;
    constexpr int WN = TBN / WT;
    static_assert((TBM / WT) * WN == 4, "4 waves");
    __shared__ __attribute__((aligned(16))) float As[2][BK * LDS_A];
    __shared__ __attribute__((aligned(16))) float Bs[2][BK * LDS_B];

    const int tiles_m = (Cout + TBM - 1) / TBM, tiles_n = (R + TBN - 1) / TBN;
    int tm, tn;
    xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * TBM, n0 = tn * TBN;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = (wave / WN) * WT, wn = (wave % WN) * WT;
    const size_t plane = (size_t)g.Cin * g.H * g.W;

    ColTGeom<TBN> cg;
    cg.init(g, R, n0, tid);
    Slice<true, VA, TBM> sa[2];
    ColTSlice<TBN> sb[2];
    // slice kt of the chunk: image n, positions p0 ..; past the chunk's end: zeros
    auto fetch = [&](auto set_c, int kt) {
        constexpr int set = decltype(set_c)::value;
        const int s = sbeg + kt;
        const bool live = kt < ns;
        const int n = live ? s / nkp : 0;
        const int p0 = live ? (s - n * nkp) * BK : 0;
        const int np = live ? min(BK, P - p0) : 0;
        sa[set].fetch(dY + (size_t)n * Cout * P, P, m0, p0, Cout, live ? P : 0, tid);
        const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float*>(X) + (size_t)n * plane, 0, (int)(4 * plane), 0x00020000);
        sb[set].fetch(xr, g, cg, p0, np, tid);
    };

    f32x16 acc[NB][NB];
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    fetch(std::integral_constant<int, 0>{}, 0);
    fetch(std::integral_constant<int, 1>{}, 1);
    sa[0].store(As[0], LDS_A, tid);
    sb[0].store(Bs[0], LDS_B, tid);
    __syncthreads();
    auto mma = [&](const float* as, const float* bs) {
#pragma unroll
        for (int kk = 0; kk < BK; kk += 2) {
            float av[NB], bv[NB];
#pragma unroll
            for (int x = 0; x < NB; ++x) {
                av[x] = as[(kk + h) * LDS_A + wm + 32 * x + l32];
                bv[x] = bs[(kk + h) * LDS_B + wn + 32 * x + l32];
            }
#pragma unroll
            for (int a = 0; a < NB; ++a)
#pragma unroll
                for (int b = 0; b < NB; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x2f32(av[a], bv[b], acc[a][b], 0, 0, 0);
        }
    };
    auto step = [&](auto cur_c, int kt) {
        constexpr int cur = decltype(cur_c)::value;
        fetch(cur_c, kt + 2);
        mma(As[cur], Bs[cur]);
        sa[cur ^ 1].store(As[cur ^ 1], LDS_A, tid);
        sb[cur ^ 1].store(Bs[cur ^ 1], LDS_B, tid);
        __syncthreads();
    };
    if (ns == 1) {
        mma(As[0], Bs[0]);
    } else {
        for (int kt = 0; kt < ns; kt += 2) {
            step(std::integral_constant<int, 0>{}, kt);
            step(std::integral_constant<int, 1>{}, kt + 1);
        }
    }
#pragma unroll
    for (int a = 0; a < NB; ++a)
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            const int col = n0 + wn + 32 * b + l32;
            if (col >= R) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < Cout) C[(size_t)row * R + col] = acc[a][b][r];
            }
        }
}

// out = beta out + sum_s part[s] for many partials: wave w of a work-group sums partials
// [w S / 4, (w + 1) S / 4) of 64 consecutive elements, then wave 0 adds the four sums in
// order (fixed order: bit-identical reruns), so four times as many waves share the loads as
// in splitk_reduce's one thread per element.
__global__ void __launch_bounds__(256) partial_sum4(const float* __restrict__ part, int S,
                                                    size_t n, float beta, float* __restrict__ out) {
    __shared__ float red[3][64];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int sb = (int)((long long)S * w / 4), se = (int)((long long)S * (w + 1) / 4);
    for (size_t e0 = (size_t)blockIdx.x * 64; e0 < n; e0 += (size_t)gridDim.x * 64) {
        const size_t e = e0 + lane;
        float v = 0.f;
        if (e < n)
            for (int q = sb; q < se; ++q) v += part[(size_t)q * n + e];
        if (w > 0) red[w - 1][lane] = v;
        __syncthreads();
        if (w == 0 && e < n) {
            v = ((v + red[0][lane]) + red[1][lane]) + red[2][lane];
            out[e] = beta == 0.f ? v : v + beta * out[e];
        }
        __syncthreads();
    }
}

template <int TBM, int TBN>
int launch_wgrad(int N, int Cout, int P, int R, const float* dY, const float* X,
                 const ConvGeom& g, float* dK, int accumulate) {
    const int cus = num_cus();
    const int tiles = ((Cout + TBM - 1) / TBM) * ((R + TBN - 1) / TBN);
    const int nkp = (P + BK - 1) / BK;
    const long long total = (long long)N * nkp;
    // chunks: about 8 work-groups per CU in all, partials within 256 MB, at most 65535
    long long S = 8ll * cus / tiles;
    const long long cap = (64ll << 20) / ((long long)Cout * R);
    S = S < 1 ? 1 : S;
    S = S > cap ? (cap < 1 ? 1 : cap) : S;
    S = S > total ? total : S;
    S = S > 65535 ? 65535 : S;
    const long long chunk = (total + S - 1) / S;
    if (chunk > INT32_MAX || total > INT32_MAX)
        return set_error(DH_ERR_UNSUPPORTED, "dh_conv2d_bwd_filter: contraction too long");
    S = (total + chunk - 1) / chunk;
    float* part = static_cast<float*>(dh_malloc((size_t)S * Cout * R * sizeof(float)));
    if (!part) return set_error(DH_ERR_OOM, "dh_conv2d_bwd_filter: partials");
    const bool va = ((uintptr_t)dY % 16 == 0) && (P % 4 == 0);
    const dim3 grid(tiles, (unsigned)S);
    hipStream_t s = stream();
    if (va)
        conv_wgrad_kernel<TBM, TBN, true><<<grid, NTHREADS, 0, s>>>(Cout, P, R, dY, X, g, nkp, (int)total, (int)chunk, part);
    else
        conv_wgrad_kernel<TBM, TBN, false><<<grid, NTHREADS, 0, s>>>(Cout, P, R, dY, X, g, nkp, (int)total, (int)chunk, part);
    int st = check_launch("dh_conv2d_bwd_filter");
    if (st == DH_OK) {
        const size_t n = (size_t)Cout * R;
        size_t blocks = (n + 63) / 64;
        if (blocks > (size_t)cus * 16) blocks = (size_t)cus * 16;
        partial_sum4<<<(unsigned)blocks, 256, 0, s>>>(part, (int)S, n, accumulate ? 1.f : 0.f, dK);
        st = check_launch("dh_conv2d_bwd_filter(reduce)");
    }
    dh_free(part);   // pooled; later users of the buffer are ordered on the stream
    return st;
}

// wgs: work-groups of a one-pass grid (0 for split-K launches), which takes the four-wave 128 x
// 128 form from four per CU.
template <bool TA, bool TB, int TBM, int TBN>
auto pick_kernel(int M, int N, int K, const float* A, int lda, long long sA, const float* B,
                 int ldb, long long sB, long long wgs = 0) {
    // 128-bit loads need 16-byte aligned bases, leading dimensions and batch strides divisible
    // by 4, and a contiguous extent (K, or M / N for the transposed storage) divisible by 4.
    const int ca = TA ? M : K, cb = TB ? K : N;
    const bool va = ((uintptr_t)A % 16 == 0) && (lda % 4 == 0) && (sA % 4 == 0) && (ca % 4 == 0);
    const bool vb = ((uintptr_t)B % 16 == 0) && (ldb % 4 == 0) && (sB % 4 == 0) && (cb % 4 == 0);
    if constexpr (TBM == 128 && TBN == 128) {
        static const bool occ4 = [] {
            const char* e = std::getenv("DH_GEMM_F32_OCC4");   // tuning knob: 0 or 1
            return !e || std::atoi(e) != 0;
        }();
        if (occ4 && va && vb && wgs >= 4LL * num_cus()) return gemm_f32_occ4_kernel<TA, TB, true, true>;
    }
    return va && vb ? gemm_f32_kernel<TA, TB, true, true, TBM, TBN>
         : va       ? gemm_f32_kernel<TA, TB, true, false, TBM, TBN>
         : vb       ? gemm_f32_kernel<TA, TB, false, true, TBM, TBN>
                    : gemm_f32_kernel<TA, TB, false, false, TBM, TBN>;
}

// One grid of the tiled kernel; gridDim.y carries the batch member, in chunks of 65535 (the
// y limit).
template <bool TA, bool TB, int TBM, int TBN>
int launch_grid(int M, int N, int K, const float* A, int lda, const float* B, int ldb,
                float beta, float* C, int ldc, const Batch& bt) {
    const int tiles = ((M + TBM - 1) / TBM) * ((N + TBN - 1) / TBN);
    auto kern = pick_kernel<TA, TB, TBM, TBN>(M, N, K, A, lda, bt.sA, B, ldb, bt.sB,
                                              (long long)tiles * bt.count);
    for (int b0 = 0; b0 < bt.count; b0 += 65535) {
        const int nb = bt.count - b0 < 65535 ? bt.count - b0 : 65535;
        kern<<<dim3(tiles, nb), NTHREADS, 0, stream()>>>(M, N, K, A + b0 * bt.sA, lda,
                                                         B + b0 * bt.sB, ldb, beta, C + b0 * bt.sC,
                                                         ldc, bt.sA, bt.sB, bt.sC, bt.bias, bt.epi, K);
        DH_TRY(check_launch("dh_gemm_f32"));
    }
    return DH_OK;
}

// One product (bt.count == 1) with K cut into about S chunks (multiples of BK) run as gridDim.y
// members writing fp32 partials, which splitk_reduce adds in order with the epilogue.
// DH_ERR_UNSUPPORTED, with nothing launched, when no workspace can be had.
template <bool TA, bool TB, int TBM, int TBN>
int launch_split_k(int M, int N, int K, int S, const float* A, int lda, const float* B, int ldb,
                   float beta, float* C, int ldc, const Batch& bt) {
    const int tiles = ((M + TBM - 1) / TBM) * ((N + TBN - 1) / TBN);
    hipStream_t s = stream();
    const int Kc = ((K + S - 1) / S + BK - 1) / BK * BK;   // chunk of K, multiple of BK
    S = (K + Kc - 1) / Kc;
    float* part = static_cast<float*>(dh_malloc((size_t)S * M * N * sizeof(float)));
    if (!part) return DH_ERR_UNSUPPORTED;
    // chunk j: A columns (or rows, TA) and B rows (or columns, TB) j Kc .. + Kc; the last
    // chunk K - (S - 1) Kc.  One grid, so the chunks run side by side.  The kernel choice sees
    // the whole K: 16-byte loads along k only where K is a multiple of 4, so that a ragged last
    // chunk has no 4-wide group crossing its end.
    const long long sA = TA ? (long long)Kc * lda : Kc, sB = TB ? Kc : (long long)Kc * ldb;
    auto kern = pick_kernel<TA, TB, TBM, TBN>(M, N, K, A, lda, sA, B, ldb, sB);
    kern<<<dim3(tiles, S), NTHREADS, 0, s>>>(M, N, Kc, A, lda, B, ldb, 0.f, part, N, sA, sB,
                                             (long long)M * N, nullptr, 0, K - (S - 1) * Kc);
    int st = check_launch("dh_gemm_f32(split-K)");
    if (st == DH_OK) {
        const int cus = num_cus();
        size_t blocks = ((size_t)M * N + 255) / 256;
        if (blocks > (size_t)cus * 8) blocks = (size_t)cus * 8;
        splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(part, S, M, N, beta, C, ldc, bt.bias, bt.epi);
        st = check_launch("dh_gemm_f32(split-K reduce)");
    }
    dh_free(part);   // pooled; later users of the buffer are ordered on the stream
    return st;
}

template <bool TA, bool TB, int TBM, int TBN>
int launch_tiles(int M, int N, int K, const float* A, int lda, const float* B, int ldb,
                 float beta, float* C, int ldc, const Batch& bt) {
    const int tm = (M + TBM - 1) / TBM, tn = (N + TBN - 1) / TBN, tiles = tm * tn;
    // Products with few output tiles and a long contraction (the weight gradients dW = dY^T X
    // of a layer, K = the batch; a layer's forward with few output columns) would leave most
    // CUs idle: split K.  Where the one-pass grid fills at most half the CUs, S aims at 4
    // work-groups per CU (measured on config 2's layer shapes: 96 tiles with K = 784, 0.088 ->
    // 0.067 ms; 21 tiles with K = 4096, 0.086 -> 0.061 ms; 1 or 2 per CU gain less).
    const int cus = num_cus();
    if (bt.count == 1 && 2 * tiles <= cus && K >= 512) {
        int S = 4 * cus / tiles;
        S = S > 32 ? 32 : S;
        S = S > K / 128 ? K / 128 : S;
        const int st = launch_split_k<TA, TB, TBM, TBN>(M, N, K, S, A, lda, B, ldb, beta, C, ldc, bt);
        if (st != DH_ERR_UNSUPPORTED) return st;
        // no workspace: the one-pass grid below
    }
    // A partial last round: the matrix cores of a CU are shared by the work-groups it holds,
    // so a grid of F full rounds of the CUs plus a few tiles runs about F + 1 tiles' time
    // (3000^3: 576 tiles of 128 on 256 CUs, 2.25 per CU, take 3).  Cut the output into a
    // part of at most F rounds (whole tile rows, or columns) and a tail strip whose K is
    // split S ways, so that the strip's S-fold grid fits one round of the CUs: the tail then
    // takes about 1/S of a tile's time.  Each part applies beta and the epilogue to its own
    // rows or columns.
    static const bool split_tail = [] {
        const char* e = std::getenv("DH_GEMM_F32_SPLIT_TAIL");   // tuning knob: 0 or 1
        return !e || std::atoi(e) != 0;
    }();
    if (split_tail && TBM == 128 && TBN == 128 && bt.count == 1 && K >= 1024 && tiles > cus &&
        tiles % cus != 0) {
        const int F = tiles / cus;
        // tail strip of r tile rows (cut along M) or tile columns (along N)
        const int rm = tm - F * cus / tn, rn = tn - F * cus / tm;
        const int Sm = rm > 0 && rm < tm ? cus / (rm * tn) : 0;
        const int Sn = rn > 0 && rn < tn ? cus / (rn * tm) : 0;
        int S = Sm >= Sn ? Sm : Sn;
        S = S > K / 256 ? K / 256 : S;
        if (S >= 2) {
            const bool cut_m = Sm >= Sn;
            const int keep = cut_m ? (tm - rm) * TBM : (tn - rn) * TBN;   // rows / columns kept
            Batch tail = bt;   // the strip's epilogue bias, offset where it runs along the cut
            int st;
            if (cut_m) {
                st = launch_grid<TA, TB, TBM, TBN>(keep, N, K, A, lda, B, ldb, beta, C, ldc, bt);
                if (st != DH_OK) return st;
                if (bt.bias && (bt.epi & DH_EPI_ROW_BIAS)) tail.bias = bt.bias + keep;
                const float* At = TA ? A + keep : A + (size_t)keep * lda;
                float* Ct = C + (size_t)keep * ldc;
                st = launch_split_k<TA, TB, TBM, TBN>(M - keep, N, K, S, At, lda, B, ldb, beta, Ct,
                                                     ldc, tail);
                if (st != DH_ERR_UNSUPPORTED) return st;
                return launch_grid<TA, TB, TBM, TBN>(M - keep, N, K, At, lda, B, ldb, beta, Ct, ldc, tail);
            }
            st = launch_grid<TA, TB, TBM, TBN>(M, keep, K, A, lda, B, ldb, beta, C, ldc, bt);
            if (st != DH_OK) return st;
            if (bt.bias && !(bt.epi & DH_EPI_ROW_BIAS)) tail.bias = bt.bias + keep;
            const float* Bt = TB ? B + (size_t)keep * ldb : B + keep;
            float* Ct = C + keep;
            st = launch_split_k<TA, TB, TBM, TBN>(M, N - keep, K, S, A, lda, Bt, ldb, beta, Ct, ldc,
                                                 tail);
            if (st != DH_ERR_UNSUPPORTED) return st;
            return launch_grid<TA, TB, TBM, TBN>(M, N - keep, K, A, lda, Bt, ldb, beta, Ct, ldc, tail);
        }
    }
    return launch_grid<TA, TB, TBM, TBN>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

// ---- skinny products: an output side of at most 16 (min(M, N) <= 16) ----------------------
// Config 2's H W2 (4096 x 10, K 257) and dW2 = H^T dY (257 x 10, K 4096) move a few MB for
// a few MFLOP: HBM- and latency-bound (a launch alone costs ~3.8 us on this stream).  The tiled
// kernels stage 64- or 128-wide tiles through LDS for them and leave most of each tile empty.
// Here a wave owns one 16 x 16 block of D = X Y (X: M x K, Y: K x N as the caller's op(A),
// op(B), or the swapped pair for M <= 16) and streams its K range straight from global memory
// into v_mfma_f32_16x16x4_f32: operand lane l holds X[i0 + l % 16][k] and Y[k][j0 + l % 16].
// The order of k inside a product is free as long as X and Y agree, so in each 16-deep group
// lane l takes k = k0 + 4 (l / 16) + j for MFMA j = 0..3 -- four consecutive k per lane, one
// 16-byte span of a k-contiguous row.  A work-group of 4 waves splits one block's K range in four and
// adds the partials through LDS in wave order; where that leaves the chip idle, K is cut
// further over work-groups, with fp32 partials that splitk_reduce adds in a fixed order.
// Reruns are bit-identical.
// D register r of lane l is D[i0 + 4 (l / 16) + r][j0 + l % 16].
template <bool TX, bool TY, int SK_WAVES>
__global__ void __launch_bounds__(64 * SK_WAVES)
gemm_f32_skinny_kernel(int M, int N, int K, const float* __restrict__ X, int ldx,
                       const float* __restrict__ Y, int ldy, float beta, float* __restrict__ C,
                       long long ldcr, long long ldcc, int mblocks, int nblocks, int Kc,
                       int split_waves, float* __restrict__ part, long long part_ld,
                       const float* __restrict__ bias, int epi) {
    __shared__ f32x4 red[SK_WAVES][64];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    // unit = (split s, m-block, n-block); split_waves: the waves share one unit's K range
    const long long unit = split_waves ? (long long)blockIdx.x
                                       : (long long)blockIdx.x * SK_WAVES + wave;
    const long long units = (long long)mblocks * nblocks * ((K + Kc - 1) / Kc > 0 ? (K + Kc - 1) / Kc : 1);
    if (unit >= units) return;   // whole waves only (split_waves grids have no spare units)
    const int nb = (int)(unit % nblocks);
    const int mb = (int)((unit / nblocks) % mblocks);
    const int sidx = (int)(unit / ((long long)nblocks * mblocks));
    const int i0 = mb * 16, j0 = nb * 16;
    int kbeg = sidx * Kc, kend = min(K, kbeg + Kc);
    if (split_waves) {
        const int len = kend - kbeg;
        const int kw = ((len + SK_WAVES - 1) / SK_WAVES + 15) & ~15;
        kbeg = min(kend, kbeg + wave * kw);
        kend = min(kend, kbeg + kw);
    }
    const int li = lane & 15, lk = 4 * (lane >> 4);
    const int xi = i0 + li, yj = j0 + li;
    const bool xin = xi < M, yin = yj < N;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    auto xat = [&](int k) { return TX ? X[(long long)k * ldx + xi] : X[(long long)xi * ldx + k]; };
    auto yat = [&](int k) { return TY ? Y[(long long)yj * ldy + k] : Y[(long long)k * ldy + yj]; };
    // Four 16-deep groups in flight: group g + 4 is loaded while group g runs.  Loads past kend
    // read nothing and give zeros, whose products add exact zeros.
    float xa[4][4], yb[4][4];
    auto load = [&](int g, float (&xs)[4], float (&ys)[4]) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int k = kbeg + 16 * g + lk + j;
            const bool kin = k < kend;
            xs[j] = xin && kin ? xat(k) : 0.f;
            ys[j] = yin && kin ? yat(k) : 0.f;
        }
    };
#pragma unroll
    for (int t = 0; t < 4; ++t) load(t, xa[t], yb[t]);
    const int ngroups = (kend - kbeg + 15) >> 4;
    for (int g = 0; g < ngroups; g += 4) {
#pragma unroll
        for (int t = 0; t < 4; ++t) {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[t][j], yb[t][j], acc, 0, 0, 0);
            load(g + 4 + t, xa[t], yb[t]);
        }
    }
    if (split_waves) {
        red[wave][lane] = acc;
        __syncthreads();
        if (wave != 0) return;
        acc = red[0][lane];
#pragma unroll
        for (int w = 1; w < SK_WAVES; ++w) acc += red[w][lane];
    }
    const int jj = j0 + li;
    if (jj >= N) return;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int ii = i0 + lk + r;
        if (ii >= M) continue;
        // D[ii][jj] is C's element (ii, jj), or (jj, ii) when the operands were swapped
        if (part) {
            part[(long long)sidx * part_ld + ii * ldcr + jj * ldcc] = acc[r];
            continue;
        }
        float* c = C + ii * ldcr + jj * ldcc;
        const long long row = ldcc == 1 ? ii : jj, col = ldcc == 1 ? jj : ii;
        float v = (beta == 0.f ? acc[r] : acc[r] + beta * *c) +
                  (bias ? bias[(epi & DH_EPI_ROW_BIAS) ? row : col] : 0.f);
        if (epi & DH_EPI_RELU) v = v < 0.f ? 0.f : v;
        *c = v;
    }
}

// D = X Y with X = op(A), Y = op(B) (swap = false), or X = op(B)^T, Y = op(A)^T (swap = true:
// M <= 16, so the short side lands on the 16 rows of a block) and C = D^T.  Returns
// DH_ERR_UNSUPPORTED when the pool cannot give the split-K partials.
template <bool TA, bool TB>
int launch_skinny(int M, int N, int K, const float* A, int lda, const float* B, int ldb,
                  float beta, float* C, int ldc, const Batch& bt) {
    const bool swap = M <= 16 && N > 16;
    const int DM = swap ? N : M, DN = swap ? M : N;
    const long long ldcr = swap ? 1 : ldc, ldcc = swap ? ldc : 1;
    const int mblocks = (DM + 15) / 16, nblocks = (DN + 15) / 16;
    const long long mn_units = (long long)mblocks * nblocks;
    const int cus = num_cus();
    // Work-group shapes.  K above 64: the 4 waves of a work-group split one block's K range;
    // K of 64 and less: each wave its own block.  Few blocks with a long K (config 2's
    // dW2 = H^T dY: 17 blocks, K = 4096) split K over work-groups, chunks of at least 256, to
    // about 4 work-groups per CU; their fp32 partials are added in order by splitk_reduce
    // (18.3 -> 9.8 us).  Measured and rejected for that shape: one 16-wave work-group per block
    // and no split (14.9 us: too few loads in flight per CU), and the reduction inside the
    // launch by the last split to take an integer ticket (14.7-17.6 us: the device-scope
    // release fence each split needs writes back its XCD's L2 under the others' streams).
    const bool split_waves = K > 64;
    const int W = 4;
    int S = 1;
    if (split_waves && mn_units < (long long)cus) {
        long long sp = (4LL * cus + mn_units - 1) / mn_units;
        sp = sp > K / 256 ? K / 256 : sp;
        S = sp < 1 ? 1 : (int)sp;
    }
    const int Kc = S == 1 ? (K > 0 ? K : 1) : ((K + S - 1) / S + 15) & ~15;
    S = K > 0 ? (K + Kc - 1) / Kc : 1;
    const long long units = mn_units * S;
    const long long wgs = split_waves ? units : (units + W - 1) / W;
    if (wgs > 0x7fffffffLL) return set_error(DH_ERR_UNSUPPORTED, "dh_gemm_f32(skinny): grid");
    float* part = nullptr;
    if (S > 1) {
        part = static_cast<float*>(dh_malloc((size_t)S * M * N * sizeof(float)));
        if (!part) return DH_ERR_UNSUPPORTED;
    }
    const long long pr = swap ? 1 : N, pc = swap ? N : 1;   // partials are row-major M x N
    hipStream_t s = stream();
#define DH_SKINNY(TX, TY, X, LDX, Y, LDY, WV)                                                    \
    gemm_f32_skinny_kernel<TX, TY, WV><<<(unsigned)wgs, 64 * WV, 0, s>>>(                         \
        DM, DN, K, X, LDX, Y, LDY, beta, C, part ? pr : ldcr, part ? pc : ldcc, mblocks, nblocks, \
        Kc, split_waves ? 1 : 0, part, (long long)M * N, bt.bias, bt.epi)
    if (!swap) DH_SKINNY(TA, TB, A, lda, B, ldb, 4);
    else DH_SKINNY(!TB, !TA, B, ldb, A, lda, 4);
#undef DH_SKINNY
    int st = check_launch("dh_gemm_f32(skinny)");
    if (part) {
        if (st == DH_OK) {
            size_t blocks = ((size_t)M * N + 255) / 256;
            if (blocks > (size_t)cus * 8) blocks = (size_t)cus * 8;
            splitk_reduce<<<(unsigned)blocks, 256, 0, s>>>(part, S, M, N, beta, C, ldc, bt.bias,
                                                           bt.epi);
            st = check_launch("dh_gemm_f32(skinny reduce)");
        }
        dh_free(part);   // pooled; later users of the buffer are ordered on the stream
    }
    return st;
}

// Tile shape.  64 x 256 when M <= 64 (a 128-row tile would be at least half empty -- conv's
// kernel @ im2col with few output channels, the bias gradient shapes), 256 x 64 when N <= 64,
// else 128 x 128; but 64 x 64 tiles (one 32 x 32 block per wave, 8 waves per SIMD fit) when
// the larger tiles leave the chip mostly idle: a 128 x 128 grid of less than one tile per CU
// that 64 x 64 tiles take past half the CUs, or a narrow grid of at most a quarter of the CUs
// that 64 x 64 tiles at least double.  Measured (config 1 and config 2's layer products):
// fp32 1024^3 43.2 -> 30.7 us; 4096 x 257 x 784 67 -> 41 us; 4096 x 784 x 257 48 -> 42 us;
// 4096 x 10 x 257 43 -> 15 us; 257 x 10 x 4096 31 -> 18 us.
template <bool TA, bool TB>
int launch_ks(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float beta,
              float* C, int ldc, const Batch& bt) {
    const int ca = TA ? M : K, cb = TB ? K : N;
    const bool va = ((uintptr_t)A % 16 == 0) && (lda % 4 == 0) && (bt.sA % 4 == 0) && (ca % 4 == 0);
    const bool vb = ((uintptr_t)B % 16 == 0) && (ldb % 4 == 0) && (bt.sB % 4 == 0) && (cb % 4 == 0);
    const int nk = (K + KS_BK - 1) / KS_BK;
    const bool deep = (nk % 4 == 0 && nk >= 8) || nk >= 40;   // a last group wastes < 10%
    auto kern = deep ? (va && vb ? gemm_f32_ks_kernel<TA, TB, true, true, 4>
                        : va     ? gemm_f32_ks_kernel<TA, TB, true, false, 4>
                        : vb     ? gemm_f32_ks_kernel<TA, TB, false, true, 4>
                                 : gemm_f32_ks_kernel<TA, TB, false, false, 4>)
                     : (va && vb ? gemm_f32_ks_kernel<TA, TB, true, true, 2>
                        : va     ? gemm_f32_ks_kernel<TA, TB, true, false, 2>
                        : vb     ? gemm_f32_ks_kernel<TA, TB, false, true, 2>
                                 : gemm_f32_ks_kernel<TA, TB, false, false, 2>);
    const int tiles = ((M + 63) / 64) * ((N + 63) / 64);
    for (int b0 = 0; b0 < bt.count; b0 += 65535) {
        const int nb = bt.count - b0 < 65535 ? bt.count - b0 : 65535;
        kern<<<dim3(tiles, nb), KS_NT, 0, stream()>>>(M, N, K, A + b0 * bt.sA, lda, B + b0 * bt.sB,
                                                       ldb, beta, C + b0 * bt.sC, ldc, bt.sA,
                                                       bt.sB, bt.sC, bt.bias, bt.epi);
        DH_TRY(check_launch("dh_gemm_f32(64x64, 8 waves)"));
    }
    return DH_OK;
}

template <bool TA, bool TB>
int launch(int M, int N, int K, const float* A, int lda, const float* B, int ldb, float beta,
           float* C, int ldc, const Batch& bt) {
    const int cus = num_cus();
    // Skinny products: a side of at most 16 rows or columns (measured on config 2: H W2 15.3 ->
    // 5.8 us, dW2 = H^T dY 18.3 -> 9.8 us).  A short K alone (dH = dY W2^T, 4096 x 257, K 10)
    // is write-bound and stays on the tiled kernels (5.8 us there, 8.3 us here).
    if (bt.count == 1 && (M <= 16 || N <= 16)) {
        const int st = launch_skinny<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        if (st != DH_ERR_UNSUPPORTED) return st;   // no workspace: the tiled kernels below
    }
    const long long t64 = (long long)((M + 63) / 64) * ((N + 63) / 64) * bt.count;
    if ((M <= 64 && N > 64) || (N <= 64 && M > 64)) {
        const long long tn = (long long)((M <= 64 ? N : M) + 255) / 256 * bt.count;
        if (4 * tn <= cus && 2 * tn < t64)
            return launch_tiles<TA, TB, 64, 64>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        if (M <= 64) return launch_tiles<TA, TB, 64, 256>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        return launch_tiles<TA, TB, 256, 64>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    }
    const long long t128 = (long long)((M + 127) / 128) * ((N + 127) / 128) * bt.count;
    if (t128 < cus && 2 * t64 > cus) {
        // At most one work-group per CU and a contraction of several 32-wide slices: two
        // waves per SIMD on each tile (config 1, 1024^3: 0.0316 -> 0.0296 ms).  With more
        // work-groups than CUs the second work-group of a CU already fills the gaps (config
        // 2's first layer, 320 tiles: 0.0382 -> 0.0406 ms with this kernel), and short
        // contractions (K = 10: 0.0058 -> 0.0070 ms) do not amortise the wide slices.
        if (t64 <= cus && K >= 256)
            return launch_ks<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        return launch_tiles<TA, TB, 64, 64>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    }
    // Grids small enough for launch_tiles' split-K path: where 128-wide tiles pad the output
    // by markedly more than 64-wide ones, split 64 x 64 tiles instead (config 2's
    // dW1 = X^T dZ1, 784 x 257 with K = 4096: 41% of the 128-tile area is padding against 24%
    // of the 64-tile area; 0.0591 -> 0.0486 ms, same box, three reps).
    if (bt.count == 1 && K >= 512 && 2 * t64 <= cus) {
        const double a128 = (double)((M + 127) / 128) * ((N + 127) / 128) * 128.0 * 128.0;
        const double a64 = (double)((M + 63) / 64) * ((N + 63) / 64) * 64.0 * 64.0;
        if (a64 < 0.9 * a128)
            return launch_tiles<TA, TB, 64, 64>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    }
    return launch_tiles<TA, TB, 128, 128>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

// Tile choice and launch shared by the forward and the data gradient: 64 x 64 tiles for few
// output channels (the bench layer: 0.271 -> 0.212 ms against 64 x 256 tiles -- 3136
// work-groups at 8 waves per SIMD instead of 832 at 2) and for small grids; 128 x 128
// otherwise.
int run_conv(int N, int Cout, long long P, long long R, const float* Kn, const float* X,
             const ConvGeom& g, float* Y, const float* bias, int accumulate) {
    const int cus = num_cus();
    const long long t128 = (long long)((Cout + 127) / 128) * ((P + 127) / 128) * N;
    const long long t64 = (long long)((Cout + 63) / 64) * ((P + 63) / 64) * N;
    if (Cout <= 64 || (t128 < cus && 2 * t64 > cus))
        return launch_conv<64, 64>(N, Cout, (int)P, (int)R, Kn, X, g, Y, bias, accumulate);
    return launch_conv<128, 128>(N, Cout, (int)P, (int)R, Kn, X, g, Y, bias, accumulate);
}

// Kt[ci][(co KH + kh) KW + kw] = Kn[co][(ci KH + KH-1-kh) KW + KW-1-kw]: the kernel of the
// data gradient (channels swapped, window flipped).
__global__ void __launch_bounds__(256) conv_flip_kernel(const float* __restrict__ Kn,
                                                        float* __restrict__ Kt, int Cout, int Cin,
                                                        int KH, int KW) {
    const size_t win = (size_t)KH * KW, n = (size_t)Cout * Cin * win;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) {
        const size_t ci = i / (Cout * win), rem = i % (Cout * win);
        const size_t co = rem / win, t = rem % win;
        const int kh = (int)(t / KW), kw = (int)(t % KW);
        Kt[i] = Kn[co * Cin * win + (ci * KH + KH - 1 - kh) * KW + KW - 1 - kw];
    }
}

}  // namespace

int splitk_reduce_launch(const float* part, int S, int M, int N, float beta, float* C, int ldc,
                         const float* bias, int epi) {
    size_t blocks = ((size_t)M * N + 255) / 256;
    if (blocks > (size_t)num_cus() * 8) blocks = (size_t)num_cus() * 8;
    splitk_reduce<<<(unsigned)blocks, 256, 0, stream()>>>(part, S, M, N, beta, C, ldc, bias, epi);
    return check_launch("split-K reduce");
}

template <int D>
int launch_dq_from_ds(int BH, int S, int causal, const float* dS, long long slice, const float* K,
                      float beta, float* dQ) {
    const int T = (S + 127) / 128;
    // 16-byte loads of dS rows need every tile's K extent (a multiple of 128, or S) to be a
    // multiple of 4; K rows (D floats) need an aligned base
    const bool va = S % 4 == 0, vb = (uintptr_t)K % 16 == 0;
    auto kern = va && vb ? flash_dq_from_ds_kernel<true, true, D>
              : va       ? flash_dq_from_ds_kernel<true, false, D>
              : vb       ? flash_dq_from_ds_kernel<false, true, D>
                         : flash_dq_from_ds_kernel<false, false, D>;
    kern<<<(unsigned)(T * BH * (D == 128 ? 1 : 2)), NTHREADS, 0, stream()>>>(BH, S, T, causal, dS,
                                                                            slice, K, beta, dQ);
    return check_launch("flash backward dQ from dS");
}

int flash_dq_from_ds_f32(int BH, int S, int D, int causal, const float* dS, long long slice,
                         const float* K, float beta, float* dQ) {
    if (D == 128) return launch_dq_from_ds<128>(BH, S, causal, dS, slice, K, beta, dQ);
    if (D == 64) return launch_dq_from_ds<64>(BH, S, causal, dS, slice, K, beta, dQ);
    return set_error(DH_ERR_INVALID, "flash backward dQ from dS: head dimension %d", D);
}

}  // namespace dh

using namespace dh;

extern "C" int dh_gemm_f32_ex(int transA, int transB, int M, int N, int K, const float* A,
                              int lda, long long strideA, const float* B, int ldb,
                              long long strideB, float beta, float* C, int ldc,
                              long long strideC, int batch, const float* bias, int epilogue) {
    DH_TRY(ensure_init());
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return set_error(DH_ERR_INVALID, "dh_gemm_f32: negative shape");
    if (M == 0 || N == 0 || batch == 0) return DH_OK;
    if (!C || (K > 0 && (!A || !B)))
        return set_error(DH_ERR_INVALID, "dh_gemm_f32: null pointer");
    // A and B are not read when K == 0, so only C's leading dimension matters then.
    if (ldc < N || (K > 0 && (lda < (transA ? M : K) || ldb < (transB ? K : N))))
        return set_error(DH_ERR_INVALID, "dh_gemm_f32: leading dimension too small");
    if (batch > 1 && (strideA < 0 || strideB < 0 || strideC < (long long)(M - 1) * ldc + N))
        return set_error(DH_ERR_INVALID, "dh_gemm_f32: batch strides overlap C or are negative");
    const Batch bt{batch > 1 ? strideA : 0, batch > 1 ? strideB : 0, batch > 1 ? strideC : 0,
                   batch, bias, epilogue};
    if (transA)
        return transB ? launch<true, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt)
                      : launch<true, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    return transB ? launch<false, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt)
                  : launch<false, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

extern "C" int dh_gemm_f32(int transA, int transB, int M, int N, int K, const float* A, int lda,
                           const float* B, int ldb, float beta, float* C, int ldc) {
    return dh_gemm_f32_ex(transA, transB, M, N, K, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1,
                          nullptr, 0);
}

extern "C" int dh_conv2d_fwd(const float* X, const float* Kn, const float* bias, float* Y, int N,
                             int Cin, int H, int W, int Cout, int KH, int KW, int pad,
                             int stride) {
    DH_TRY(ensure_init());
    if (N < 0 || Cin < 1 || H < 1 || W < 1 || Cout < 1 || KH < 1 || KW < 1 || pad < 0 ||
        stride < 1)
        return set_error(DH_ERR_INVALID, "dh_conv2d_fwd: invalid shape");
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        return set_error(DH_ERR_INVALID, "dh_conv2d_fwd: kernel larger than the padded input");
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const long long P = (long long)OH * OW, R = (long long)Cin * KH * KW;
    if (N == 0) return DH_OK;
    if (!X || !Kn || !Y) return set_error(DH_ERR_INVALID, "dh_conv2d_fwd: null pointer");
    if (P >= (1ll << 30) || R >= (1ll << 30) || (long long)H * W >= (1ll << 30) ||
        (long long)Cout * P >= (1ll << 31) || 4ll * Cin * H * W >= (long long)CONV_OOB)
        return set_error(DH_ERR_UNSUPPORTED, "dh_conv2d_fwd: plane or window too large");
    ConvGeom g{Cin, H, W, KH, KW, pad, pad, stride, OH, OW, make_fastdiv((uint32_t)OW),
               make_fastdiv((uint32_t)KW), make_fastdiv((uint32_t)(KH * KW))};
    return run_conv(N, Cout, P, R, Kn, X, g, Y, bias, 0);
}

// dX (+)= the input gradient of a stride-1 convolution: for stride 1, col2im(K^T dY) is the
// convolution of dY (Cout channels, OH x OW) with the flipped, channel-swapped kernel, padded
// by KH - 1 - pad rows and KW - 1 - pad columns -- one implicit-GEMM launch (Cin x H W x
// Cout KH KW per image) after a small flip kernel, no column matrices.
extern "C" int dh_conv2d_bwd_data(const float* dY, const float* Kn, float* dX, int N, int Cin,
                                  int H, int W, int Cout, int KH, int KW, int pad, int stride,
                                  int accumulate) {
    DH_TRY(ensure_init());
    if (N < 0 || Cin < 1 || H < 1 || W < 1 || Cout < 1 || KH < 1 || KW < 1 || pad < 0 ||
        stride < 1)
        return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_data: invalid shape");
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_data: kernel larger than the padded input");
    if (stride != 1 || pad > KH - 1 || pad > KW - 1)
        return set_error(DH_ERR_UNSUPPORTED,
                         "dh_conv2d_bwd_data: stride %d, pad %d (stride 1 and pad < kernel size "
                         "only; use dh_gemm_f32 + dh_col2im)", stride, pad);
    const int OH = H + 2 * pad - KH + 1, OW = W + 2 * pad - KW + 1;
    const long long P = (long long)H * W, R = (long long)Cout * KH * KW;
    if (N == 0) return DH_OK;
    if (!dY || !Kn || !dX) return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_data: null pointer");
    if (P >= (1ll << 30) || R >= (1ll << 30) || (long long)OH * OW >= (1ll << 30) ||
        (long long)Cin * P >= (1ll << 31) || 4ll * Cout * OH * OW >= (long long)CONV_OOB)
        return set_error(DH_ERR_UNSUPPORTED, "dh_conv2d_bwd_data: plane or window too large");
    float* Kt = static_cast<float*>(dh_malloc((size_t)Cin * R * sizeof(float)));
    if (!Kt) return set_error(DH_ERR_OOM, "dh_conv2d_bwd_data: flipped kernel");
    const size_t nk = (size_t)Cin * R;
    size_t blocks = (nk + 255) / 256;
    if (blocks > (size_t)num_cus() * 8) blocks = (size_t)num_cus() * 8;
    conv_flip_kernel<<<(unsigned)blocks, 256, 0, stream()>>>(Kn, Kt, Cout, Cin, KH, KW);
    int st = check_launch("dh_conv2d_bwd_data(flip)");
    if (st == DH_OK) {
        ConvGeom g{Cout, OH, OW, KH, KW, KH - 1 - pad, KW - 1 - pad, 1, H, W,
                   make_fastdiv((uint32_t)W), make_fastdiv((uint32_t)KW),
                   make_fastdiv((uint32_t)(KH * KW))};
        st = run_conv(N, Cin, P, R, Kt, dY, g, dX, nullptr, accumulate ? 1 : 0);
    }
    dh_free(Kt);   // pooled; later users of the buffer are ordered on the stream
    return st;
}

// gK (+)= the kernel gradient of a convolution, any pad and stride: sum over images of
// dY_n col_n^T with col_n gathered from X inside the GEMM loader (no im2col matrix, no
// channel-first copy of dY), split over the (image, position) contraction and reduced in a
// fixed order.
extern "C" int dh_conv2d_bwd_filter(const float* dY, const float* X, float* dK, int N, int Cin,
                                    int H, int W, int Cout, int KH, int KW, int pad, int stride,
                                    int accumulate) {
    DH_TRY(ensure_init());
    if (N < 0 || Cin < 1 || H < 1 || W < 1 || Cout < 1 || KH < 1 || KW < 1 || pad < 0 ||
        stride < 1)
        return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_filter: invalid shape");
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_filter: kernel larger than the padded input");
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const long long P = (long long)OH * OW, R = (long long)Cin * KH * KW;
    if (!dK) return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_filter: null pointer");
    if (P >= (1ll << 30) || R >= (1ll << 30) || (long long)H * W >= (1ll << 30) ||
        (long long)Cout * P >= (1ll << 31) || (long long)Cout * R >= (1ll << 31) ||
        4ll * Cin * H * W >= (long long)CONV_OOB)
        return set_error(DH_ERR_UNSUPPORTED, "dh_conv2d_bwd_filter: plane or window too large");
    if (N == 0)   // an empty sum: dK = 0, or unchanged with accumulate
        return accumulate ? DH_OK : dh_memset(dK, 0, (size_t)Cout * R * sizeof(float));
    if (!dY || !X) return set_error(DH_ERR_INVALID, "dh_conv2d_bwd_filter: null pointer");
    ConvGeom g{Cin, H, W, KH, KW, pad, pad, stride, OH, OW, make_fastdiv((uint32_t)OW),
               make_fastdiv((uint32_t)KW), make_fastdiv((uint32_t)(KH * KW))};
    if (Cout <= 64)
        return launch_wgrad<64, 64>(N, Cout, (int)P, (int)R, dY, X, g, dK, accumulate);
    return launch_wgrad<128, 128>(N, Cout, (int)P, (int)R, dY, X, g, dK, accumulate);
}
