// dh_gemm_bf16.hip -- bf16 x bf16 -> fp32 GEMM on gfx950 (v_mfma_f32_32x32x16_bf16).
//
// Same contract as dh_gemm_f32 (NN / NT / TN / TT, beta, batch strides, bias + ReLU epilogue),
// with bf16 operands and fp32 accumulation and output.  Replaces the reference's fp16 cublasGemmEx branch
// (runtime/ops/elementwise.inc:1046-1071) for tensor_matmul in reduced-precision mode.
//
// Work decomposition
//   BIG   : 256 x 256 C tile per work-group, 4 waves as 2 x 2, wave tile 128 x 128
//           (4 x 4 MFMA blocks, 256 fp32 accumulators per lane), K slice 64.
//   SMALL : 128 x 128 tile, wave tile 64 x 64, K slice 64 (small or skinny shapes).
//   LDS holds both operands k-contiguous (As[i][k], Bs[j][k], rows padded by 16 bytes)
//   and is double-buffered; the next slice is fetched into registers while the
//   matrix cores consume the current one.
// MFMA operand layout (32x32x16 bf16): lane l supplies 8 consecutive-k values
//   A[i = l % 32][8 * (l / 32) .. +7] and B[8 * (l / 32) .. +7][j = l % 32], one
//   128-bit LDS read each; accumulator layout as for the fp32 32x32 MFMA.
// Operands stored with k as the slow (row) index -- B in NN, A in TN -- are fetched
// as 4 (k) x 8 (i or j) blocks and transposed in registers with v_perm_b32 before
// the LDS write.
#include <cstdlib>
#include <type_traits>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int NTHREADS = 256;

// 16 bytes = 8 bf16 of one row, zero outside [0, rows) x [0, cols).
template <bool VEC>
__device__ inline u32x4 load8(const uint16_t* __restrict__ p, int ld, int rows, int cols, int r,
                              int c) {
    u32x4 v = {0u, 0u, 0u, 0u};
    if (r >= rows) return v;
    const uint16_t* q = p + (size_t)r * ld + c;
    if (VEC && c + 7 < cols) return *reinterpret_cast<const u32x4*>(q);
    uint16_t e[8];
#pragma unroll
    for (int x = 0; x < 8; ++x) e[x] = (c + x < cols) ? q[x] : (uint16_t)0;
#pragma unroll
    for (int x = 0; x < 4; ++x) v[x] = (uint32_t)e[2 * x] | ((uint32_t)e[2 * x + 1] << 16);
    return v;
}

// One operand's K slice: TILE rows (i or j) x BK columns (k), written to LDS as
// lds[t * STRIDE + k].
template <bool KCONTIG, bool VEC, int TILE, int BK>
struct Slice {
    static constexpr int STRIDE = BK + 8;   // bf16 elements per LDS row
    // k-contiguous: chunks of 8 k; otherwise blocks of 4 k x 8 t.
    static constexpr int CHUNKS = KCONTIG ? TILE * BK / 8 / NTHREADS : TILE * BK / 32 / NTHREADS;
    static_assert(CHUNKS >= 1, "tile too small for the thread count");
    u32x4 v[KCONTIG ? CHUNKS : 4 * CHUNKS];

    __device__ void fetch(const uint16_t* __restrict__ base, int ld, int t0, int k0,
                          int extent_t, int extent_k, int tid) {
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const int f = tid + c * NTHREADS;
            if (KCONTIG) {   // stored [t][k]
                const int t = f / (BK / 8), kq = f % (BK / 8);
                v[c] = load8<VEC>(base, ld, extent_t, extent_k, t0 + t, k0 + 8 * kq);
            } else {         // stored [k][t]: 4 rows of k, 8 t each
                const int kq = f % (BK / 4), tb = f / (BK / 4);
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    v[4 * c + r] = load8<VEC>(base, ld, extent_k, extent_t, k0 + 4 * kq + r,
                                              t0 + 8 * tb);
            }
        }
    }

    __device__ void store(uint16_t* lds, int tid) const {
#pragma unroll
        for (int c = 0; c < CHUNKS; ++c) {
            const int f = tid + c * NTHREADS;
            if (KCONTIG) {
                const int t = f / (BK / 8), kq = f % (BK / 8);
                *reinterpret_cast<u32x4*>(&lds[t * STRIDE + 8 * kq]) = v[c];
            } else {
                const int kq = f % (BK / 4), tb = f / (BK / 4);
                const u32x4* r = &v[4 * c];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    // element (k = r, t = 2q + s) sits in half s of r[k][q]
                    u32x2 lo = {pack_lo16(r[0][q], r[1][q]), pack_lo16(r[2][q], r[3][q])};
                    u32x2 hi = {pack_hi16(r[0][q], r[1][q]), pack_hi16(r[2][q], r[3][q])};
                    *reinterpret_cast<u32x2*>(&lds[(8 * tb + 2 * q) * STRIDE + 4 * kq]) = lo;
                    *reinterpret_cast<u32x2*>(&lds[(8 * tb + 2 * q + 1) * STRIDE + 4 * kq]) = hi;
                }
            }
        }
    }
};

template <int BM, int BN, int BK, int WAVES_M, bool TA, bool TB, bool VA, bool VB>
__global__ void __launch_bounds__(NTHREADS)
gemm_bf16_kernel(int M, int N, int K, const uint16_t* __restrict__ A, int lda,
                 const uint16_t* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                 int ldc, long long sA, long long sB, long long sC,
                 const float* __restrict__ bias, int epi) {
    A += blockIdx.y * sA;   // batch member blockIdx.y
    B += blockIdx.y * sB;
    C += blockIdx.y * sC;
    constexpr int WAVES_N = 4 / WAVES_M;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    using SA = Slice<!TA, VA, BM, BK>;
    using SB = Slice<TB, VB, BN, BK>;
    constexpr int STRIDE = SA::STRIDE;

    extern __shared__ __attribute__((aligned(16))) uint16_t smem[];
    // stage s: A tile at smem + s * BM * STRIDE, B tile after both A stages.
    uint16_t* const a_lds = smem;
    uint16_t* const b_lds = smem + 2 * BM * STRIDE;

    const int tiles_m = (M + BM - 1) / BM, tiles_n = (N + BN - 1) / BN;
    int tm, tn;
    xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 8, tm, tn);
    const int m0 = tm * BM, n0 = tn * BN;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = (wave / WAVES_N) * WTM, wn = (wave % WAVES_N) * WTN;

    SA sa;
    SB sb;
    f32x16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    const int nk = (K + BK - 1) / BK;
    if (nk > 0) {
        sa.fetch(A, lda, m0, 0, M, K, tid);
        sb.fetch(B, ldb, n0, 0, N, K, tid);
        sa.store(a_lds, tid);
        sb.store(b_lds, tid);
        __syncthreads();
    }
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) {
            sa.fetch(A, lda, m0, (kt + 1) * BK, M, K, tid);
            sb.fetch(B, ldb, n0, (kt + 1) * BK, N, K, tid);
        }
        const uint16_t* as = a_lds + cur * BM * STRIDE;
        const uint16_t* bs = b_lds + cur * BN * STRIDE;
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            bf16x8 af[FM], bfr[FN];
#pragma unroll
            for (int a = 0; a < FM; ++a)
                af[a] = *reinterpret_cast<const bf16x8*>(
                    &as[(wm + 32 * a + l32) * STRIDE + kk + 8 * h]);
#pragma unroll
            for (int b = 0; b < FN; ++b)
                bfr[b] = *reinterpret_cast<const bf16x8*>(
                    &bs[(wn + 32 * b + l32) * STRIDE + kk + 8 * h]);
#pragma unroll
            for (int a = 0; a < FM; ++a)
#pragma unroll
                for (int b = 0; b < FN; ++b)
                    acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[a], bfr[b], acc[a][b],
                                                                       0, 0, 0);
        }
        if (more) {
            sa.store(a_lds + (cur ^ 1) * BM * STRIDE, tid);
            sb.store(b_lds + (cur ^ 1) * BN * STRIDE, tid);
        }
        __syncthreads();
    }

#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b) {
            const int col = n0 + wn + 32 * b + l32;
            if (col >= N) continue;
            const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS);
            const float bv = bias && !row_bias ? bias[col] : 0.f;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < M) {
                    float* c = C + (size_t)row * ldc + col;
                    float v = (beta == 0.f ? acc[a][b][r] : acc[a][b][r] + beta * *c) +
                              (row_bias ? bias[row] : bv);
                    if (epi & DH_EPI_RELU) v = v < 0.f ? 0.f : v;
                    __builtin_nontemporal_store(v, c);
                }
            }
        }
}

struct Batch {
    long long sA, sB, sC;   // element strides between batch members (0 for one product)
    int count;
    const float* bias;      // per-column bias of the epilogue, or null
    int epi;                // DH_EPI_* flags
};

template <int BM, int BN, int BK, int WAVES_M, bool TA, bool TB, bool VA, bool VB>
int launch_cfg(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
               float beta, float* C, int ldc, const Batch& bt) {
    auto kern = gemm_bf16_kernel<BM, BN, BK, WAVES_M, TA, TB, VA, VB>;
    const size_t lds = (size_t)2 * (BM + BN) * (BK + 8) * sizeof(uint16_t);
    static bool attr_set = false;
    if (!attr_set) {
        hipError_t e = hipFuncSetAttribute((const void*)kern,
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        if (e != hipSuccess)
            return set_error(DH_ERR_HIP, "dh_gemm_bf16: LDS attribute: %s", hipGetErrorString(e));
        attr_set = true;
    }
    const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
    for (int b0 = 0; b0 < bt.count; b0 += 65535) {   // gridDim.y = batch member
        const int nb = bt.count - b0 < 65535 ? bt.count - b0 : 65535;
        kern<<<dim3(tiles, nb), NTHREADS, lds, stream()>>>(
            M, N, K, A + b0 * bt.sA, lda, B + b0 * bt.sB, ldb, beta, C + b0 * bt.sC, ldc, bt.sA,
            bt.sB, bt.sC, bt.bias, bt.epi);
        DH_TRY(check_launch("dh_gemm_bf16"));
    }
    return DH_OK;
}

template <bool TA, bool TB, bool VA, bool VB>
int launch_vec(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
               float beta, float* C, int ldc, const Batch& bt) {
    // The 256 x 256 tile needs enough tiles to cover the chip; otherwise use 128 x 128.
    const long long big_tiles = (long long)((M + 255) / 256) * ((N + 255) / 256) * bt.count;
    if (M >= 256 && N >= 256 && big_tiles >= num_cus())
        return launch_cfg<256, 256, 64, 2, TA, TB, VA, VB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    return launch_cfg<128, 128, 64, 2, TA, TB, VA, VB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

// ---------------------------------------------------------------------------------
// Fast path for tile-aligned shapes (M, N multiples of 256, K of 32, leading dims of 8,
// 16-byte aligned operands): both operands travel global -> LDS by direct-to-LDS DMA
// (buffer_load_dwordx4 ... lds: lane l's 16 bytes land at base + 16 l), so no registers or
// LDS-write instructions are spent on staging.  LDS tiles keep the global orientation:
//   k-contiguous operand  : [256 rows][32 k],  16-byte chunk c of row r at position
//                           c ^ (r / 4 % 4)  -> MFMA fragment = one ds_read_b128
//   mn-contiguous operand : [32 k][256 cols], chunk c of row k at c ^ 4 (k % 4)
//                           -> MFMA fragment = two ds_read_b64_tr_b16
// ds_read_b64_tr_b16 semantics (measured on gfx950): in each 16-lane group, lane i names
// a row R_i of 4 consecutive 16-bit values; lane j receives R_{j/4 + 4e}[j % 4] for
// e = 0..3.  Pointing lane i at [kb + i/4][nb + 4 (i % 4)] therefore hands lane j the 4
// values [kb .. kb + 3][nb + j], the MFMA operand layout.  The LDS serves 64 banks of
// 4 bytes (16 lanes of a b128 read, 32 lanes of a b64 read per pass); both swizzles make
// the fragment reads conflict free under that model.  A ring of four LDS stages (128 KB);
// fragments of the next k-step are read while the matrix cores run the current one.
// ---------------------------------------------------------------------------------

template <bool KCONTIG, int WAVES, int T = 256>
struct FastOperand {
    // One 32-k stage of a T-wide operand tile (T = 256 or 128) is T / 16 DMA blocks of 1 KB;
    // wave w issues blocks PER*w .. PER*w + PER-1.  Per-lane element offsets at k0 = 0 and
    // the per-stage step.
    static constexpr int NBLK = T / 16;
    static constexpr int PER = NBLK / WAVES;
    static constexpr int KPB = 512 / T;    // k rows of an mn-contiguous tile per DMA block
    static constexpr int CPR = T / 8;      // 16-byte chunks in one of those rows
    static constexpr int CPR_LOG = T == 256 ? 5 : 4;
    static_assert(T == 256 || T == 128, "tile widths");
    uint32_t off[PER];     // byte offsets from the operand base at stage 0
    uint32_t step;         // bytes per stage
    uint32_t bytes;        // operand extent (rows x ld x 2 < 2^32, checked by the host)

    __device__ void init(int ld, int rows, int t0, int wave, int lane) {
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int b = PER * wave + t;
            if (KCONTIG) {                     // block b = rows 16b .. 16b+15 of [t][32 k]
                const int row = 16 * b + (lane >> 2);
                const int c = (lane & 3) ^ ((lane >> 4) & 3);   // = p ^ ((row >> 2) & 3)
                off[t] = 2u * ((uint32_t)(t0 + row) * ld + 8 * c);
            } else {                           // block b = k rows KPB b .. of [32 k][T]
                const int k = KPB * b + (lane >> CPR_LOG);
                const int c = (lane & (CPR - 1)) ^ (4 * (k & 3));
                off[t] = 2u * ((uint32_t)k * ld + t0 + 8 * c);
            }
        }
        step = KCONTIG ? 64u : 64u * (uint32_t)ld;
        bytes = 2u * (uint32_t)rows * (uint32_t)ld;
    }
    // Buffer-resource DMA: the per-lane offsets stay in VGPRs for the whole loop and the
    // stage advance is a scalar offset, so an issue costs no vector instructions.
    __device__ void issue(const uint16_t* __restrict__ g, int kt, uint16_t* lds, int wave) const {
        const uint32_t soff = __builtin_amdgcn_readfirstlane((uint32_t)kt * step);
        const uint32_t base = __builtin_amdgcn_readfirstlane(lds_addr(lds) + 1024u * PER * wave);
        const u32x4 rs = make_rsrc(g, bytes);
#pragma unroll
        for (int t = 0; t < PER; ++t) lds_dma16_buf_so(off[t], rs, soff, base + 1024u * t);
    }
    // MFMA operand for tile rows/cols o .. o+31, k-step kk (16 k) of the stage.
    __device__ static bf16x8 frag(const uint16_t* lds, int o, int kk, int lane) {
        const int h = lane >> 5;
        if (KCONTIG) {                         // [256][32]: chunk c of row r at c ^ (r/4 % 4)
            const int row = o + (lane & 31);
            const int p = (2 * kk + h) ^ ((row >> 2) & 3);
            return *reinterpret_cast<const bf16x8*>(lds + row * 32 + 8 * p);
        } else {                               // [32][T]: chunk c of row k at c ^ 4 (k % 4)
            const int G = (lane & 31) >> 4, i = lane & 15;
            const int n = o + 16 * G + 4 * (i & 3);
            s16x4 r[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int k = 16 * kk + 8 * h + 4 * q + (i >> 2);
                const int p = (n >> 3) ^ (4 * (k & 3));
                r[q] = ds_read_tr(lds + k * T + 8 * p + 4 * ((n >> 2) & 1));
            }
            return __builtin_bit_cast(bf16x8, __builtin_shufflevector(r[0], r[1], 0, 1, 2, 3, 4, 5, 6, 7));
        }
    }
    // The same fragment as PARTS separate LDS instructions (one b128 read, or two
    // transposing b64 reads), so that a schedule can place each between matrix-core ops.
    static constexpr int PARTS = KCONTIG ? 1 : 2;
    __device__ static void part(const uint16_t* lds, int o, int kk, int lane, int q,
                                s16x4 (&f)[2]) {
        const int h = lane >> 5;
        if (KCONTIG) {
            const int row = o + (lane & 31);
            const int p = (2 * kk + h) ^ ((row >> 2) & 3);
            const s16x8 v = *reinterpret_cast<const s16x8*>(lds + row * 32 + 8 * p);
            f[0] = __builtin_shufflevector(v, v, 0, 1, 2, 3);
            f[1] = __builtin_shufflevector(v, v, 4, 5, 6, 7);
        } else {
            const int G = (lane & 31) >> 4, i = lane & 15;
            const int n = o + 16 * G + 4 * (i & 3);
            const int k = 16 * kk + 8 * h + 4 * q + (i >> 2);
            const int p = (n >> 3) ^ (4 * (k & 3));
            f[q] = ds_read_tr(lds + k * T + 8 * p + 4 * ((n >> 2) & 1));
        }
    }
    // DMA block t of this wave's share of a stage (see issue()).
    __device__ void issue_one(u32x4 rs, uint32_t soff, uint32_t base, int t) const {
        lds_dma16_buf_so(off[t], rs, soff, base + 1024u * t);
    }
};

// A k-contiguous operand in double stages of 64 k for the one-wave-per-SIMD schedule: the
// 32-k stages above fetch 64 bytes per row, half an L2 line (the next stage fetches the other
// half again), while a 64-k stage fetches each row's full 128-byte line once.  LDS tile
// [256 rows][64 k] = 32 KB; 16-byte chunk c of row r at position c ^ ((r >> 1) & 7): the 16
// rows of one b128 pass fall on 8 even and 8 odd rows, so the 16-byte units they read are
// all different (conflict free).  DMA block b = rows 8b .. 8b+7, 8 lanes x 16 B per row;
// 32 blocks per double stage, 32 / WAVES per wave.
template <int WAVES>
struct DeepKOperand {
    static constexpr int PER = 32 / WAVES;
    static constexpr int PARTS = 1;
    static constexpr int ELEMS = 256 * 64;   // elements of one double stage
    uint32_t off[PER];                        // byte offsets from the operand base, pair 0
    uint32_t bytes;

    __device__ void init(int ld, int rows, int t0, int wave, int lane) {
#pragma unroll
        for (int t = 0; t < PER; ++t) {
            const int row = 8 * (PER * wave + t) + (lane >> 3);
            const int c = (lane & 7) ^ ((row >> 1) & 7);
            off[t] = 2u * ((uint32_t)(t0 + row) * ld + 8 * c);
        }
        bytes = 2u * (uint32_t)rows * (uint32_t)ld;
    }
    static constexpr uint32_t STEP = 128u;    // bytes per double stage along a row
    __device__ void issue_one(u32x4 rs, uint32_t soff, uint32_t base, int t) const {
        lds_dma16_buf_so(off[t], rs, soff, base + 1024u * t);
    }
    // k-step kk (0..3, 16 k each) of the double stage for tile rows o .. o+31.
    __device__ static void part(const uint16_t* lds, int o, int kk, int lane, int,
                                s16x4 (&f)[2]) {
        const int row = o + (lane & 31);
        const int p = (2 * kk + (lane >> 5)) ^ ((row >> 1) & 7);
        const s16x8 v = *reinterpret_cast<const s16x8*>(lds + row * 64 + 8 * p);
        f[0] = __builtin_shufflevector(v, v, 0, 1, 2, 3);
        f[1] = __builtin_shufflevector(v, v, 4, 5, 6, 7);
    }
};

constexpr int FAST_TILE = 256 * 32;   // elements of one operand stage (32 k)
constexpr int FAST_NSTAGE = 4;        // LDS ring: 4 x (A + B) x 16 KB = 128 KB

// Fragments of one 16-k step for the wave's FM x FN block of 32 x 32 MFMA tiles (the stage's
// B tile BOFF elements after its A tile).
template <typename OA, typename OB, int FM, int FN, int BOFF = FAST_TILE>
__device__ inline void load_frags(const uint16_t* st, int kk, int wm, int wn, int lane,
                                  bf16x8 (&fa)[FM], bf16x8 (&fb)[FN]) {
#pragma unroll
    for (int x = 0; x < FM; ++x) fa[x] = OA::frag(st, wm + 32 * x, kk, lane);
#pragma unroll
    for (int x = 0; x < FN; ++x) fb[x] = OB::frag(st + BOFF, wn + 32 * x, kk, lane);
}

template <int FM, int FN>
__device__ inline void mfma_block(const bf16x8 (&fa)[FM], const bf16x8 (&fb)[FN],
                                  f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
            acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[a], fb[b], acc[a][b], 0, 0, 0);
}

__device__ inline bf16x8 cat8(const s16x4 (&f)[2]) {
    return __builtin_bit_cast(bf16x8, __builtin_shufflevector(f[0], f[1], 0, 1, 2, 3, 4, 5, 6, 7));
}

// One 16-k step of a one-wave-per-SIMD schedule: the FM x FN matrix-core ops on the
// current fragments (ca, cb), with the LDS reads of the next fragments (na, nb, from stage
// `nst`, k-step nkk) and, when DMA, this wave's 2 x PER DMA blocks of a later stage placed
// one per op.  A single wave per SIMD issues at most one instruction every few cycles, so
// grouped reads or DMA issues would leave the matrix core idle; spread out, each hides
// under the op before it.
template <typename OA, typename OB, int FM, int FN, bool DMA>
__device__ inline void step_interleaved(const s16x4 (&ca)[FM][2], const s16x4 (&cb)[FN][2],
                                        f32x16 (&acc)[FM][FN], const uint16_t* nst, int nkk,
                                        int wm, int wn, int lane, s16x4 (&na)[FM][2],
                                        s16x4 (&nb)[FN][2], const OA& oa, const OB& ob,
                                        u32x4 rsa, u32x4 rsb, uint32_t soa, uint32_t sob,
                                        uint32_t basea, uint32_t baseb) {
    constexpr int NRA = FM * OA::PARTS, NR = NRA + FN * OB::PARTS;
    constexpr int NDMA = DMA ? OA::PER + OB::PER : 0;
    static_assert(NR <= FM * FN && NDMA <= FM * FN, "schedule slots");
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
        const int a = i / FN, b = i % FN;
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat8(ca[a]), cat8(cb[b]), acc[a][b],
                                                            0, 0, 0);
        if (i < NRA) {
            OA::part(nst, wm + 32 * (i / OA::PARTS), nkk, lane, i % OA::PARTS, na[i / OA::PARTS]);
        } else if (i < NR) {
            const int j = i - NRA;
            OB::part(nst + FAST_TILE, wn + 32 * (j / OB::PARTS), nkk, lane, j % OB::PARTS,
                     nb[j / OB::PARTS]);
        }
        // DMA blocks go after the later ops, once the reads are under way.
        const int d = i - (FM * FN - NDMA);
        if (d >= 0) {
            if (d < OA::PER) oa.issue_one(rsa, soa, basea, d);
            else ob.issue_one(rsb, sob, baseb, d - OA::PER);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// As step_interleaved, with the two operands' next fragments in separate LDS stages (A of
// the deep ring, B of the 32-k ring) and NDB B blocks then NDA A blocks of DMA.
template <typename OA, typename OB, int FM, int FN, int NDA, int NDB>
__device__ inline void step_deep(const s16x4 (&ca)[FM][2], const s16x4 (&cb)[FN][2],
                                 f32x16 (&acc)[FM][FN], const uint16_t* la, int kka,
                                 const uint16_t* lb, int kkb, int wm, int wn, int lane,
                                 s16x4 (&na)[FM][2], s16x4 (&nb)[FN][2], const OA& oa,
                                 const OB& ob, u32x4 rsa, u32x4 rsb, uint32_t soa, uint32_t sob,
                                 uint32_t basea, uint32_t baseb) {
    constexpr int NRA = FM * OA::PARTS, NR = NRA + FN * OB::PARTS;
    constexpr int ND = NDA + NDB;
    static_assert(NR <= FM * FN && ND <= FM * FN, "schedule slots");
#pragma unroll
    for (int i = 0; i < FM * FN; ++i) {
        const int a = i / FN, b = i % FN;
        acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat8(ca[a]), cat8(cb[b]), acc[a][b],
                                                            0, 0, 0);
        if (i < NRA) {
            OA::part(la, wm + 32 * (i / OA::PARTS), kka, lane, i % OA::PARTS, na[i / OA::PARTS]);
        } else if (i < NR) {
            const int j = i - NRA;
            OB::part(lb, wn + 32 * (j / OB::PARTS), kkb, lane, j % OB::PARTS, nb[j / OB::PARTS]);
        }
        const int d = i - (FM * FN - ND);
        if (d >= 0) {
            if (d < NDB) ob.issue_one(rsb, sob, baseb, d);
            else oa.issue_one(rsa, soa, basea, d - NDB);
        }
        __builtin_amdgcn_sched_barrier(0);
    }
}

// Wait until at most n of this wave's DMA stages (2 * PER loads each) are in flight.
template <int PER2>
__device__ inline void wait_dma_stages(int n) {
    if (PER2 == 8) {
        if (n >= 2) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else if (n == 1) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
        if (n >= 2) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        else if (n == 1) asm volatile("s_waitcnt vmcnt(4)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    }
}

// K % 32 tail (the DMA stages cover k < 32 nk): one or two 16-k steps whose operands come
// straight from global memory, zero at k >= K (and m >= M, n >= N on edge tiles) -- no
// value from outside the operands' rows enters the sums.  Lane (l32, h) supplies
// op(A)[m][k] and op(B)[k][n] for k = k16 + 8 h + e; mw, nw: the wave's first row and column.
template <bool TA, bool TB, int FM, int FN>
__device__ inline void k_tail(int M, int N, int K, int nk, const uint16_t* __restrict__ A,
                              int lda, const uint16_t* __restrict__ B, int ldb, int mw, int nw,
                              int lane, f32x16 (&acc)[FM][FN]) {
    const int l32 = lane & 31, h = lane >> 5;
    for (int k16 = 32 * nk; k16 < K; k16 += 16) {
        bf16x8 ta[FM], tb[FN];
        const int kb = k16 + 8 * h;
#pragma unroll
        for (int a = 0; a < FM; ++a) {
            const int m = mw + 32 * a + l32;
            s16x8 v;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = kb + e;
                v[e] = (m < M && k < K)
                           ? (short)(TA ? A[(size_t)k * lda + m] : A[(size_t)m * lda + k])
                           : (short)0;
            }
            ta[a] = __builtin_bit_cast(bf16x8, v);
        }
#pragma unroll
        for (int b = 0; b < FN; ++b) {
            const int n = nw + 32 * b + l32;
            s16x8 v;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = kb + e;
                v[e] = (n < N && k < K)
                           ? (short)(TB ? B[(size_t)n * ldb + k] : B[(size_t)k * ldb + n])
                           : (short)0;
            }
            tb[b] = __builtin_bit_cast(bf16x8, v);
        }
        mfma_block<FM, FN>(ta, tb, acc);
    }
}

// Register r of block (a, b) is C[32 a + 8 (r / 4) + 4 (lane / 32) + r % 4][32 b + lane % 32]
// (relative to the wave's tile): each store instruction writes two 128-byte row pieces,
// non-temporally -- C is not read again here, and streaming it past the caches leaves them
// to the A / B panels (8192^3: +3.2%, measured A/B on one box; the flash kernels' narrower
// output pieces lost 8-9% the same way, so they store normally).
// One uniform branch on the epilogue form keeps each form straight-line code.
template <int FM, int FN, int T>
__device__ inline void store_tile(int M, int N, float beta, float* __restrict__ C, int ldc,
                                  const float* __restrict__ bias, int epi, int m0, int n0, int wm,
                                  int wn, int lane, const f32x16 (&acc)[FM][FN]) {
    const int l32 = lane & 31, h = lane >> 5;
    float* cw = C + (size_t)(m0 + wm + 4 * h) * ldc + n0 + wn + l32;
    auto at = [&](int a, int b, int r) {
        return cw + (size_t)(32 * a + 8 * (r >> 2) + (r & 3)) * ldc + 32 * b;
    };
    if (m0 + T > M || n0 + T > N) {
        // Edge tile of a ragged shape: rows >= M and columns >= N hold products of the
        // zeros (or neighbouring values) the loads returned past the operands' extents and
        // are not stored; bias indices are clamped so nothing outside C or the bias is read.
        const int row0 = m0 + wm + 4 * h, col0 = n0 + wn + l32;
        const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS);
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b) {
                const int col = col0 + 32 * b;
                const float bcol = bias && !row_bias ? bias[min(col, N - 1)] : 0.f;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = row0 + 32 * a + 8 * (r >> 2) + (r & 3);
                    if (row >= M || col >= N) continue;
                    float* c = at(a, b, r);
                    float v = (beta == 0.f ? acc[a][b][r] : acc[a][b][r] + beta * *c) +
                              (row_bias ? bias[row] : bcol);
                    if (epi & DH_EPI_RELU) v = v < 0.f ? 0.f : v;
                    __builtin_nontemporal_store(v, c);
                }
            }
        return;
    }
    if (beta == 0.f && !bias && !(epi & DH_EPI_RELU)) {
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) __builtin_nontemporal_store(acc[a][b][r], at(a, b, r));
    } else {
        // C = acc + beta C + bias (by column, or by row with DH_EPI_ROW_BIAS), then max(., 0)
        // with DH_EPI_RELU (NaN passes).
        const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS);
        float bv[FN];
#pragma unroll
        for (int b = 0; b < FN; ++b)
            bv[b] = bias && !row_bias ? bias[n0 + wn + 32 * b + l32] : 0.f;
        const float* brow = row_bias ? bias + m0 + wm + 4 * h : nullptr;
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float* c = at(a, b, r);
                    float v = (beta == 0.f ? acc[a][b][r] : acc[a][b][r] + beta * *c) +
                              (row_bias ? brow[32 * a + 8 * (r >> 2) + (r & 3)] : bv[b]);
                    if (epi & DH_EPI_RELU) v = v < 0.f ? 0.f : v;
                    __builtin_nontemporal_store(v, c);
                }
    }
}

// WAVES = 4 (DH_GEMM_BF16_WAVES=4): 2 x 2 waves of 128 x 128 (one wave per SIMD, 256
// accumulators in AGPRs), reads and DMA issues interleaved op by op.
// WAVES = 8 (the default): 2 x 4 waves of 128 x 64 (two waves per SIMD, 128 accumulators
// each, so one wave's MFMAs cover the other's barrier and LDS-read gaps), which reads 1.5x the
// LDS fragment bytes per matrix-core op.  DEEP8: a k-contiguous A (NN, NT) in 64-k double
// stages on 8 waves (the default for those; off only through the tuning knob).
template <bool TA, bool TB, int WAVES, bool DEEP8>
__global__ void __launch_bounds__(64 * WAVES)
gemm_bf16_fast_kernel(int M, int N, int K, const uint16_t* __restrict__ A, int lda,
                      const uint16_t* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                      int ldc, long long sA, long long sB, long long sC,
                      const float* __restrict__ bias, int epi, int tile0, int tail) {
    A += blockIdx.y * sA;   // batch member blockIdx.y
    B += blockIdx.y * sB;
    C += blockIdx.y * sC;
    using OA = FastOperand<!TA, WAVES>;
    using OB = FastOperand<TB, WAVES>;
    constexpr int WN_CNT = WAVES / 2;                 // waves along N
    constexpr int FM = 4, FN = 4 / (WAVES / 4);       // 128 x (128 or 64) per wave
    // Ring of FAST_NSTAGE stages, each an A tile then a B tile.  Stage kt + 3 is fetched
    // while stage kt is consumed, so every DMA has three stages of MFMA work to land.  With a
    // k-contiguous A (NN, NT; on 4 waves, or on 8 with DEEP8) A is instead held in 3 double
    // stages of 64 k and B in 4 stages of 32 k: 96 + 64 = 160 KB.
    constexpr bool DEEP_A = !TA && (WAVES == 4 || DEEP8);
    using DK = DeepKOperand<WAVES>;
    constexpr int RING = DEEP_A ? 3 * DK::ELEMS + FAST_NSTAGE * FAST_TILE
                                : FAST_NSTAGE * 2 * FAST_TILE;
    __shared__ __attribute__((aligned(16))) uint16_t ring[RING];

    const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    int tm, tn;
    // Each XCD's 32 tiles in flight form a 4 x 8 block (4 A panels, 8 B panels).  Same-box
    // A/B at 8192^3 (NN, ms): groups of 4 tile rows 0.862-0.867, 8 rows (8 x 4 blocks)
    // 0.879-0.881, 2: 0.893, 3: 0.889, 5: 0.894, 6: 0.885, 16: 0.903.
    // tail: the K chunk blockIdx.y of logical tile tile0 + blockIdx.x (no XCD remap)
    if (tail) grouped_tile(tile0 + blockIdx.x, tiles_m, tiles_n, 4, tm, tn);
    else xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 4, tm, tn);
    const int m0 = tm * 256, n0 = tn * 256;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int l32 = lane & 31, h = lane >> 5;
    const int wm = (wave / WN_CNT) * 128, wn = (wave % WN_CNT) * (256 / WN_CNT);

    OA oa;
    OB ob;
    oa.init(lda, TA ? K : M, m0, wave, lane);
    ob.init(ldb, TB ? N : K, n0, wave, lane);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    const int nk = K / 32;
    if constexpr (DEEP_A) {
        // A in double stages (pair p = stages 2p, 2p+1, slot p % 3), B in 32-k stages (slot
        // kt % 4).  Issue order: pair p at stage 2p - 4, B stage s at stage s - 3, pairs after
        // B within a stage; past the end both are clamped to the last pair / stage (refetched
        // into a slot nobody reads any more), so the counts are constant: at the barrier of
        // stage kt, stage kt+1 must have landed while the 24 (kt even) or 16 (kt odd) younger
        // loads may still be in flight.
        DK da;
        da.init(lda, M, m0, wave, lane);
        const u32x4 rsa = make_rsrc(A, da.bytes), rsb = make_rsrc(B, ob.bytes);
        uint16_t* const ring_a = ring;
        uint16_t* const ring_b = ring + 3 * DK::ELEMS;
        const int npair = (nk + 1) / 2;
        auto a_slot = [&](int p) { return ring_a + (p % 3) * DK::ELEMS; };
        auto b_slot = [&](int st) { return ring_b + (st % FAST_NSTAGE) * FAST_TILE; };
        auto a_dma = [&](int p, uint32_t& base, uint32_t& soff) {
            base = __builtin_amdgcn_readfirstlane(lds_addr(a_slot(p)) + 1024u * DK::PER * wave);
            soff = __builtin_amdgcn_readfirstlane((uint32_t)min(p, npair - 1) * DK::STEP);
        };
        auto b_dma = [&](int st, uint32_t& base, uint32_t& soff) {
            base = __builtin_amdgcn_readfirstlane(lds_addr(b_slot(st)) + 1024u * OB::PER * wave);
            soff = __builtin_amdgcn_readfirstlane((uint32_t)min(st, nk - 1) * ob.step);
        };
        auto issue_a = [&](int p) {
            uint32_t base, soff;
            a_dma(p, base, soff);
#pragma unroll
            for (int t = 0; t < DK::PER; ++t) da.issue_one(rsa, soff, base, t);
        };
        auto issue_b = [&](int st) {
            uint32_t base, soff;
            b_dma(st, base, soff);
#pragma unroll
            for (int t = 0; t < OB::PER; ++t) ob.issue_one(rsb, soff, base, t);
        };
        // vmcnt constants below: 4 waves issue 8 A blocks per pair and 4 B blocks per stage,
        // 8 waves half as many
        static_assert(OB::PER == 16 / WAVES && DK::PER == 32 / WAVES, "vmcnt constants below");
        issue_a(0);
        issue_b(0);
        issue_b(1);
        issue_a(1);
        issue_b(2);
        if constexpr (WAVES == 4) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        else asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
        __syncthreads();
        asm volatile("" ::"s"(C), "s"(ldc), "s"(beta), "s"(bias), "s"(epi));
        s16x4 f0a[FM][2], f0b[FN][2], f1a[FM][2], f1b[FN][2];
#pragma unroll
        for (int x = 0; x < FM; ++x) DK::part(a_slot(0), wm + 32 * x, 0, lane, 0, f0a[x]);
#pragma unroll
        for (int x = 0; x < FN; ++x)
#pragma unroll
            for (int q = 0; q < OB::PARTS; ++q) OB::part(b_slot(0), wn + 32 * x, 0, lane, q, f0b[x]);
        // Stage kt: X = MFMA f0 | reads of k-step 1 -> f1 | DMA B kt+3 (+ A pair kt/2 + 2 when kt
        // is even); barrier; Y = MFMA f1 | reads of stage kt+1 k-step 0 -> f0.
        auto body = [&](int kt, auto even_tag) {
            constexpr bool EVEN = decltype(even_tag)::value;
            uint32_t ba = 0, sa = 0, bb, sb;
            if (EVEN) a_dma(kt / 2 + 2, ba, sa);
            b_dma(kt + 3, bb, sb);
            step_deep<DK, OB, FM, FN, EVEN ? DK::PER : 0, OB::PER>(
                f0a, f0b, acc, a_slot(kt / 2), 2 * (kt & 1) + 1, b_slot(kt), 1, wm, wn, lane, f1a,
                f1b, da, ob, rsa, rsb, sa, sb, ba, bb);
            if constexpr (WAVES == 4) {
                if (EVEN) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(24)" ::: "memory");
                else asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(16)" ::: "memory");
            } else {
                if (EVEN) asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(12)" ::: "memory");
                else asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(8)" ::: "memory");
            }
            __syncthreads();
            step_deep<DK, OB, FM, FN, 0, 0>(
                f1a, f1b, acc, a_slot((kt + 1) / 2), 2 * ((kt + 1) & 1), b_slot(kt + 1), 0, wm, wn,
                lane, f0a, f0b, da, ob, rsa, rsb, 0u, 0u, 0u, 0u);
        };
        using Even = std::integral_constant<bool, true>;
        using Odd = std::integral_constant<bool, false>;
        int kt = 0;
        for (; kt + 2 < nk; kt += 2) {
            body(kt, Even{});
            body(kt + 1, Odd{});
        }
        if (kt + 1 < nk) {
            body(kt, Even{});
            ++kt;
        }
        // last stage kt = nk - 1: k-step 1 from its slots, then its MFMAs
        step_deep<DK, OB, FM, FN, 0, 0>(f0a, f0b, acc, a_slot(kt / 2), 2 * (kt & 1) + 1,
                                                  b_slot(kt), 1, wm, wn, lane, f1a, f1b, da, ob,
                                                  rsa, rsb, 0u, 0u, 0u, 0u);
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat8(f1a[a]), cat8(f1b[b]),
                                                                    acc[a][b], 0, 0, 0);
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // refetches land before exit
    } else if constexpr (WAVES == 4) {
        // One wave per SIMD, 128 x 128 each: half the LDS fragment traffic per matrix-core op
        // of the two-wave form, with the reads and DMA issues interleaved op by op.  Stage
        // indices past the last stage are clamped (the last stage is fetched again into a
        // slot nobody reads any more), so every stage issues the same DMA count and the
        // waits are constants: before the barrier of stage kt, stage kt+1 must have landed
        // while kt+2 and kt+3 may still be in flight.
        const u32x4 rsa = make_rsrc(A, oa.bytes), rsb = make_rsrc(B, ob.bytes);
        auto slot_bases = [&](int s, uint32_t& ba, uint32_t& bb) {
            const uint32_t st = lds_addr(ring + (s % FAST_NSTAGE) * 2 * FAST_TILE);
            ba = __builtin_amdgcn_readfirstlane(st + 1024u * OA::PER * wave);
            bb = __builtin_amdgcn_readfirstlane(st + 2u * FAST_TILE + 1024u * OB::PER * wave);
        };
        auto soffs = [&](int s, uint32_t& sa, uint32_t& sb) {
            const uint32_t k = (uint32_t)min(s, nk - 1);
            sa = __builtin_amdgcn_readfirstlane(k * oa.step);
            sb = __builtin_amdgcn_readfirstlane(k * ob.step);
        };
        for (int s = 0; s < FAST_NSTAGE - 1; ++s) {
            uint32_t ba, bb, sa, sb;
            slot_bases(s, ba, bb);
            soffs(s, sa, sb);
#pragma unroll
            for (int t = 0; t < OA::PER; ++t) oa.issue_one(rsa, sa, ba, t);
#pragma unroll
            for (int t = 0; t < OB::PER; ++t) ob.issue_one(rsb, sb, bb, t);
        }
        static_assert(2 * (OA::PER + OB::PER) == 16, "vmcnt below assumes 8 DMAs per stage");
        asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
        __syncthreads();
        asm volatile("" ::"s"(C), "s"(ldc), "s"(beta), "s"(bias), "s"(epi));
        s16x4 f0a[FM][2], f0b[FN][2], f1a[FM][2], f1b[FN][2];
#pragma unroll
        for (int x = 0; x < FM; ++x)
#pragma unroll
            for (int q = 0; q < OA::PARTS; ++q) OA::part(ring, wm + 32 * x, 0, lane, q, f0a[x]);
#pragma unroll
        for (int x = 0; x < FN; ++x)
#pragma unroll
            for (int q = 0; q < OB::PARTS; ++q)
                OB::part(ring + FAST_TILE, wn + 32 * x, 0, lane, q, f0b[x]);
        for (int kt = 0; kt < nk - 1; ++kt) {
            uint32_t ba, bb, sa, sb;
            slot_bases(kt + FAST_NSTAGE - 1, ba, bb);
            soffs(kt + FAST_NSTAGE - 1, sa, sb);
            step_interleaved<OA, OB, FM, FN, true>(f0a, f0b, acc, ring + (kt % FAST_NSTAGE) * 2 * FAST_TILE,
                                                   1, wm, wn, lane, f1a, f1b, oa, ob, rsa, rsb,
                                                   sa, sb, ba, bb);
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_waitcnt vmcnt(16)" ::: "memory");
            __syncthreads();
            step_interleaved<OA, OB, FM, FN, false>(
                f1a, f1b, acc, ring + ((kt + 1) % FAST_NSTAGE) * 2 * FAST_TILE, 0, wm, wn, lane,
                f0a, f0b, oa, ob, rsa, rsb, 0u, 0u, 0u, 0u);
        }
        step_interleaved<OA, OB, FM, FN, false>(f0a, f0b, acc,
                                                ring + ((nk - 1) % FAST_NSTAGE) * 2 * FAST_TILE, 1,
                                                wm, wn, lane, f1a, f1b, oa, ob, rsa, rsb, 0u, 0u,
                                                0u, 0u);
#pragma unroll
        for (int a = 0; a < FM; ++a)
#pragma unroll
            for (int b = 0; b < FN; ++b)
                acc[a][b] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(cat8(f1a[a]), cat8(f1b[b]),
                                                                    acc[a][b], 0, 0, 0);
        // The clamped refetches may still be landing in free slots: drain them before the
        // work-group can end and its LDS be handed to another.
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    } else {
    auto issue = [&](int kt) {
        uint16_t* st = ring + (kt % FAST_NSTAGE) * 2 * FAST_TILE;
        oa.issue(A, kt, st, wave);
        ob.issue(B, kt, st + FAST_TILE, wave);
    };
    auto stage_ptr = [&](int kt) { return ring + (kt % FAST_NSTAGE) * 2 * FAST_TILE; };
    const int pre = nk < FAST_NSTAGE - 1 ? nk : FAST_NSTAGE - 1;
    for (int s = 0; s < pre; ++s) issue(s);
    wait_dma_stages<2 * OA::PER>(pre - 1);
    __syncthreads();
    // Software pipeline per 32-k stage kt (fragments of k-step 0 already in f0):
    //   DMA stage kt+3 | read k-step 1 -> f1 | MFMA f0 | wait LDS reads + DMA of kt+1 |
    //   barrier | read k-step 0 of kt+1 -> f0 | MFMA f1
    // The matrix cores run f0 across the barrier wait and f1 across the next reads.  A
    // ring slot is refilled (DMA kt+3 -> slot of kt-1) only after the barrier that follows
    // every wave's last read of it.
    // The last stage is peeled off the loop: with it inside, the compiler's wait before
    // the f1 block has to cover a path without the trailing reads and waits for those
    // reads too, so they would no longer overlap the f1 MFMAs.
    // The epilogue's kernel arguments are fetched here: a scalar load still in flight at
    // the loop entry would make every LDS wait in the loop a full lgkmcnt(0).
    asm volatile("" ::"s"(C), "s"(ldc), "s"(beta), "s"(bias), "s"(epi));
    bf16x8 f0a[FM], f0b[FN], f1a[FM], f1b[FN];
    load_frags<OA, OB, FM, FN>(stage_ptr(0), 0, wm, wn, lane, f0a, f0b);
    for (int kt = 0; kt < nk - 1; ++kt) {
        if (kt + FAST_NSTAGE - 1 < nk) issue(kt + FAST_NSTAGE - 1);
        load_frags<OA, OB, FM, FN>(stage_ptr(kt), 1, wm, wn, lane, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        mfma_block<FM, FN>(f0a, f0b, acc);
        __builtin_amdgcn_sched_barrier(0);
        const int ahead = min(nk - 1, kt + FAST_NSTAGE - 1) - (kt + 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_dma_stages<2 * OA::PER>(ahead);
        __syncthreads();
        load_frags<OA, OB, FM, FN>(stage_ptr(kt + 1), 0, wm, wn, lane, f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        mfma_block<FM, FN>(f1a, f1b, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    load_frags<OA, OB, FM, FN>(stage_ptr(nk - 1), 1, wm, wn, lane, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    mfma_block<FM, FN>(f0a, f0b, acc);
    mfma_block<FM, FN>(f1a, f1b, acc);
    }

    k_tail<TA, TB, FM, FN>(M, N, K, nk, A, lda, B, ldb, m0 + wm, n0 + wn, lane, acc);
    if (tail) {   // the tile's fp32 partial, compact: 256 x 256 at C + 65536 blockIdx.x
        store_tile<FM, FN, 256>(min(M - m0, 256), min(N - n0, 256), 0.f,
                                C + (size_t)blockIdx.x * 65536, 256, nullptr, 0, 0, 0, wm, wn,
                                lane, acc);
        return;
    }
    store_tile<FM, FN, 256>(M, N, beta, C, ldc, bias, epi, m0, n0, wm, wn, lane, acc);
}

// The partial last round of a split product (launch_fast): C = beta C + sum_s part[s] (in
// order, so reruns are bit-identical) + bias, then ReLU, for the R tail tiles (logical tiles
// tile0 + r), each part[s] tile compact (256 x 256, row stride 256, tile r at 65536 r, chunk s
// at sstride s).  Work-group (r, 4-row block), 4 columns per thread.
__global__ void __launch_bounds__(256)
tail_reduce(const float* __restrict__ part, int S, long long sstride, int tile0, int tiles_m,
            int tiles_n, int M, int N, float beta, float* __restrict__ C, int ldc,
            const float* __restrict__ bias, int epi) {
    const int r = blockIdx.x >> 6, i = 4 * (blockIdx.x & 63) + (threadIdx.x >> 6);
    const int j = 4 * (threadIdx.x & 63);
    int tm, tn;
    grouped_tile(tile0 + r, tiles_m, tiles_n, 4, tm, tn);
    const int row = tm * 256 + i, col0 = tn * 256 + j;
    if (row >= M || col0 >= N) return;
    const float* p = part + (size_t)r * 65536 + i * 256 + j;
    f32x4 v = *reinterpret_cast<const f32x4*>(p);
    for (int s = 1; s < S; ++s) v += *reinterpret_cast<const f32x4*>(p + s * sstride);
    const bool row_bias = bias && (epi & DH_EPI_ROW_BIAS);
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int col = col0 + e;
        if (col >= N) break;
        float* c = C + (size_t)row * ldc + col;
        float x = (beta == 0.f ? v[e] : v[e] + beta * *c) + (bias ? bias[row_bias ? row : col] : 0.f);
        if (epi & DH_EPI_RELU) x = x < 0.f ? 0.f : x;
        *c = x;
    }
}

// ---------------------------------------------------------------------------------
// Mid-size path: 128 x 128 tiles for shapes whose 256 x 256 tiles leave the CUs short of one
// round (2048^3: 64 tiles of 256 against 256 of 128).  The fast path's direct-to-LDS ring in
// 32-k stages of 128-wide tiles (8 KB per operand and stage, four stages = 64 KB, so two
// work-groups fit a CU); 4 waves as 2 x 2 of 64 x 64 (2 x 2 MFMA blocks each), the same
// software pipeline as the 8-wave fast loop: DMA of stage kt+3 | reads of k-step 1 | MFMAs
// of k-step 0 | wait + barrier | reads of stage kt+1's k-step 0 | MFMAs of k-step 1.  Same
// contract for ragged shapes (edge tiles, masked K tail) as the fast path.
// ---------------------------------------------------------------------------------
constexpr int MID_TILE = 128 * 32;    // elements of one operand stage (32 k)
constexpr int MID_NSTAGE = 4;         // LDS ring: 4 x (A + B) x 8 KB = 64 KB

template <bool TA, bool TB>
__global__ void __launch_bounds__(256)
gemm_bf16_mid_kernel(int M, int N, int K, const uint16_t* __restrict__ A, int lda,
                     const uint16_t* __restrict__ B, int ldb, float beta, float* __restrict__ C,
                     int ldc, long long sA, long long sB, long long sC,
                     const float* __restrict__ bias, int epi) {
    A += blockIdx.y * sA;   // batch member blockIdx.y
    B += blockIdx.y * sB;
    C += blockIdx.y * sC;
    using OA = FastOperand<!TA, 4, 128>;
    using OB = FastOperand<TB, 4, 128>;
    constexpr int FM = 2, FN = 2;
    __shared__ __attribute__((aligned(16))) uint16_t ring[MID_NSTAGE * 2 * MID_TILE];

    const int tiles_m = (M + 127) / 128, tiles_n = (N + 127) / 128;
    int tm, tn;
    xcd_tile_order(blockIdx.x, gridDim.x, tiles_m, tiles_n, 4, tm, tn);
    const int m0 = tm * 128, n0 = tn * 128;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    OA oa;
    OB ob;
    oa.init(lda, TA ? K : M, m0, wave, lane);
    ob.init(ldb, TB ? N : K, n0, wave, lane);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int a = 0; a < FM; ++a)
#pragma unroll
        for (int b = 0; b < FN; ++b)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[a][b][r] = 0.f;

    const int nk = K / 32;   // >= 1 (the host sends K < 32 elsewhere)
    auto stage_ptr = [&](int kt) { return ring + (kt % MID_NSTAGE) * 2 * MID_TILE; };
    auto issue = [&](int kt) {
        uint16_t* st = stage_ptr(kt);
        oa.issue(A, kt, st, wave);
        ob.issue(B, kt, st + MID_TILE, wave);
    };
    const int pre = nk < MID_NSTAGE - 1 ? nk : MID_NSTAGE - 1;
    for (int s = 0; s < pre; ++s) issue(s);
    static_assert(OA::PER == 2 && OB::PER == 2, "wait_dma_stages<4>: 4 loads per stage");
    wait_dma_stages<2 * OA::PER>(pre - 1);
    __syncthreads();
    asm volatile("" ::"s"(C), "s"(ldc), "s"(beta), "s"(bias), "s"(epi));
    bf16x8 f0a[FM], f0b[FN], f1a[FM], f1b[FN];
    load_frags<OA, OB, FM, FN, MID_TILE>(stage_ptr(0), 0, wm, wn, lane, f0a, f0b);
    for (int kt = 0; kt < nk - 1; ++kt) {
        if (kt + MID_NSTAGE - 1 < nk) issue(kt + MID_NSTAGE - 1);
        load_frags<OA, OB, FM, FN, MID_TILE>(stage_ptr(kt), 1, wm, wn, lane, f1a, f1b);
        __builtin_amdgcn_sched_barrier(0);
        mfma_block<FM, FN>(f0a, f0b, acc);
        __builtin_amdgcn_sched_barrier(0);
        const int ahead = min(nk - 1, kt + MID_NSTAGE - 1) - (kt + 1);
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        wait_dma_stages<2 * OA::PER>(ahead);
        __syncthreads();
        load_frags<OA, OB, FM, FN, MID_TILE>(stage_ptr(kt + 1), 0, wm, wn, lane, f0a, f0b);
        __builtin_amdgcn_sched_barrier(0);
        mfma_block<FM, FN>(f1a, f1b, acc);
        __builtin_amdgcn_sched_barrier(0);
    }
    load_frags<OA, OB, FM, FN, MID_TILE>(stage_ptr(nk - 1), 1, wm, wn, lane, f1a, f1b);
    __builtin_amdgcn_sched_barrier(0);
    mfma_block<FM, FN>(f0a, f0b, acc);
    mfma_block<FM, FN>(f1a, f1b, acc);

    k_tail<TA, TB, FM, FN>(M, N, K, nk, A, lda, B, ldb, m0 + wm, n0 + wn, lane, acc);
    store_tile<FM, FN, 128>(M, N, beta, C, ldc, bias, epi, m0, n0, wm, wn, lane, acc);
}

template <bool TA, bool TB>
int launch_fast(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                float beta, float* C, int ldc, const Batch& bt) {
    // Default: 8 waves (two per SIMD), with A in 64-k double stages when it is k-contiguous
    // (NN, NT).  Same-box A/B at 8192^3 (ms): NN 0.803 (8 waves, 64-k A) / 0.860 (8 waves, 32-k
    // A) / 0.85-0.87 (4 waves, 64-k A); NT 0.795 / 0.857 / 0.836.  TN and TT (k-contiguous B
    // only): within 1-3% of each other on 4 and 8 waves at 8192^3 and 4096^3 (either ahead,
    // by box), and 8 waves ahead at shorter K: 8192 x 8192 x 1024 TN 176 against 226 us, TT 176
    // against 195; K = 2048 TN 287 against 323 us.  The 32-k stages fetch half an L2 line per row of a
    // k-contiguous operand (the next stage fetches the other half again): 40% more L2
    // requests than the vendor library for the same bytes.
    static const int env_waves = [] {
        const char* e = std::getenv("DH_GEMM_BF16_WAVES");   // tuning knob: 4 or 8
        return e ? (std::atoi(e) == 8 ? 8 : 4) : 0;
    }();
    const int waves = env_waves ? env_waves : 8;
    static const bool deep8 = [] {
        const char* e = std::getenv("DH_GEMM_BF16_DEEP8");   // tuning knob: 0 or 1
        return !e || std::atoi(e) != 0;
    }();
    auto kern = waves == 4 ? gemm_bf16_fast_kernel<TA, TB, 4, false>
              : deep8      ? gemm_bf16_fast_kernel<TA, TB, 8, true>
                           : gemm_bf16_fast_kernel<TA, TB, 8, false>;
    const int tiles_m = (M + 255) / 256, tiles_n = (N + 255) / 256;
    const int tiles = tiles_m * tiles_n, cus = num_cus();
    // One product with K >= 4096 whose last round of tiles fills at most half the CUs: the
    // full rounds as usual, then the R tiles of the last round split into S chunks of K (a
    // multiple of 64, the last chunk taking the rest) whose fp32 partials tail_reduce adds in
    // order with the epilogue: the last round takes about 1/S of a tile's time instead of a
    // whole one, for two more launches and 8 S R 256^2 bytes of partials.  Same box, µs:
    // 7000^3 754 -> 701, 4352^3 196 -> 191 (TN 218 -> 204); at K = 1000 and 2048 (4300 x
    // 4400, 4608 x 4096) the extra launches and partials cost more than they save (83 -> 98,
    // 107 -> 120), hence the bound on K.
    static const bool split_tail = [] {
        const char* e = std::getenv("DH_GEMM_BF16_SPLIT_TAIL");   // tuning knob: 0 or 1
        return !e || std::atoi(e) != 0;
    }();
    const int R = tiles % cus;
    int S = R > 0 ? cus / R : 0;
    if (S > K / 256) S = K / 256;
    if (split_tail && bt.count == 1 && K >= 4096 && tiles > cus && 2 * R <= cus && S >= 2) {
        const int Kc = K / S / 64 * 64;
        const long long cstride = 65536LL * R;
        float* part = static_cast<float*>(dh_malloc((size_t)S * cstride * sizeof(float)));
        if (part) {
            const int full = tiles - R;
            kern<<<dim3(full, 1), 64 * waves, 0, stream()>>>(M, N, K, A, lda, B, ldb, beta, C, ldc,
                                                            0, 0, 0, bt.bias, bt.epi, 0, 0);
            int st = check_launch("dh_gemm_bf16(fast)");
            const long long sA = TA ? (long long)Kc * lda : Kc, sB = TB ? Kc : (long long)Kc * ldb;
            if (st == DH_OK) {
                kern<<<dim3(R, S - 1), 64 * waves, 0, stream()>>>(
                    M, N, Kc, A, lda, B, ldb, 0.f, part, 256, sA, sB, cstride, nullptr, 0, full, 1);
                st = check_launch("dh_gemm_bf16(fast, split tail)");
            }
            if (st == DH_OK) {
                kern<<<dim3(R, 1), 64 * waves, 0, stream()>>>(
                    M, N, K - (S - 1) * Kc, A + (S - 1) * sA, lda, B + (S - 1) * sB, ldb, 0.f,
                    part + (S - 1) * cstride, 256, 0, 0, 0, nullptr, 0, full, 1);
                st = check_launch("dh_gemm_bf16(fast, split tail)");
            }
            if (st == DH_OK) {
                tail_reduce<<<R * 64, 256, 0, stream()>>>(part, S, cstride, full, tiles_m, tiles_n,
                                                          M, N, beta, C, ldc, bt.bias, bt.epi);
                st = check_launch("dh_gemm_bf16(split tail reduce)");
            }
            dh_free(part);   // pooled; later users of the buffer are ordered on the stream
            return st;
        }
        // no workspace: the plain grid
    }
    for (int b0 = 0; b0 < bt.count; b0 += 65535) {   // gridDim.y = batch member
        const int nb = bt.count - b0 < 65535 ? bt.count - b0 : 65535;
        kern<<<dim3(tiles, nb), 64 * waves, 0, stream()>>>(
            M, N, K, A + b0 * bt.sA, lda, B + b0 * bt.sB, ldb, beta, C + b0 * bt.sC, ldc, bt.sA,
            bt.sB, bt.sC, bt.bias, bt.epi, 0, 0);
        DH_TRY(check_launch("dh_gemm_bf16(fast)"));
    }
    return DH_OK;
}

template <bool TA, bool TB>
int launch_mid_grid(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                    float beta, float* C, int ldc, const Batch& bt) {
    for (int b0 = 0; b0 < bt.count; b0 += 65535) {   // gridDim.y = batch member
        const int nb = bt.count - b0 < 65535 ? bt.count - b0 : 65535;
        gemm_bf16_mid_kernel<TA, TB><<<dim3(((M + 127) / 128) * ((N + 127) / 128), nb), 256, 0,
                                       stream()>>>(
            M, N, K, A + b0 * bt.sA, lda, B + b0 * bt.sB, ldb, beta, C + b0 * bt.sC, ldc, bt.sA,
            bt.sB, bt.sC, bt.bias, bt.epi);
        DH_TRY(check_launch("dh_gemm_bf16(mid)"));
    }
    return DH_OK;
}

// One product whose 128 x 128 tiles fill at most half the CUs with a long contraction (weight
// gradients, K = the batch; 512 x 512 x 8192) splits K into S chunks of Kc (a multiple of 32,
// the last chunk taking the rest) run as batch members of the same kernel, each writing an fp32
// partial, which splitk_reduce_launch adds in a fixed order (reruns stay bit-identical) with
// beta, the bias and ReLU.  The partials cost 8 S M N bytes of HBM traffic, so S aims at only
// 2 work-groups per CU, at most 16 chunks of at least 256, and K below 2048 is not split
// (1024^3: 13.4 us unsplit against 27.7 us in 8 chunks; 512^2 x 8192: 79 us unsplit, 34 us in
// 32 chunks).
template <bool TA, bool TB>
int launch_mid(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
               float beta, float* C, int ldc, const Batch& bt) {
    const int tiles = ((M + 127) / 128) * ((N + 127) / 128);
    const int cus = num_cus();
    static const bool split_on = [] {
        const char* e = std::getenv("DH_GEMM_BF16_SPLITK");   // tuning knob: 0 or 1
        return !e || std::atoi(e) != 0;
    }();
    if (split_on && bt.count == 1 && 2 * tiles <= cus && K >= 2048) {
        int S = 2 * cus / tiles;
        S = S > 16 ? 16 : S;
        S = S > K / 256 ? K / 256 : S;
        const int Kc = K / S / 32 * 32;
        float* part = static_cast<float*>(dh_malloc((size_t)S * M * N * sizeof(float)));
        if (part) {
            const long long MN = (long long)M * N;
            const Batch pb{TA ? (long long)Kc * lda : Kc, TB ? Kc : (long long)Kc * ldb, MN, S - 1,
                           nullptr, 0};
            int st = launch_mid_grid<TA, TB>(M, N, Kc, A, lda, B, ldb, 0.f, part, N, pb);
            if (st == DH_OK)
                st = launch_mid_grid<TA, TB>(M, N, K - (S - 1) * Kc, A + (S - 1) * pb.sA, lda,
                                             B + (S - 1) * pb.sB, ldb, 0.f, part + (S - 1) * MN, N,
                                             Batch{0, 0, 0, 1, nullptr, 0});
            if (st == DH_OK) st = splitk_reduce_launch(part, S, M, N, beta, C, ldc, bt.bias, bt.epi);
            dh_free(part);   // pooled; later users of the buffer are ordered on the stream
            return st;
        }
        // no workspace: the one-pass grid
    }
    return launch_mid_grid<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

template <bool TA, bool TB>
int launch_general(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
                   float beta, float* C, int ldc, const Batch& bt) {
    const bool va = ((uintptr_t)A % 16 == 0) && (lda % 8 == 0) && (bt.sA % 8 == 0);
    const bool vb = ((uintptr_t)B % 16 == 0) && (ldb % 8 == 0) && (bt.sB % 8 == 0);
    if (va && vb) return launch_vec<TA, TB, true, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    if (va) return launch_vec<TA, TB, true, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    if (vb) return launch_vec<TA, TB, false, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    return launch_vec<TA, TB, false, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

// Rows of cols bf16 values at leading dimension ld -> rows at ldo (a multiple of 8, dst
// 16-byte aligned), zero-filled to ldo: 16 bytes per thread and store, grid-stride.
__global__ __launch_bounds__(256) void copy_rows_bf16(const uint16_t* __restrict__ src, int ld,
                                                     uint16_t* __restrict__ dst, int ldo,
                                                     int rows, int cols) {
    const int chunks = ldo / 8;
    const long long total = (long long)rows * chunks;
    for (long long x = (long long)blockIdx.x * 256 + threadIdx.x; x < total;
         x += (long long)gridDim.x * 256) {
        const int r = (int)(x / chunks), c = (int)(x - (long long)r * chunks) * 8;
        const uint16_t* sp = src + (size_t)r * ld + c;
        s16x8 v;
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = c + e < cols ? (short)sp[e] : (short)0;
        *reinterpret_cast<s16x8*>(dst + (size_t)r * ldo + c) = v;
    }
}

// A stored operand (rows x cols, leading dimension ld) copied to pool memory with 16-byte
// aligned rows (leading dimension cols rounded up to 8, zero-padded).
uint16_t* aligned_copy(const uint16_t* src, int rows, int cols, int ld, int& ld_out) {
    ld_out = (cols + 7) & ~7;
    uint16_t* d = static_cast<uint16_t*>(dh_malloc((size_t)rows * ld_out * sizeof(uint16_t)));
    if (!d) return nullptr;
    const long long total = (long long)rows * (ld_out / 8);
    long long blocks = (total + 255) / 256;
    if (blocks > 8LL * num_cus()) blocks = 8LL * num_cus();
    copy_rows_bf16<<<(unsigned)blocks, 256, 0, stream()>>>(src, ld, d, ld_out, rows, cols);
    if (check_launch("dh_gemm_bf16(aligned copy)") != DH_OK) {
        dh_free(d);
        return nullptr;
    }
    return d;
}

template <bool TA, bool TB>
int launch(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
           float beta, float* C, int ldc, const Batch& bt) {
    // The direct-to-LDS paths need 16-byte operand rows (aligned bases, leading dimensions
    // and batch strides in multiples of 8 elements): 256 x 256 tiles when there are more of
    // them than half the CUs, else 128 x 128 (DH_GEMM_BF16_MID=0 sends those shapes to the
    // general kernel instead).  Between half a round and a round the 256 tiles, one per CU
    // with some CUs idle, still beat four times as many 128 tiles (same box: 3840^3 125 against
    // 158 us, 3072^3 79 against 99 us; 2048 x 4096, 128 tiles, 45-50 us either way).  Ragged M and N are edge tiles, a K that is not a multiple of
    // 32 ends with the kernels' masked tail steps (a DMA'd k-contiguous tile would read the
    // next row's values, possibly non-finite, past K); rows that are not 16-byte aligned are
    // copied to aligned ones first (one product, and for the 128 x 128 path one of at least
    // 2^22 multiply-adds: a pass over the operand and a launch, where the general kernel on
    // such rows takes ~5-10x the direct-to-LDS time).
    static const bool mid_on = [] {
        const char* e = std::getenv("DH_GEMM_BF16_MID");   // tuning knob: 0 or 1
        return !e || std::atoi(e) != 0;
    }();
    const long long tiles = (long long)((M + 255) / 256) * ((N + 255) / 256) * bt.count;
    static const int mid_max = [] {   // tuning knob: most 256 x 256 tiles for the 128 path
        const char* e = std::getenv("DH_GEMM_BF16_MID_MAX_TILES");
        return e ? std::atoi(e) : -1;   // default: num_cus() / 2
    }();
    const bool mid = tiles <= (mid_max >= 0 ? mid_max : num_cus() / 2);
    const int K32 = K - K % 32;
    const long long a_bytes = 2LL * ((TA ? K : M) + 255) * lda,
                    b_bytes = 2LL * ((TB ? N : K) + 255) * ldb;
    if (K32 == 0 || (mid && !mid_on) || a_bytes >= (1LL << 32) || b_bytes >= (1LL << 32))
        return launch_general<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    const bool va = ((uintptr_t)A % 16 == 0) && (lda % 8 == 0) && (bt.sA % 8 == 0);
    const bool vb = ((uintptr_t)B % 16 == 0) && (ldb % 8 == 0) && (bt.sB % 8 == 0);
    if (!va || !vb) {
        if (bt.count > 1 || (mid && (long long)M * N * K < (1LL << 22)))
            return launch_general<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        int la = lda, lb = ldb;
        uint16_t* a2 = va ? nullptr : aligned_copy(A, TA ? K : M, TA ? M : K, lda, la);
        uint16_t* b2 = vb ? nullptr : aligned_copy(B, TB ? N : K, TB ? K : N, ldb, lb);
        int st;
        if ((!va && !a2) || (!vb && !b2))
            st = launch_general<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
        else
            st = launch<TA, TB>(M, N, K, a2 ? a2 : A, la, b2 ? b2 : B, lb, beta, C, ldc, bt);
        if (a2) dh_free(a2);   // pooled: stream order keeps them alive for the queued work
        if (b2) dh_free(b2);
        return st;
    }
    return mid ? launch_mid<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt)
               : launch_fast<TA, TB>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" int dh_gemm_bf16_ex(int transA, int transB, int M, int N, int K, const uint16_t* A,
                               int lda, long long strideA, const uint16_t* B, int ldb,
                               long long strideB, float beta, float* C, int ldc,
                               long long strideC, int batch, const float* bias, int epilogue) {
    DH_TRY(ensure_init());
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: negative shape");
    if (M == 0 || N == 0 || batch == 0) return DH_OK;
    if (!C || (K > 0 && (!A || !B)))
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: null pointer");
    // A and B are not read when K == 0, so only C's leading dimension matters then.
    if (ldc < N || (K > 0 && (lda < (transA ? M : K) || ldb < (transB ? K : N))))
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: leading dimension too small");
    if (batch > 1 && (strideA < 0 || strideB < 0 || strideC < (long long)(M - 1) * ldc + N))
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: batch strides overlap C or are negative");
    const Batch bt{batch > 1 ? strideA : 0, batch > 1 ? strideB : 0, batch > 1 ? strideC : 0,
                   batch, bias, epilogue};
    if (transA)
        return transB ? launch<true, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt)
                      : launch<true, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
    return transB ? launch<false, true>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt)
                  : launch<false, false>(M, N, K, A, lda, B, ldb, beta, C, ldc, bt);
}

extern "C" int dh_gemm_bf16(int transA, int transB, int M, int N, int K, const uint16_t* A,
                            int lda, const uint16_t* B, int ldb, float beta, float* C, int ldc) {
    return dh_gemm_bf16_ex(transA, transB, M, N, K, A, lda, 0, B, ldb, 0, beta, C, ldc, 0, 1,
                           nullptr, 0);
}
