// dh_gemm_bf16.hip -- bf16 x bf16 -> fp32 GEMM on gfx950 (v_mfma_f32_32x32x16_bf16).
//
// Same contract as dh_gemm_f32 (NN / NT / TN / TT, beta), with bf16 operands and fp32
// accumulation and output.  Replaces the reference's fp16 cublasGemmEx branch
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
                 int ldc) {
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
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm + 32 * a + 8 * (r >> 2) + 4 * h + (r & 3);
                if (row < M) {
                    float* c = C + (size_t)row * ldc + col;
                    *c = beta == 0.f ? acc[a][b][r] : acc[a][b][r] + beta * *c;
                }
            }
        }
}

template <int BM, int BN, int BK, int WAVES_M, bool TA, bool TB, bool VA, bool VB>
int launch_cfg(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
               float beta, float* C, int ldc) {
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
    kern<<<tiles, NTHREADS, lds, stream()>>>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    return check_launch("dh_gemm_bf16");
}

template <bool TA, bool TB, bool VA, bool VB>
int launch_vec(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
               float beta, float* C, int ldc) {
    // The 256 x 256 tile needs enough tiles to cover the chip; otherwise use 128 x 128.
    const long long big_tiles = (long long)((M + 255) / 256) * ((N + 255) / 256);
    if (M >= 256 && N >= 256 && big_tiles >= num_cus())
        return launch_cfg<256, 256, 64, 2, TA, TB, VA, VB>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    return launch_cfg<128, 128, 64, 2, TA, TB, VA, VB>(M, N, K, A, lda, B, ldb, beta, C, ldc);
}

template <bool TA, bool TB>
int launch(int M, int N, int K, const uint16_t* A, int lda, const uint16_t* B, int ldb,
           float beta, float* C, int ldc) {
    const bool va = ((uintptr_t)A % 16 == 0) && (lda % 8 == 0);
    const bool vb = ((uintptr_t)B % 16 == 0) && (ldb % 8 == 0);
    if (va && vb) return launch_vec<TA, TB, true, true>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    if (va) return launch_vec<TA, TB, true, false>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    if (vb) return launch_vec<TA, TB, false, true>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    return launch_vec<TA, TB, false, false>(M, N, K, A, lda, B, ldb, beta, C, ldc);
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" int dh_gemm_bf16(int transA, int transB, int M, int N, int K, const uint16_t* A,
                            int lda, const uint16_t* B, int ldb, float beta, float* C, int ldc) {
    DH_TRY(ensure_init());
    if (M < 0 || N < 0 || K < 0) return set_error(DH_ERR_INVALID, "dh_gemm_bf16: negative shape");
    if (M == 0 || N == 0) return DH_OK;
    if (!C || (K > 0 && (!A || !B)))
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: null pointer");
    // A and B are not read when K == 0, so only C's leading dimension matters then.
    if (ldc < N || (K > 0 && (lda < (transA ? M : K) || ldb < (transB ? K : N))))
        return set_error(DH_ERR_INVALID, "dh_gemm_bf16: leading dimension too small");
    if (transA)
        return transB ? launch<true, true>(M, N, K, A, lda, B, ldb, beta, C, ldc)
                      : launch<true, false>(M, N, K, A, lda, B, ldb, beta, C, ldc);
    return transB ? launch<false, true>(M, N, K, A, lda, B, ldb, beta, C, ldc)
                  : launch<false, false>(M, N, K, A, lda, B, ldb, beta, C, ldc);
}
