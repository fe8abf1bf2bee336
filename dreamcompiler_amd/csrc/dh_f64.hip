// dh_f64.hip -- the fp64 half of the hot path: the products and attention the reference
// computes in double precision.
//
// The reference runs `@` below its dispatch threshold (M*N < gpu_dispatch_threshold()) in
// fp64 with dream_gemm_d (runtime/ops/elementwise.inc:1033-1040, 593-638), flash attention
// outside B*S*S >= 262144 && dk <= 128 with its fp64 online-softmax loop
// (runtime/nn/training.inc:307-308, 336, 366-399), and standard attention always in fp64
// (training.inc:178-263).  This file gives those results on the GPU in fp64.
//
// GEMM.  dream_gemm_d zeroes C and, per 256-deep k block (its KC), adds to every element the
// sum of that block's products, each block's sum being one fused multiply-add chain in k
// order started from zero (the 4x8 AVX2 micro-kernel, elementwise.inc:547-585).  Here the
// fp64 matrix cores run exactly those chains: v_mfma_f64_16x16x4f64 performs the four
// products of each output as sequential IEEE fused multiply-adds in k order (round to nearest
// even, as _mm256_fmadd_pd), so an accumulator started from zero and fed the k-steps in order
// is the chain; it is added to a running total at every 256-boundary of k.  With beta = 0 and
// alpha = 1 the result is therefore bit-identical to the reference's fp64 `@`.  Grids too
// small for the chip split K at those 256-boundaries and sum the block sums in k order in a
// second launch, which keeps the identity.
//
// Attention.  The standard form of training.inc:178-263 on fp64 GEMMs: scores = Q K^T
// (one batched NT product per chunk of slices), a row kernel applies the scale, the causal
// mask and the softmax (max, exp, sum, divide), O = P V; the backward
// (runtime/ops/autograd.inc:675-778) recomputes P, then dV += P^T dO, dP = dO V^T,
// dS = P (dP - rowsum(dP P)), dQ += scale dS K, dK += scale dS^T Q.  Score buffers come from
// the pool in chunks of slices (at most 256 MB per buffer).
#include "dh_common.hpp"

#include <math.h>
#include <cstdlib>

namespace dh {
namespace {

constexpr int F64_KT = 16;        // k per LDS stage
constexpr int F64_KC = 256;       // the reference's KC: chains restart every 256 k
constexpr int F64_THREADS = 256;  // four waves as 2 x 2, each WB x WB blocks of 16 x 16

typedef double f64x4 __attribute__((ext_vector_type(4)));

template <int WB>
struct F64Cfg {
    static constexpr int TILE = 32 * WB;                       // work-group tile side
    static constexpr int NLD = TILE * F64_KT / F64_THREADS;    // A (and B) values per thread
    // LDS copy of an operand tile in its global order, so the stores from global memory
    // are conflict-free as well as the MFMA operand reads (16 consecutive rows or columns
    // of one k, times 4 k, per wave):
    //   k-contiguous (A untransposed, B transposed): [row][k], row pitch KT + 1 doubles;
    //   row-contiguous (A transposed, B untransposed): [k][row], k pitch TILE + 16 doubles
    //   (128 bytes past a multiple of the 256-byte bank sweep).
    static constexpr int KP = F64_KT + 1, RP = TILE + 16;
    static constexpr int SZ_K = TILE * KP, SZ_R = F64_KT * RP;
};

// One TILE x TILE output tile over the k range [kbeg, kend): all of K, or (split mode,
// part != null) the single 256-deep block blockIdx.z, whose chain sum goes to the partial
// buffer.  Products run on v_mfma_f64_16x16x4f64, which performs its four products of an
// output as sequential IEEE fused multiply-adds in k order (a GPU probe over 7 M outputs --
// integers, N(0,1), exponents over 2^+-30, subnormals, infinities and NaNs, 64-step chains --
// found it bitwise equal to the fma chain), so each accumulator is exactly the reference's
// chain.  Operand layout: lane l holds A[l % 16][k0 + l / 16] and B[k0 + l / 16][l % 16];
// result register r holds D[l / 16 + 4 r][l % 16].  k past the range is zero in both
// operands, and fma(0, 0, c) = c for every chain value (a chain started at +0 never holds
// -0), so the padded k-steps of a last partial stage change nothing.  Stages of 16 k are
// double-buffered in LDS; the next stage's global loads are issued before the current
// stage's products.
template <int TA, int TB, int WB>
__global__ __launch_bounds__(F64_THREADS) void gemm_f64_kernel(
    int M, int N, int K, double alpha, const double* __restrict__ A, int lda, long long sA,
    const double* __restrict__ B, int ldb, long long sB, double beta, double* __restrict__ C,
    int ldc, long long sC, int tilesN, double* __restrict__ part) {
    using Cf = F64Cfg<WB>;
    constexpr int TILE = Cf::TILE, NLD = Cf::NLD, KP = Cf::KP, RP = Cf::RP;
    __shared__ double As[2][TA == 0 ? Cf::SZ_K : Cf::SZ_R];
    __shared__ double Bs[2][TB == 1 ? Cf::SZ_K : Cf::SZ_R];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int wr = 16 * WB * (wave & 1), wc = 16 * WB * (wave >> 1);   // wave's sub-tile
    const int tile = blockIdx.x;
    const int m0 = (tile / tilesN) * TILE, n0 = (tile % tilesN) * TILE;
    const long long b = blockIdx.y;
    int kbeg = 0, kend = K;
    if (part) {
        kbeg = blockIdx.z * F64_KC;
        kend = min(K, kbeg + F64_KC);
    }
    const int ns = (kend - kbeg + F64_KT - 1) / F64_KT;

    // Element (row, k) of an operand tile in LDS.
    auto a_at = [&](int buf, int row, int k) -> double& {
        return TA == 0 ? As[buf][row * KP + k] : As[buf][k * RP + row];
    };
    auto b_at = [&](int buf, int row, int k) -> double& {
        return TB == 1 ? Bs[buf][row * KP + k] : Bs[buf][k * RP + row];
    };
    // This thread's NLD (row, k) positions per operand, read along the contiguous index
    // (k-contiguous: 16 lanes per 128-byte row piece; row-contiguous: TILE lanes), with a
    // loop-invariant pointer to k = kbeg + the position's k and the row's validity.
    int arow[NLD], ak[NLD], brow[NLD], bk[NLD];
    const double* ap[NLD];
    const double* bp[NLD];
    bool aok[NLD], bok[NLD];
#pragma unroll
    for (int r = 0; r < NLD; ++r) {
        if (TA == 0) { ak[r] = t & 15; arow[r] = (t >> 4) + 16 * r; }
        else         { arow[r] = t % TILE; ak[r] = t / TILE + (F64_THREADS / TILE) * r; }
        if (TB == 1) { bk[r] = t & 15; brow[r] = (t >> 4) + 16 * r; }
        else         { brow[r] = t % TILE; bk[r] = t / TILE + (F64_THREADS / TILE) * r; }
        const int gm = m0 + arow[r], gn = n0 + brow[r];
        aok[r] = gm < M;
        bok[r] = gn < N;
        const long long ka = kbeg + ak[r], kb = kbeg + bk[r];
        ap[r] = A + b * sA + (aok[r] ? (TA == 0 ? (long long)gm * lda + ka : ka * lda + gm) : 0);
        bp[r] = B + b * sB + (bok[r] ? (TB == 1 ? (long long)gn * ldb + kb : kb * ldb + gn) : 0);
    }
    const long long astep = TA == 0 ? F64_KT : (long long)F64_KT * lda;   // pointer step per stage
    const long long bstep = TB == 1 ? F64_KT : (long long)F64_KT * ldb;
    double ra[NLD], rb[NLD];
    auto fetch = [&](int s) {           // stage s: k = kbeg + 16 s + position
        const int kleft = kend - kbeg - F64_KT * s;   // valid k in this stage (may exceed 16)
#pragma unroll
        for (int r = 0; r < NLD; ++r) {
            ra[r] = aok[r] && ak[r] < kleft ? ap[r][s * astep] : 0.0;
            rb[r] = bok[r] && bk[r] < kleft ? bp[r][s * bstep] : 0.0;
        }
    };
    auto stash = [&](int buf) {
#pragma unroll
        for (int r = 0; r < NLD; ++r) {
            a_at(buf, arow[r], ak[r]) = ra[r];
            b_at(buf, brow[r], bk[r]) = rb[r];
        }
    };

    f64x4 tot[WB][WB], acc[WB][WB];
#pragma unroll
    for (int i = 0; i < WB; ++i)
#pragma unroll
        for (int j = 0; j < WB; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) tot[i][j][r] = acc[i][j][r] = 0.0;
    auto step = [&](int buf, int k4) {
        const int kr = 4 * k4 + (lane >> 4), c = lane & 15;
        double a[WB], bb[WB];
#pragma unroll
        for (int i = 0; i < WB; ++i) a[i] = a_at(buf, wr + 16 * i + c, kr);
#pragma unroll
        for (int j = 0; j < WB; ++j) bb[j] = b_at(buf, wc + 16 * j + c, kr);
#pragma unroll
        for (int i = 0; i < WB; ++i)
#pragma unroll
            for (int j = 0; j < WB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f64_16x16x4f64(a[i], bb[j], acc[i][j], 0, 0, 0);
    };

    // Every stage runs its four k-steps (zeros past kend), so the loop has no branch around
    // the accumulators; a fetch past the last stage loads nothing and its stash lands in the
    // buffer no later stage reads.  Blocks of 256 k (kbeg is a multiple of 256): the chain
    // sum of each is added to tot in k order.
    fetch(0);
    stash(0);
    __syncthreads();
    for (int s = 0; s < ns;) {
        const int s_end = min(ns, s + F64_KC / F64_KT);
        for (; s < s_end; ++s) {
            const int buf = s & 1;
            fetch(s + 1);
#pragma unroll
            for (int k4 = 0; k4 < F64_KT / 4; ++k4) step(buf, k4);
            stash(buf ^ 1);   // the buffer stage s - 1 read, released below
            __syncthreads();
        }
#pragma unroll
        for (int i = 0; i < WB; ++i)
#pragma unroll
            for (int j = 0; j < WB; ++j)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    tot[i][j][r] = tot[i][j][r] + acc[i][j][r];
                    acc[i][j][r] = 0.0;
                }
    }
    // lane l, register r of block (i, j): row wr + 16 i + l / 16 + 4 r, column wc + 16 j + l % 16
    double* out = part ? part + ((long long)blockIdx.z * gridDim.y + b) * ((long long)M * N)
                       : C + b * sC;
    const long long ld = part ? N : ldc;
#pragma unroll
    for (int i = 0; i < WB; ++i)
#pragma unroll
        for (int j = 0; j < WB; ++j) {
            const int gn = n0 + wc + 16 * j + (lane & 15);
            if (gn >= N) continue;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int gm = m0 + wr + 16 * i + (lane >> 4) + 4 * r;
                if (gm >= M) continue;
                double* c = out + (long long)gm * ld + gn;
                if (part) {             // this block's chain sum, compact M x N per (block, member)
                    *c = tot[i][j][r];
                } else {
                    const double v = alpha == 1.0 ? tot[i][j][r] : alpha * tot[i][j][r];
                    *c = beta == 0.0 ? v : beta * *c + v;
                }
            }
        }
}

// Split-K finish: C = alpha * (((0 + s_0) + s_1) + ...) over the per-block chain sums in k
// order -- the reference's accumulation of its block sums into a zeroed C -- then beta.
__global__ __launch_bounds__(256) void gemm_f64_reduce(int M, int N, int nkb, int batch,
                                                       const double* __restrict__ part,
                                                       double alpha, double beta,
                                                       double* __restrict__ C, int ldc,
                                                       long long sC) {
    const long long mn = (long long)M * N, total = mn * batch;
    for (long long idx = (long long)blockIdx.x * 256 + threadIdx.x; idx < total;
         idx += (long long)gridDim.x * 256) {
        const long long b = idx / mn, rem = idx - b * mn;
        double tot = 0.0;
        for (int z = 0; z < nkb; ++z) tot = tot + part[((long long)z * batch + b) * mn + rem];
        double* c = C + b * sC + (rem / N) * (long long)ldc + rem % N;
        const double v = alpha == 1.0 ? tot : alpha * tot;
        *c = beta == 0.0 ? v : beta * *c + v;
    }
}

// Row softmax of one chunk of attention scores, in place: row r is query i = r mod S of its
// slice; x_j = s_j * scale over the row's visible keys (j <= i when causal), then
// p_j = exp(x_j - max x) / sum exp(x - max x), and exact zeros for masked keys
// (training.inc:193-201, 240-247).  One wave per row.
// P holds `rows` score rows of S keys: consecutive groups of R rows are query rows
// row0 .. row0 + R - 1 of a slice (R = S, row0 = 0 for whole slices).
__global__ __launch_bounds__(256) void attn_softmax_f64(double* __restrict__ P, int S,
                                                        long long rows, int R, int row0,
                                                        double scale, int causal) {
    // x = s * scale is rounded before the subtraction, as the reference stores it first.
#pragma clang fp contract(off)
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int i = row0 + (int)(r % R);
    const int n = causal ? i + 1 : S;
    double* row = P + r * (long long)S;
    double mx = -1e30;
    for (int j = lane; j < n; j += 64) mx = fmax(mx, row[j] * scale);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) mx = fmax(mx, __shfl_xor(mx, d));
    double sum = 0.0;
    for (int j = lane; j < n; j += 64) {
        const double e = exp(row[j] * scale - mx);
        row[j] = e;
        sum += e;
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) sum += __shfl_xor(sum, d);
    for (int j = lane; j < S; j += 64) row[j] = j < n ? row[j] / sum : 0.0;
}

// dS = P o (dP - rowsum(dP o P)) in place of dP, zeros on masked keys (the softmax JVP of
// autograd.inc:711-714, 758-761).
__global__ __launch_bounds__(256) void attn_softmax_bwd_f64(const double* __restrict__ P,
                                                            double* __restrict__ dP, int S,
                                                            long long rows, int R, int row0,
                                                            int causal) {
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int i = row0 + (int)(r % R);
    const int n = causal ? i + 1 : S;
    const double* p = P + r * (long long)S;
    double* g = dP + r * (long long)S;
    double rd = 0.0;
    for (int j = lane; j < n; j += 64) rd = __builtin_fma(g[j], p[j], rd);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) rd += __shfl_xor(rd, d);
    for (int j = lane; j < S; j += 64) g[j] = j < n ? p[j] * (g[j] - rd) : 0.0;
}

template <int WB>
void launch_f64(int transA, int transB, dim3 grid, int M, int N, int K, double alpha,
                const double* A, int lda, long long sA, const double* B, int ldb, long long sB,
                double beta, double* C, int ldc, long long sC, int tilesN, double* part) {
#define DH_F64_LAUNCH(TA, TB)                                                                  \
    gemm_f64_kernel<TA, TB, WB><<<grid, F64_THREADS, 0, stream()>>>(                           \
        M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc, sC, tilesN, part)
    if (!transA && !transB) DH_F64_LAUNCH(0, 0);
    else if (!transA) DH_F64_LAUNCH(0, 1);
    else if (!transB) DH_F64_LAUNCH(1, 0);
    else DH_F64_LAUNCH(1, 1);
#undef DH_F64_LAUNCH
}

int gemm_f64_launch(int transA, int transB, int M, int N, int K, double alpha, const double* A,
                    int lda, long long sA, const double* B, int ldb, long long sB, double beta,
                    double* C, int ldc, long long sC, int batch) {
    // 64 x 64 tiles (2 x 2 blocks per wave) when they fill the chip twice over, else 32 x 32.
    // Grids still too small split K at the reference's 256-deep block boundaries (one
    // work-group per block, each block's chain sum stored, then summed in k order by
    // gemm_f64_reduce), which leaves every result bit-identical.
    const long long fill = 2LL * num_cus();
    const int wb = ((M + 63) / 64) * (long long)((N + 63) / 64) * batch >= fill ? 2 : 1;
    const long long tilesM = (M + 32 * wb - 1) / (32 * wb), tilesN = (N + 32 * wb - 1) / (32 * wb);
    const long long nkb = ((long long)K + F64_KC - 1) / F64_KC;
    const size_t pbytes = (size_t)nkb * batch * M * N * sizeof(double);
    double* part = nullptr;
    if (nkb > 1 && nkb <= 65535 && tilesM * tilesN * batch < fill && pbytes <= ((size_t)512 << 20))
        part = static_cast<double*>(dh_malloc(pbytes));   // none: the unsplit grid
    const dim3 grid((unsigned)(tilesM * tilesN), (unsigned)batch, part ? (unsigned)nkb : 1u);
    if (wb == 2)
        launch_f64<2>(transA, transB, grid, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc,
                      sC, (int)tilesN, part);
    else
        launch_f64<1>(transA, transB, grid, M, N, K, alpha, A, lda, sA, B, ldb, sB, beta, C, ldc,
                      sC, (int)tilesN, part);
    if (part) {
        const long long total = (long long)M * N * batch;
        long long blocks = (total + 255) / 256;
        if (blocks > 8LL * num_cus()) blocks = 8LL * num_cus();
        gemm_f64_reduce<<<(unsigned)blocks, 256, 0, stream()>>>(M, N, (int)nkb, batch, part,
                                                                 alpha, beta, C, ldc, sC);
        dh_free(part);   // pooled: stream order keeps the buffer alive for the queued work
    }
    return check_launch("dh_gemm_f64");
}

int check_gemm_f64(const char* op, int transA, int transB, int M, int N, int K, const void* A,
                   int lda, long long sA, const void* B, int ldb, long long sB, const void* C,
                   int ldc, long long sC, int batch) {
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return set_error(DH_ERR_INVALID, "%s: negative shape (M=%d N=%d K=%d batch=%d)", op, M, N,
                         K, batch);
    if (M == 0 || N == 0 || batch == 0) return DH_OK;
    if (!C || (K > 0 && (!A || !B))) return set_error(DH_ERR_INVALID, "%s: null pointer", op);
    if ((K > 0 && (lda < (transA ? M : K) || ldb < (transB ? K : N))) || ldc < N)
        return set_error(DH_ERR_INVALID, "%s: leading dimension too small (lda=%d ldb=%d ldc=%d)",
                         op, lda, ldb, ldc);
    if (sA < 0 || sB < 0 || sC < 0)
        return set_error(DH_ERR_INVALID, "%s: negative batch stride", op);
    if (batch > 1 && sC < (long long)(M - 1) * ldc + N)
        return set_error(DH_ERR_INVALID, "%s: batch members of C overlap (strideC=%lld)", op, sC);
    if (batch > 65535)
        return set_error(DH_ERR_UNSUPPORTED, "%s: batch %d above 65535", op, batch);
    const long long tiles = (long long)((M + 31) / 32) * ((N + 31) / 32);
    if (tiles > 0x7fffffffLL)
        return set_error(DH_ERR_UNSUPPORTED, "%s: %lld output tiles", op, tiles);
    return DH_OK;
}

// Bytes one fp64 score buffer may take: 256 MB (DH_ATTN_F64_SCORE_BYTES overrides it, for
// tests of the row-block path at small S).
size_t attn_budget() {
    const char* e = std::getenv("DH_ATTN_F64_SCORE_BYTES");
    const long long v = e && *e ? std::atoll(e) : 0;
    return v > 0 ? (size_t)v : ((size_t)256 << 20);
}

// Work per pass over the scores: `chunk` whole slices of S x S scores when one slice fits the
// budget, else (chunk = 1) blocks of `rows` query rows of one slice, rows x S scores each.
struct AttnPass {
    int chunk, rows;
};
AttnPass attn_pass(int BH, int S) {
    const size_t budget = attn_budget();
    const size_t per = (size_t)S * S * sizeof(double);
    if (per <= budget) {
        size_t c = budget / (per ? per : 1);
        if (c > (size_t)BH) c = BH;
        if (c > 65535) c = 65535;
        return {(int)c, S};
    }
    size_t r = budget / ((size_t)S * sizeof(double));
    if (r < 1) r = 1;
    return {1, (int)r};
}

int check_attn_f64(const char* op, int BH, int S, int D) {
    if (BH < 0 || S < 0 || D < 0)
        return set_error(DH_ERR_INVALID, "%s: negative shape (BH=%d S=%d D=%d)", op, BH, S, D);
    if ((long long)S * D > 0x7fffffffLL)
        return set_error(DH_ERR_UNSUPPORTED, "%s: S*D = %lld above 2^31", op, (long long)S * D);
    if (S > 46340)
        return set_error(DH_ERR_UNSUPPORTED, "%s: S = %d (S*S above 2^31)", op, S);
    return DH_OK;
}

void launch_softmax(double* P, int S, long long rows, int R, int row0, double scale,
                    int causal) {
    attn_softmax_f64<<<(unsigned)((rows + 3) / 4), 256, 0, stream()>>>(P, S, rows, R, row0,
                                                                      scale, causal);
}

void launch_softmax_bwd(const double* P, double* G, int S, long long rows, int R, int row0,
                        int causal) {
    attn_softmax_bwd_f64<<<(unsigned)((rows + 3) / 4), 256, 0, stream()>>>(P, G, S, rows, R,
                                                                          row0, causal);
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" {

int dh_gemm_f64_ex(int transA, int transB, int M, int N, int K, double alpha, const double* d_A,
                   int lda, long long strideA, const double* d_B, int ldb, long long strideB,
                   double beta, double* d_C, int ldc, long long strideC, int batch) {
    DH_TRY(ensure_init());
    DH_TRY(check_gemm_f64("dh_gemm_f64", transA, transB, M, N, K, d_A, lda, strideA, d_B, ldb,
                          strideB, d_C, ldc, strideC, batch));
    if (M == 0 || N == 0 || batch == 0) return DH_OK;
    return gemm_f64_launch(transA ? 1 : 0, transB ? 1 : 0, M, N, K, alpha, d_A, lda, strideA, d_B,
                           ldb, strideB, beta, d_C, ldc, strideC, batch);
}

int dh_gemm_f64(int transA, int transB, int M, int N, int K, const double* d_A, int lda,
                const double* d_B, int ldb, double beta, double* d_C, int ldc) {
    return dh_gemm_f64_ex(transA, transB, M, N, K, 1.0, d_A, lda, 0, d_B, ldb, 0, beta, d_C, ldc,
                          0, 1);
}

int dh_attention_f64_fwd(int BH, int S, int D, double scale, int causal, const double* d_Q,
                         const double* d_K, const double* d_V, double* d_O) {
    DH_TRY(ensure_init());
    DH_TRY(check_attn_f64("dh_attention_f64_fwd", BH, S, D));
    if (BH == 0 || S == 0 || D == 0) return DH_OK;
    if (!d_Q || !d_K || !d_V || !d_O)
        return set_error(DH_ERR_INVALID, "dh_attention_f64_fwd: null pointer");
    if (!(scale > 0.0) || !isfinite(scale))
        return set_error(DH_ERR_INVALID, "dh_attention_f64_fwd: scale must be positive and finite");
    const AttnPass ps = attn_pass(BH, S);
    const long long SD = (long long)S * D;
    const long long RS = (long long)ps.rows * S;   // scores per slice and pass
    double* P = static_cast<double*>(dh_malloc((size_t)ps.chunk * RS * sizeof(double)));
    if (!P)
        return set_error(DH_ERR_OOM, "dh_attention_f64_fwd: %d score blocks of %d x %d",
                         ps.chunk, ps.rows, S);
    int st = DH_OK;
    for (int b0 = 0; b0 < BH && st == DH_OK; b0 += ps.chunk) {
        const int nb = BH - b0 < ps.chunk ? BH - b0 : ps.chunk;
        for (int r0 = 0; r0 < S && st == DH_OK; r0 += ps.rows) {
            const int nr = S - r0 < ps.rows ? S - r0 : ps.rows;
            const long long off = (long long)b0 * SD, qoff = off + (long long)r0 * D;
            // scores of query rows r0 .. r0 + nr - 1 = Q K^T
            st = gemm_f64_launch(0, 1, nr, S, D, 1.0, d_Q + qoff, D, SD, d_K + off, D, SD, 0.0,
                                 P, S, RS, nb);
            if (st != DH_OK) break;
            launch_softmax(P, S, (long long)nb * nr, nr, r0, scale, causal);
            st = check_launch("dh_attention_f64_fwd");
            if (st != DH_OK) break;
            // O = P V
            st = gemm_f64_launch(0, 0, nr, D, S, 1.0, P, S, RS, d_V + off, D, SD, 0.0,
                                 d_O + qoff, D, SD, nb);
        }
    }
    dh_free(P);   // pooled: stream order keeps the buffer alive for the queued work
    return st;
}

int dh_attention_f64_bwd(int BH, int S, int D, double scale, int causal, const double* d_Q,
                         const double* d_K, const double* d_V, const double* d_dO, double* d_dQ,
                         double* d_dK, double* d_dV, int accumulate) {
    DH_TRY(ensure_init());
    DH_TRY(check_attn_f64("dh_attention_f64_bwd", BH, S, D));
    if (BH == 0 || S == 0 || D == 0) return DH_OK;
    if (!d_Q || !d_K || !d_V || !d_dO || !d_dQ || !d_dK || !d_dV)
        return set_error(DH_ERR_INVALID, "dh_attention_f64_bwd: null pointer");
    if (!(scale > 0.0) || !isfinite(scale))
        return set_error(DH_ERR_INVALID, "dh_attention_f64_bwd: scale must be positive and finite");
    const long long SD = (long long)S * D;
    const size_t gbytes = (size_t)BH * SD * sizeof(double);
    // Shared gradient buffers (one tensor passed as several of Q, K, V) receive the sum of
    // their gradients: every product below adds into its output, after one clearing pass.
    if (!accumulate) {
        double* outs[3] = {d_dQ, d_dK, d_dV};
        for (int x = 0; x < 3; ++x) {
            bool seen = false;
            for (int y = 0; y < x; ++y) seen |= outs[y] == outs[x];
            if (!seen) DH_TRY(dh_memset(outs[x], 0, gbytes));
        }
    }
    const AttnPass ps = attn_pass(BH, S);
    const long long RS = (long long)ps.rows * S;   // scores per slice and pass
    double* P = static_cast<double*>(dh_malloc((size_t)ps.chunk * RS * sizeof(double)));
    double* G = static_cast<double*>(dh_malloc((size_t)ps.chunk * RS * sizeof(double)));
    if (!P || !G) {
        if (P) dh_free(P);
        if (G) dh_free(G);
        return set_error(DH_ERR_OOM, "dh_attention_f64_bwd: %d score blocks of %d x %d",
                         ps.chunk, ps.rows, S);
    }
    int st = DH_OK;
    for (int b0 = 0; b0 < BH && st == DH_OK; b0 += ps.chunk) {
        const int nb = BH - b0 < ps.chunk ? BH - b0 : ps.chunk;
        const long long off = (long long)b0 * SD;
        const double *Q = d_Q + off, *K = d_K + off, *V = d_V + off, *dO = d_dO + off;
        // Query rows r0 .. r0 + nr - 1 per pass (whole slices when they fit the budget).
        for (int r0 = 0; r0 < S && st == DH_OK; r0 += ps.rows) {
            const int nr = S - r0 < ps.rows ? S - r0 : ps.rows;
            const long long ro = (long long)r0 * D;
            // P recomputed from Q, K exactly as the forward computes it
            st = gemm_f64_launch(0, 1, nr, S, D, 1.0, Q + ro, D, SD, K, D, SD, 0.0, P, S, RS, nb);
            if (st != DH_OK) break;
            launch_softmax(P, S, (long long)nb * nr, nr, r0, scale, causal);
            if ((st = check_launch("dh_attention_f64_bwd")) != DH_OK) break;
            // dV += P^T dO
            st = gemm_f64_launch(1, 0, S, D, nr, 1.0, P, S, RS, dO + ro, D, SD, 1.0, d_dV + off,
                                 D, SD, nb);
            if (st != DH_OK) break;
            // dP = dO V^T, then dS in its place
            st = gemm_f64_launch(0, 1, nr, S, D, 1.0, dO + ro, D, SD, V, D, SD, 0.0, G, S, RS, nb);
            if (st != DH_OK) break;
            launch_softmax_bwd(P, G, S, (long long)nb * nr, nr, r0, causal);
            if ((st = check_launch("dh_attention_f64_bwd")) != DH_OK) break;
            // dQ += scale dS K ;  dK += scale dS^T Q
            st = gemm_f64_launch(0, 0, nr, D, S, scale, G, S, RS, K, D, SD, 1.0,
                                 d_dQ + off + ro, D, SD, nb);
            if (st != DH_OK) break;
            st = gemm_f64_launch(1, 0, S, D, nr, scale, G, S, RS, Q + ro, D, SD, 1.0,
                                 d_dK + off, D, SD, nb);
        }
    }
    dh_free(P);
    dh_free(G);
    return st;
}

}  // extern "C"
