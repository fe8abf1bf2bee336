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
// order started from zero (the 4x8 AVX2 micro-kernel, elementwise.inc:547-585).  Here each
// lane owns a 4x4 block of outputs and runs exactly those chains with v_fma_f64 (IEEE fma,
// round to nearest even, as _mm256_fmadd_pd), adding the chain to its running total at every
// 256-boundary of k.  With beta = 0 and alpha = 1 the result is therefore bit-identical to the
// reference's fp64 `@`.  FP64 FMA on the VALU runs at the chip's full fp64 rate (the same
// 78.6 TFLOP/s as the fp64 matrix cores), so the kernel stays on plain FMA.
//
// Attention.  The standard form of training.inc:178-263 on fp64 GEMMs: scores = Q K^T
// (one batched NT product per chunk of slices), a row kernel applies the scale, the causal
// mask and the softmax (max, exp, sum, divide), O = P V; the backward
// (runtime/ops/autograd.inc:675-778) recomputes P, then dV += P^T dO, dP = dO V^T,
// dS = P (dP - rowsum(dP P)), dQ += scale dS K, dK += scale dS^T Q.  Score buffers come from
// the pool in chunks of slices (at most 256 MB per buffer).
#include "dh_common.hpp"

#include <math.h>

namespace dh {
namespace {

constexpr int F64_TILE = 32;     // 32 x 32 outputs per work-group
constexpr int F64_KT = 16;       // k-step staged through LDS
constexpr int F64_KC = 256;      // the reference's KC: chains restart every 256 k
constexpr int F64_THREADS = 64;  // one wave; lane (tx, ty) in 8 x 8, outputs ty + 8i, tx + 8j

template <int TA, int TB>
__global__ __launch_bounds__(F64_THREADS) void gemm_f64_kernel(
    int M, int N, int K, double alpha, const double* __restrict__ A, int lda, long long sA,
    const double* __restrict__ B, int ldb, long long sB, double beta, double* __restrict__ C,
    int ldc, long long sC, int tilesN) {
    __shared__ double As[F64_KT][F64_TILE + 1];
    __shared__ double Bs[F64_KT][F64_TILE + 1];
    const int t = threadIdx.x, tx = t & 7, ty = t >> 3;
    const int tile = blockIdx.x;
    const int m0 = (tile / tilesN) * F64_TILE, n0 = (tile % tilesN) * F64_TILE;
    const long long b = blockIdx.y;
    A += b * sA;
    B += b * sB;
    C += b * sC;

    double tot[4][4], acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) tot[i][j] = acc[i][j] = 0.0;

    for (int k0 = 0; k0 < K; k0 += F64_KT) {
        const int kt = K - k0 < F64_KT ? K - k0 : F64_KT;
        // A tile (32 rows m x 16 k) -> As[k][m]; reads run along the contiguous index.
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            int m, k;
            if (TA == 0) { k = t & 15; m = (t >> 4) + 4 * r; }
            else         { m = t & 31; k = (t >> 5) + 2 * r; }
            const int gm = m0 + m, gk = k0 + k;
            double v = 0.0;
            if (gm < M && gk < K) v = TA == 0 ? A[(long long)gm * lda + gk] : A[(long long)gk * lda + gm];
            As[k][m] = v;
        }
        // B tile (16 k x 32 cols n) -> Bs[k][n]
#pragma unroll
        for (int r = 0; r < 8; ++r) {
            int n, k;
            if (TB == 0) { n = t & 31; k = (t >> 5) + 2 * r; }
            else         { k = t & 15; n = (t >> 4) + 4 * r; }
            const int gn = n0 + n, gk = k0 + k;
            double v = 0.0;
            if (gn < N && gk < K) v = TB == 0 ? B[(long long)gk * ldb + gn] : B[(long long)gn * ldb + gk];
            Bs[k][n] = v;
        }
        __syncthreads();
        // Exactly kt products per chain: no padded products enter a sum.
        for (int kk = 0; kk < kt; ++kk) {
            double a[4], bb[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) a[i] = As[kk][ty + 8 * i];
#pragma unroll
            for (int j = 0; j < 4; ++j) bb[j] = Bs[kk][tx + 8 * j];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fma(a[i], bb[j], acc[i][j]);
        }
        __syncthreads();
        if ((k0 + F64_KT) % F64_KC == 0 || k0 + F64_KT >= K) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    tot[i][j] = tot[i][j] + acc[i][j];
                    acc[i][j] = 0.0;
                }
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int gm = m0 + ty + 8 * i;
        if (gm >= M) continue;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int gn = n0 + tx + 8 * j;
            if (gn >= N) continue;
            double* c = C + (long long)gm * ldc + gn;
            const double v = alpha == 1.0 ? tot[i][j] : alpha * tot[i][j];
            *c = beta == 0.0 ? v : beta * *c + v;
        }
    }
}

// Row softmax of one chunk of attention scores, in place: row r is query i = r mod S of its
// slice; x_j = s_j * scale over the row's visible keys (j <= i when causal), then
// p_j = exp(x_j - max x) / sum exp(x - max x), and exact zeros for masked keys
// (training.inc:193-201, 240-247).  One wave per row.
__global__ __launch_bounds__(256) void attn_softmax_f64(double* __restrict__ P, int S,
                                                        long long rows, double scale,
                                                        int causal) {
    // x = s * scale is rounded before the subtraction, as the reference stores it first.
#pragma clang fp contract(off)
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int i = (int)(r % S);
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
                                                            long long rows, int causal) {
    const long long r = (long long)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const int i = (int)(r % S);
    const int n = causal ? i + 1 : S;
    const double* p = P + r * (long long)S;
    double* g = dP + r * (long long)S;
    double rd = 0.0;
    for (int j = lane; j < n; j += 64) rd = __builtin_fma(g[j], p[j], rd);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) rd += __shfl_xor(rd, d);
    for (int j = lane; j < S; j += 64) g[j] = j < n ? p[j] * (g[j] - rd) : 0.0;
}

int gemm_f64_launch(int transA, int transB, int M, int N, int K, double alpha, const double* A,
                    int lda, long long sA, const double* B, int ldb, long long sB, double beta,
                    double* C, int ldc, long long sC, int batch) {
    const long long tilesM = (M + F64_TILE - 1) / F64_TILE, tilesN = (N + F64_TILE - 1) / F64_TILE;
    const dim3 grid((unsigned)(tilesM * tilesN), (unsigned)batch);
#define DH_F64_LAUNCH(TA, TB)                                                                  \
    gemm_f64_kernel<TA, TB><<<grid, F64_THREADS, 0, stream()>>>(M, N, K, alpha, A, lda, sA, B, \
                                                                ldb, sB, beta, C, ldc, sC,     \
                                                                (int)tilesN)
    if (!transA && !transB) DH_F64_LAUNCH(0, 0);
    else if (!transA) DH_F64_LAUNCH(0, 1);
    else if (!transB) DH_F64_LAUNCH(1, 0);
    else DH_F64_LAUNCH(1, 1);
#undef DH_F64_LAUNCH
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
    const long long tiles = (long long)((M + F64_TILE - 1) / F64_TILE) * ((N + F64_TILE - 1) / F64_TILE);
    if (tiles > 0x7fffffffLL)
        return set_error(DH_ERR_UNSUPPORTED, "%s: %lld output tiles", op, tiles);
    return DH_OK;
}

// Slices per chunk so that one S x S fp64 score buffer stays within 256 MB.
int attn_chunk(int BH, int S) {
    const size_t per = (size_t)S * S * sizeof(double);
    size_t c = ((size_t)256 << 20) / (per ? per : 1);
    if (c < 1) c = 1;
    if (c > (size_t)BH) c = BH;
    if (c > 65535) c = 65535;
    return (int)c;
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

void launch_softmax(double* P, int S, long long rows, double scale, int causal) {
    attn_softmax_f64<<<(unsigned)((rows + 3) / 4), 256, 0, stream()>>>(P, S, rows, scale, causal);
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
    const int chunk = attn_chunk(BH, S);
    const long long SD = (long long)S * D, SS = (long long)S * S;
    double* P = static_cast<double*>(dh_malloc((size_t)chunk * SS * sizeof(double)));
    if (!P) return set_error(DH_ERR_OOM, "dh_attention_f64_fwd: %d score blocks of %d x %d", chunk, S, S);
    int st = DH_OK;
    for (int b0 = 0; b0 < BH && st == DH_OK; b0 += chunk) {
        const int nb = BH - b0 < chunk ? BH - b0 : chunk;
        const long long off = (long long)b0 * SD;
        // scores = Q K^T
        st = gemm_f64_launch(0, 1, S, S, D, 1.0, d_Q + off, D, SD, d_K + off, D, SD, 0.0, P, S, SS, nb);
        if (st != DH_OK) break;
        launch_softmax(P, S, (long long)nb * S, scale, causal);
        st = check_launch("dh_attention_f64_fwd");
        if (st != DH_OK) break;
        // O = P V
        st = gemm_f64_launch(0, 0, S, D, S, 1.0, P, S, SS, d_V + off, D, SD, 0.0, d_O + off, D, SD, nb);
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
    const long long SD = (long long)S * D, SS = (long long)S * S;
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
    const int chunk = attn_chunk(BH, S);
    double* P = static_cast<double*>(dh_malloc((size_t)chunk * SS * sizeof(double)));
    double* G = static_cast<double*>(dh_malloc((size_t)chunk * SS * sizeof(double)));
    if (!P || !G) {
        if (P) dh_free(P);
        if (G) dh_free(G);
        return set_error(DH_ERR_OOM, "dh_attention_f64_bwd: %d score blocks of %d x %d", chunk, S, S);
    }
    int st = DH_OK;
    for (int b0 = 0; b0 < BH && st == DH_OK; b0 += chunk) {
        const int nb = BH - b0 < chunk ? BH - b0 : chunk;
        const long long off = (long long)b0 * SD;
        const double *Q = d_Q + off, *K = d_K + off, *V = d_V + off, *dO = d_dO + off;
        // P recomputed from Q, K exactly as the forward computes it
        st = gemm_f64_launch(0, 1, S, S, D, 1.0, Q, D, SD, K, D, SD, 0.0, P, S, SS, nb);
        if (st != DH_OK) break;
        launch_softmax(P, S, (long long)nb * S, scale, causal);
        if ((st = check_launch("dh_attention_f64_bwd")) != DH_OK) break;
        // dV += P^T dO
        st = gemm_f64_launch(1, 0, S, D, S, 1.0, P, S, SS, dO, D, SD, 1.0, d_dV + off, D, SD, nb);
        if (st != DH_OK) break;
        // dP = dO V^T, then dS in its place
        st = gemm_f64_launch(0, 1, S, S, D, 1.0, dO, D, SD, V, D, SD, 0.0, G, S, SS, nb);
        if (st != DH_OK) break;
        attn_softmax_bwd_f64<<<(unsigned)(((long long)nb * S + 3) / 4), 256, 0, stream()>>>(
            P, G, S, (long long)nb * S, causal);
        if ((st = check_launch("dh_attention_f64_bwd")) != DH_OK) break;
        // dQ += scale dS K ;  dK += scale dS^T Q
        st = gemm_f64_launch(0, 0, S, D, S, scale, G, S, SS, K, D, SD, 1.0, d_dQ + off, D, SD, nb);
        if (st != DH_OK) break;
        st = gemm_f64_launch(1, 0, S, D, S, scale, G, S, SS, Q, D, SD, 1.0, d_dK + off, D, SD, nb);
    }
    dh_free(P);
    dh_free(G);
    return st;
}

}  // extern "C"
