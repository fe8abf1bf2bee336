// dream_oracle.cpp -- CPU restatement of the Dream reference hot path.
//
// TEST INFRASTRUCTURE ONLY: used by tests/, __graft_entry__.smoke() and bench.py's
// cpu_baseline leg as the checker / CPU comparison.  The product never links it.
//
// Written from the reference's documented behaviour; each function names the
// reference lines it restates.  Loop orders, blocking constants and the points
// where "+=" accumulates are kept, because they fix the exact fp64 values the
// reference produces (tests compare against its golden vectors at <=1e-12).
#include "dream_oracle.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <random>
#include <vector>

namespace {

// One process-wide generator, like get_rng() (elementwise.inc:30-33).
std::mt19937& rng() {
    static std::mt19937 g(42u);
    return g;
}

}  // namespace

// The exported functions take C linkage from their declarations in dream_oracle.h.

// ---------------------------------------------------------------------------
// RNG: set_seed / randn (elementwise.inc:35-54), uniform draws of the selftests
// (elementwise.inc:815, 897), kaiming_init (builtins.inc:511-519).
// ---------------------------------------------------------------------------
void orc_set_seed(unsigned int seed) { rng().seed(seed); }

void orc_randn(double* out, long long n) {
    std::normal_distribution<double> nd(0.0, 1.0);
    for (long long i = 0; i < n; ++i) out[i] = nd(rng());
}

void orc_uniform(double* out, long long n, double lo, double hi) {
    std::uniform_real_distribution<double> ud(lo, hi);
    for (long long i = 0; i < n; ++i) out[i] = ud(rng());
}

void orc_uniform_f32(float* out, long long n, float lo, float hi) {
    std::uniform_real_distribution<float> ud(lo, hi);
    for (long long i = 0; i < n; ++i) out[i] = ud(rng());
}

void orc_kaiming(double* out, int rows, int cols) {
    // std = sqrt(2 / cols): the reference treats the column count as fan_in.
    std::normal_distribution<double> nd(0.0, std::sqrt(2.0 / cols));
    long long n = (long long)rows * cols;
    for (long long i = 0; i < n; ++i) out[i] = nd(rng());
}

// ---------------------------------------------------------------------------
// GEMM
// ---------------------------------------------------------------------------
void orc_gemm_ref_d(const double* A, const double* B, double* C, int M, int K, int N) {
    // elementwise.inc:878-886: one fp64 dot product per output, k ascending.
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) s += A[(size_t)i * K + k] * B[(size_t)k * N + j];
            C[(size_t)i * N + j] = s;
        }
}

namespace {

// Blocked GEMM skeleton shared by the fp64 and fp32 restatements.
// Blocking (elementwise.inc:518-519, 645): NC columns of B per outer panel,
// KC-deep slices of K (B packed once per slice), MC-row blocks of A handed to
// OpenMP threads, and an MR x NR register tile whose per-k update is one fused
// multiply-add per element.  Each C element therefore receives, per KC slice, an
// FMA chain over that slice started from zero, added onto C once the slice ends.
template <typename T, int MR, int NR>
struct Blocked {
    static constexpr int KC = 256, MC = 128, NC_CAP = 4096;

    // [panel][k][MR], zero padded (elementwise.inc:522-532).
    static void pack_a(const T* A, int lda, int mc, int kc, T* dst) {
        for (int ir = 0; ir < mc; ir += MR) {
            const int mr = std::min(MR, mc - ir);
            for (int k = 0; k < kc; ++k, dst += MR)
                for (int i = 0; i < MR; ++i)
                    dst[i] = i < mr ? A[(size_t)(ir + i) * lda + k] : T(0);
        }
    }
    // [panel][k][NR], zero padded (elementwise.inc:535-545).
    static void pack_b(const T* B, int ldb, int kc, int nc, T* dst) {
        for (int jr = 0; jr < nc; jr += NR) {
            const int nr = std::min(NR, nc - jr);
            for (int k = 0; k < kc; ++k, dst += NR)
                for (int j = 0; j < NR; ++j)
                    dst[j] = j < nr ? B[(size_t)k * ldb + jr + j] : T(0);
        }
    }
    // Register tile: acc = fma chain over kc, then C(mr x nr) += acc
    // (ukern_4x8 / ukern_edge, elementwise.inc:548-588; fgemm ukern 667-684).
    static void tile(int kc, const T* Ap, const T* Bp, T* C, int ldc, int mr, int nr) {
        T acc[MR][NR];
        for (int i = 0; i < MR; ++i)
            for (int j = 0; j < NR; ++j) acc[i][j] = T(0);
        for (int k = 0; k < kc; ++k) {
            const T* b = Bp + (size_t)k * NR;
            const T* a = Ap + (size_t)k * MR;
            for (int i = 0; i < MR; ++i)
                for (int j = 0; j < NR; ++j) acc[i][j] = std::fma(a[i], b[j], acc[i][j]);
        }
        for (int i = 0; i < mr; ++i)
            for (int j = 0; j < nr; ++j) C[(size_t)i * ldc + j] += acc[i][j];
    }

    static void run(const T* A, const T* B, T* C, int M, int K, int N) {
        // C is zeroed first (elementwise.inc:595, 691).
        std::fill(C, C + (size_t)M * N, T(0));
        if (M <= 0 || K <= 0 || N <= 0) return;
        const int ncb = std::min(N, NC_CAP);
        std::vector<T> bpack((size_t)KC * ((ncb + NR - 1) / NR) * NR);
        const bool par = (size_t)M * K * N >= 262144;   // elementwise.inc:606, 702
        for (int jc = 0; jc < N; jc += ncb) {
            const int nc = std::min(ncb, N - jc);
            for (int pc = 0; pc < K; pc += KC) {
                const int kc = std::min(KC, K - pc);
                pack_b(B + (size_t)pc * N + jc, N, kc, nc, bpack.data());
#pragma omp parallel for schedule(dynamic) if (par)
                for (int ic = 0; ic < M; ic += MC) {
                    const int mc = std::min(MC, M - ic);
                    std::vector<T> apack((size_t)KC * ((MC + MR - 1) / MR) * MR);
                    pack_a(A + (size_t)ic * K + pc, K, mc, kc, apack.data());
                    for (int jr = 0; jr < nc; jr += NR) {
                        const int nr = std::min(NR, nc - jr);
                        const T* bp = bpack.data() + (size_t)(jr / NR) * kc * NR;
                        for (int ir = 0; ir < mc; ir += MR) {
                            const int mr = std::min(MR, mc - ir);
                            const T* ap = apack.data() + (size_t)(ir / MR) * kc * MR;
                            tile(kc, ap, bp, C + (size_t)(ic + ir) * N + jc + jr, N, mr, nr);
                        }
                    }
                }
            }
        }
    }
};

}  // namespace

void orc_gemm_d(const double* A, const double* B, double* C, int M, int K, int N) {
    Blocked<double, 4, 8>::run(A, B, C, M, K, N);
}

void orc_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N) {
    Blocked<float, 8, 16>::run(A, B, C, M, K, N);
}

void orc_gemm_general_d(int transA, int transB, int M, int N, int K,
                        const double* A, int lda, const double* B, int ldb,
                        double beta, double* C, int ldc) {
#pragma omp parallel for schedule(static) if ((size_t)M * N * K >= 2097152)
    for (int i = 0; i < M; ++i)
        for (int j = 0; j < N; ++j) {
            double s = 0.0;
            for (int k = 0; k < K; ++k) {
                const double a = transA ? A[(size_t)k * lda + i] : A[(size_t)i * lda + k];
                const double b = transB ? B[(size_t)j * ldb + k] : B[(size_t)k * ldb + j];
                s += a * b;
            }
            double* c = C + (size_t)i * ldc + j;
            *c = (beta == 0.0 ? 0.0 : beta * *c) + s;
        }
}

void orc_matmul_bwd(const double* A, const double* B, const double* dY,
                    double* dA, double* dB, int M, int K, int N) {
    const bool par = (long long)M * K * N >= 2097152;   // autograd.inc:104, 117
    // dA[i,k] += sum_j dY[i,j] * B[k,j]: dot over j, added once per (i,k) (autograd.inc:104-113).
#pragma omp parallel for schedule(static) if (par)
    for (int i = 0; i < M; ++i)
        for (int k = 0; k < K; ++k) {
            double acc = 0.0;
            for (int j = 0; j < N; ++j) acc += dY[(size_t)i * N + j] * B[(size_t)k * N + j];
            dA[(size_t)i * K + k] += acc;
        }
    // dB[k,j] += A[i,k] * dY[i,j], i ascending, axpy into the dB row (autograd.inc:116-124).
#pragma omp parallel for schedule(static) if (par)
    for (int k = 0; k < K; ++k) {
        double* row = dB + (size_t)k * N;
        for (int i = 0; i < M; ++i) {
            const double a = A[(size_t)i * K + k];
            const double* dy = dY + (size_t)i * N;
            for (int j = 0; j < N; ++j) row[j] += a * dy[j];
        }
    }
}

// ---------------------------------------------------------------------------
// Attention forward
// ---------------------------------------------------------------------------
namespace {

inline double dot(const double* a, const double* b, int n) {
    double s = 0.0;
    for (int k = 0; k < n; ++k) s += a[k] * b[k];
    return s;
}

// Materialized SDPA for one slice: scores, row softmax (max-subtracted, divided by
// the sum), then P @ V.  causal keeps j <= i only, masked entries stay 0
// (training.inc:196-217 and 235-260).
void sdpa_slice(const double* Q, const double* K, const double* V, double* O,
                int S, int dk, bool causal, std::vector<double>& P) {
    const double scale = 1.0 / std::sqrt((double)dk);
    P.assign((size_t)S * S, 0.0);
    for (int i = 0; i < S; ++i) {
        const int jn = causal ? i + 1 : S;
        double* p = &P[(size_t)i * S];
        double mx = -1e30;
        for (int j = 0; j < jn; ++j) {
            p[j] = dot(Q + (size_t)i * dk, K + (size_t)j * dk, dk) * scale;
            if (p[j] > mx) mx = p[j];
        }
        double sum = 0.0;
        for (int j = 0; j < jn; ++j) { p[j] = std::exp(p[j] - mx); sum += p[j]; }
        for (int j = 0; j < jn; ++j) p[j] /= sum;
    }
    // O = P V; each O[i][k] sums over j in ascending order (the loop over k is innermost
    // only so that rows are read contiguously).
    for (int i = 0; i < S; ++i) {
        const int jn = causal ? i + 1 : S;
        double* o = O + (size_t)i * dk;
        for (int k = 0; k < dk; ++k) o[k] = 0.0;
        for (int j = 0; j < jn; ++j) {
            const double p = P[(size_t)i * S + j];
            const double* v = V + (size_t)j * dk;
            for (int k = 0; k < dk; ++k) o[k] += p * v[k];
        }
    }
}

}  // namespace

// Slices are independent; they run in parallel, each with the single-slice loop order.
void orc_attention(const double* Q, const double* K, const double* V, double* O,
                   int B, int S, int dk) {
#pragma omp parallel
    {
        std::vector<double> P;
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b) {
            const size_t off = (size_t)b * S * dk;
            sdpa_slice(Q + off, K + off, V + off, O + off, S, dk, false, P);
        }
    }
}

void orc_attention_causal(const double* Q, const double* K, const double* V, double* O,
                          int B, int S, int dk) {
#pragma omp parallel
    {
        std::vector<double> P;
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b) {
            const size_t off = (size_t)b * S * dk;
            sdpa_slice(Q + off, K + off, V + off, O + off, S, dk, true, P);
        }
    }
}

void orc_flash_fwd(const double* Q, const double* K, const double* V, double* O,
                   int B, int S, int dk, int Bc) {
    // training.inc:288-289, 366-399: causal online softmax over key blocks of Bc.
    if (Bc < 1) Bc = 64;
    const double scale = 1.0 / std::sqrt((double)dk);
    std::vector<double> sc((size_t)Bc), acc((size_t)dk);
    for (int b = 0; b < B; ++b) {
        const size_t off = (size_t)b * S * dk;
        const double *Qb = Q + off, *Kb = K + off, *Vb = V + off;
        double* Ob = O + off;
        for (int i = 0; i < S; ++i) {
            double m = -1e30, l = 0.0;
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int jb = 0; jb <= i; jb += Bc) {
                const int je = std::min(i, jb + Bc - 1);
                double mb = -1e30;
                for (int j = jb; j <= je; ++j) {
                    sc[j - jb] = dot(Qb + (size_t)i * dk, Kb + (size_t)j * dk, dk) * scale;
                    mb = std::max(mb, sc[j - jb]);
                }
                const double mn = std::max(m, mb);
                const double corr = std::exp(m - mn);   // rescale the running state
                l *= corr;
                for (int k = 0; k < dk; ++k) acc[k] *= corr;
                for (int j = jb; j <= je; ++j) {
                    const double p = std::exp(sc[j - jb] - mn);
                    l += p;
                    for (int k = 0; k < dk; ++k) acc[k] += p * Vb[(size_t)j * dk + k];
                }
                m = mn;
            }
            const double inv = l > 0.0 ? 1.0 / l : 0.0;
            for (int k = 0; k < dk; ++k) Ob[(size_t)i * dk + k] = acc[k] * inv;
        }
    }
}

// ---------------------------------------------------------------------------
// Attention backward ("+=" into dQ, dK, dV)
// ---------------------------------------------------------------------------
void orc_attention_bwd(const double* Q, const double* K, const double* V, const double* dO,
                       double* dQ, double* dK, double* dV, int B, int S, int dk, int causal) {
    // autograd.inc:675-778.  P recomputed; dV = P^T dO; dP = dO V^T;
    // dS = P o (dP - rowsum(dP o P)); dQ += dS K * scale; dK += dS^T Q * scale.
    // Every output element sums its terms in ascending order of the contracted index; the
    // innermost loop runs over the head dim so that rows are read contiguously.  Slices are
    // independent and run in parallel.
    const double scale = 1.0 / std::sqrt((double)dk);
#pragma omp parallel
    {
        std::vector<double> P, dP((size_t)S * S), dS((size_t)S * S), O((size_t)S * dk),
            acc((size_t)S * dk);
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b) {
            const size_t off = (size_t)b * S * dk;
            const double *Qb = Q + off, *Kb = K + off, *Vb = V + off, *dOb = dO + off;
            double *dQb = dQ + off, *dKb = dK + off, *dVb = dV + off;
            sdpa_slice(Qb, Kb, Vb, O.data(), S, dk, causal != 0, P);
            // dV[j] += sum_i P[i][j] dO[i]   (i ascending)
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int i = 0; i < S; ++i)
                for (int j = 0; j < (causal ? i + 1 : S); ++j) {
                    const double p = P[(size_t)i * S + j];
                    const double* g = dOb + (size_t)i * dk;
                    double* a = &acc[(size_t)j * dk];
                    for (int k = 0; k < dk; ++k) a[k] += p * g[k];
                }
            for (size_t x = 0; x < (size_t)S * dk; ++x) dVb[x] += acc[x];
            std::fill(dP.begin(), dP.end(), 0.0);
            for (int i = 0; i < S; ++i) {
                const int jn = causal ? i + 1 : S;
                for (int j = 0; j < jn; ++j)
                    dP[(size_t)i * S + j] = dot(dOb + (size_t)i * dk, Vb + (size_t)j * dk, dk);
            }
            std::fill(dS.begin(), dS.end(), 0.0);
            for (int i = 0; i < S; ++i) {
                const int jn = causal ? i + 1 : S;
                double rd = 0.0;
                for (int j = 0; j < jn; ++j) rd += dP[(size_t)i * S + j] * P[(size_t)i * S + j];
                for (int j = 0; j < jn; ++j)
                    dS[(size_t)i * S + j] = P[(size_t)i * S + j] * (dP[(size_t)i * S + j] - rd);
            }
            // dQ[i] += scale * sum_j dS[i][j] K[j]   (j ascending)
            for (int i = 0; i < S; ++i) {
                const int jn = causal ? i + 1 : S;
                double* a = &acc[(size_t)i * dk];
                for (int k = 0; k < dk; ++k) a[k] = 0.0;
                for (int j = 0; j < jn; ++j) {
                    const double d = dS[(size_t)i * S + j];
                    const double* kr = Kb + (size_t)j * dk;
                    for (int k = 0; k < dk; ++k) a[k] += d * kr[k];
                }
                for (int k = 0; k < dk; ++k) dQb[(size_t)i * dk + k] += a[k] * scale;
            }
            // dK[j] += scale * sum_i dS[i][j] Q[i]   (i ascending)
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int i = 0; i < S; ++i)
                for (int j = 0; j < (causal ? i + 1 : S); ++j) {
                    const double d = dS[(size_t)i * S + j];
                    const double* q = Qb + (size_t)i * dk;
                    double* a = &acc[(size_t)j * dk];
                    for (int k = 0; k < dk; ++k) a[k] += d * q[k];
                }
            for (size_t x = 0; x < (size_t)S * dk; ++x) dKb[x] += acc[x] * scale;
        }
    }
}

void orc_attention_rows(const double* Q, const double* K, const double* V, const double* dO,
                        const int* rows, int nrows, double* O_rows, double* dQ_rows, int B,
                        int S, int dk, int causal) {
    // One query row i at a time, the operations of sdpa_slice (training.inc:196-217,
    // 235-260) and of orc_attention_bwd's dQ (autograd.inc:675-778) restricted to that row:
    // scores, max-subtracted exp, divide by the sum, O_i = sum_j P_ij V_j; dP_ij = dO_i . V_j,
    // rd = sum_j dP_ij P_ij, dS_ij = P_ij (dP_ij - rd), dQ_i = scale * sum_j dS_ij K_j.
    const double scale = 1.0 / std::sqrt((double)dk);
#pragma omp parallel
    {
        std::vector<double> p((size_t)S), ds((size_t)S), acc((size_t)dk);
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b) {
            const size_t off = (size_t)b * S * dk;
            const double *Qb = Q + off, *Kb = K + off, *Vb = V + off, *dOb = dO + off;
            for (int r = 0; r < nrows; ++r) {
                const int i = rows[(size_t)b * nrows + r];
                const int jn = causal ? i + 1 : S;
                double mx = -1e30;
                for (int j = 0; j < jn; ++j) {
                    p[j] = dot(Qb + (size_t)i * dk, Kb + (size_t)j * dk, dk) * scale;
                    if (p[j] > mx) mx = p[j];
                }
                double sum = 0.0;
                for (int j = 0; j < jn; ++j) { p[j] = std::exp(p[j] - mx); sum += p[j]; }
                for (int j = 0; j < jn; ++j) p[j] /= sum;
                double* o = O_rows + ((size_t)b * nrows + r) * dk;
                for (int k = 0; k < dk; ++k) o[k] = 0.0;
                for (int j = 0; j < jn; ++j)
                    for (int k = 0; k < dk; ++k) o[k] += p[j] * Vb[(size_t)j * dk + k];
                const double* g = dOb + (size_t)i * dk;
                double rd = 0.0;
                for (int j = 0; j < jn; ++j) {
                    ds[j] = dot(g, Vb + (size_t)j * dk, dk);
                    rd += ds[j] * p[j];
                }
                for (int j = 0; j < jn; ++j) ds[j] = p[j] * (ds[j] - rd);
                for (int k = 0; k < dk; ++k) acc[k] = 0.0;
                for (int j = 0; j < jn; ++j)
                    for (int k = 0; k < dk; ++k) acc[k] += ds[j] * Kb[(size_t)j * dk + k];
                double* q = dQ_rows + ((size_t)b * nrows + r) * dk;
                for (int k = 0; k < dk; ++k) q[k] = acc[k] * scale;
            }
        }
    }
}

namespace {

// Pass 1 of the flash backward (autograd.inc:799-812): per-row running max m and
// normalizer l over key blocks of Bc, same recurrence as the forward.
void row_stats(const double* Qb, const double* Kb, int S, int dk, int Bc, bool causal,
               double scale, std::vector<double>& sc, double* m_out, double* l_out) {
    for (int i = 0; i < S; ++i) {
        double m = -1e30, l = 0.0;
        const int last = causal ? i : S - 1;
        for (int jb = 0; jb <= last; jb += Bc) {
            const int je = std::min(last, jb + Bc - 1);
            double mb = -1e30;
            for (int j = jb; j <= je; ++j) {
                sc[j - jb] = dot(Qb + (size_t)i * dk, Kb + (size_t)j * dk, dk) * scale;
                mb = std::max(mb, sc[j - jb]);
            }
            const double mn = std::max(m, mb);
            l *= std::exp(m - mn);
            for (int j = jb; j <= je; ++j) l += std::exp(sc[j - jb] - mn);
            m = mn;
        }
        m_out[i] = m;
        l_out[i] = l;
    }
}

}  // namespace

void orc_flash_bwd(const double* Q, const double* K, const double* V, const double* dO,
                   double* dQ, double* dK, double* dV, int B, int S, int dk) {
    // autograd.inc:779-840.
    const double scale = 1.0 / std::sqrt((double)dk);
    const int Bc = 64;
    std::vector<double> sc(Bc), acc(dk), lrow(S), mrow(S), Drow(S);
    for (int b = 0; b < B; ++b) {
        const size_t off = (size_t)b * S * dk;
        const double *Qb = Q + off, *Kb = K + off, *Vb = V + off, *dOb = dO + off;
        double *dQb = dQ + off, *dKb = dK + off, *dVb = dV + off;
        row_stats(Qb, Kb, S, dk, Bc, true, scale, sc, mrow.data(), lrow.data());
        // pass 2 (813-820): D_i = dO_i . O_i with O_i recomputed from (m, l).
        for (int i = 0; i < S; ++i) {
            std::fill(acc.begin(), acc.end(), 0.0);
            for (int j = 0; j <= i; ++j) {
                const double s = dot(Qb + (size_t)i * dk, Kb + (size_t)j * dk, dk);
                const double p = std::exp(s * scale - mrow[i]) / lrow[i];
                for (int k = 0; k < dk; ++k) acc[k] += p * Vb[(size_t)j * dk + k];
            }
            Drow[i] = dot(dOb + (size_t)i * dk, acc.data(), dk);
        }
        // pass 3 (821-838): recompute a_ij, dS_ij = a_ij (dA_ij - D_i), scatter.
        for (int i = 0; i < S; ++i) {
            for (int j = 0; j <= i; ++j) {
                const double s = dot(Qb + (size_t)i * dk, Kb + (size_t)j * dk, dk);
                const double a = std::exp(s * scale - mrow[i]) / lrow[i];
                const double dA = dot(dOb + (size_t)i * dk, Vb + (size_t)j * dk, dk);
                const double ds = a * (dA - Drow[i]);
                for (int k = 0; k < dk; ++k) {
                    dVb[(size_t)j * dk + k] += a * dOb[(size_t)i * dk + k];
                    dQb[(size_t)i * dk + k] += ds * Kb[(size_t)j * dk + k] * scale;
                    dKb[(size_t)j * dk + k] += ds * Qb[(size_t)i * dk + k] * scale;
                }
            }
        }
    }
}

void orc_flash_lse(const double* Q, const double* K, double* lse, int B, int S, int dk,
                   int causal) {
    const double scale = 1.0 / std::sqrt((double)dk);
#pragma omp parallel
    {
        std::vector<double> sc(64), m(S), l(S);
#pragma omp for schedule(dynamic, 1)
        for (int b = 0; b < B; ++b) {
            const size_t off = (size_t)b * S * dk;
            row_stats(Q + off, K + off, S, dk, 64, causal != 0, scale, sc, m.data(), l.data());
            for (int i = 0; i < S; ++i) lse[(size_t)b * S + i] = m[i] + std::log(l[i]);
        }
    }
}

// ---------------------------------------------------------------------------
// Row reductions
// ---------------------------------------------------------------------------
void orc_softmax_rows(const double* X, double* Y, int R, int C) {
    // elementwise.inc:346-356: max, exp(x - max) with running sum, divide.
    for (int r = 0; r < R; ++r) {
        const double* x = X + (size_t)r * C;
        double* y = Y + (size_t)r * C;
        double mx = x[0];
        for (int j = 1; j < C; ++j) mx = std::max(mx, x[j]);
        double s = 0.0;
        for (int j = 0; j < C; ++j) { y[j] = std::exp(x[j] - mx); s += y[j]; }
        for (int j = 0; j < C; ++j) y[j] /= s;
    }
}

void orc_log_softmax_rows(const double* X, double* Y, int R, int C) {
    // elementwise.inc:1557-1567: x - (max + log(sum exp(x - max))).
    for (int r = 0; r < R; ++r) {
        const double* x = X + (size_t)r * C;
        double* y = Y + (size_t)r * C;
        double mx = x[0];
        for (int j = 1; j < C; ++j) mx = std::max(mx, x[j]);
        double s = 0.0;
        for (int j = 0; j < C; ++j) s += std::exp(x[j] - mx);
        const double lse = mx + std::log(s);
        for (int j = 0; j < C; ++j) y[j] = x[j] - lse;
    }
}

void orc_softmax_bwd(const double* Y, const double* G, double* GX, int R, int C) {
    // autograd.inc:396-409: per row dot = sum_j g_j y_j, then gx_j += y_j (g_j - dot).
    for (int r = 0; r < R; ++r) {
        const double* y = Y + (size_t)r * C;
        const double* g = G + (size_t)r * C;
        double* gx = GX + (size_t)r * C;
        double dot = 0.0;
        for (int j = 0; j < C; ++j) dot += g[j] * y[j];
        for (int j = 0; j < C; ++j) gx[j] += y[j] * (g[j] - dot);
    }
}

void orc_log_softmax_bwd(const double* X, const double* G, double* GX, int N, int C) {
    // autograd.inc:212-233: softmax recomputed from x (max, exp, normalise), then
    // dx_j += dy_j - sm_j * sum_k dy_k.
    std::vector<double> sm(C > 0 ? C : 1);
    for (int n = 0; n < N; ++n) {
        const double* x = X + (size_t)n * C;
        const double* g = G + (size_t)n * C;
        double* gx = GX + (size_t)n * C;
        double mx = x[0];
        for (int j = 1; j < C; ++j) if (x[j] > mx) mx = x[j];
        double s = 0.0;
        for (int j = 0; j < C; ++j) { sm[j] = std::exp(x[j] - mx); s += sm[j]; }
        for (int j = 0; j < C; ++j) sm[j] /= s;
        double gs = 0.0;
        for (int j = 0; j < C; ++j) gs += g[j];
        for (int j = 0; j < C; ++j) gx[j] += g[j] - sm[j] * gs;
    }
}

void orc_layer_norm(const double* X, double* Y, int R, int C) {
    // builtins.inc:167-188: per row mean, biased variance, y = (x - mu) / sqrt(var + 1e-5).
    for (int r = 0; r < R; ++r) {
        const double* x = X + (size_t)r * C;
        double* y = Y + (size_t)r * C;
        double mu = 0.0;
        for (int j = 0; j < C; ++j) mu += x[j];
        mu /= C;
        double var = 0.0;
        for (int j = 0; j < C; ++j) { const double d = x[j] - mu; var += d * d; }
        var /= C;
        const double inv_std = 1.0 / std::sqrt(var + 1e-5);
        for (int j = 0; j < C; ++j) y[j] = (x[j] - mu) * inv_std;
    }
}

void orc_layer_norm_bwd(const double* X, const double* Y, const double* DY, double* GX, int R,
                        int C) {
    // autograd.inc:453-471: inv_std recomputed from x; per row
    // gx_j += inv_std / C * (C dy_j - sum dy - y_j sum(dy y)).
    for (int r = 0; r < R; ++r) {
        const double* x = X + (size_t)r * C;
        const double* y = Y + (size_t)r * C;
        const double* dy = DY + (size_t)r * C;
        double* gx = GX + (size_t)r * C;
        double mu = 0.0;
        for (int j = 0; j < C; ++j) mu += x[j];
        mu /= C;
        double var = 0.0;
        for (int j = 0; j < C; ++j) { const double d = x[j] - mu; var += d * d; }
        var /= C;
        const double inv_std = 1.0 / std::sqrt(var + 1e-5);
        double sdy = 0.0, sdyy = 0.0;
        for (int j = 0; j < C; ++j) { sdy += dy[j]; sdyy += dy[j] * y[j]; }
        for (int j = 0; j < C; ++j) gx[j] += inv_std / C * (C * dy[j] - sdy - y[j] * sdyy);
    }
}

// ---------------------------------------------------------------------------
// Linear layers and batched matmul
// ---------------------------------------------------------------------------
void orc_linear(const double* X, const double* W, const double* b, double* Y, int N, int in_dim,
                int out_dim, int relu) {
    // elementwise.inc:1432-1510: Y = bias (broadcast), then Y[i,:] += X[i,k] * W^T[k,:] in
    // (i, k, j) order over an explicit transpose of W; linear_relu clamps Y < 0 to 0.
    std::vector<double> Wt((size_t)in_dim * out_dim);
    for (int j = 0; j < out_dim; ++j)
        for (int k = 0; k < in_dim; ++k) Wt[(size_t)k * out_dim + j] = W[(size_t)j * in_dim + k];
    for (int i = 0; i < N; ++i) {
        double* y = Y + (size_t)i * out_dim;
        for (int j = 0; j < out_dim; ++j) y[j] = b[j];
        for (int k = 0; k < in_dim; ++k) {
            const double xik = X[(size_t)i * in_dim + k];
            const double* wt = &Wt[(size_t)k * out_dim];
            for (int j = 0; j < out_dim; ++j) y[j] += xik * wt[j];
        }
    }
    if (relu)
        for (size_t i = 0; i < (size_t)N * out_dim; ++i) if (Y[i] < 0) Y[i] = 0;
}

void orc_linear_bwd(const double* X, const double* W, const double* Y, double* dY, double* dX,
                    double* dW, double* db, int N, int in_dim, int out_dim, int relu) {
    // autograd.inc:156-205.  linear_relu first zeroes dY where Y <= 0 -- in place, as the
    // reference does to the node's own gradient -- then db += column sums of dY,
    // dX += dY W (i, j, k order), dW += dY^T X (j, i, k order).
    if (relu)
        for (size_t i = 0; i < (size_t)N * out_dim; ++i) if (Y[i] <= 0) dY[i] = 0;
    for (int j = 0; j < out_dim; ++j) {
        double s = 0.0;
        for (int i = 0; i < N; ++i) s += dY[(size_t)i * out_dim + j];
        db[j] += s;
    }
    for (int i = 0; i < N; ++i)
        for (int j = 0; j < out_dim; ++j) {
            const double dy = dY[(size_t)i * out_dim + j];
            const double* w = W + (size_t)j * in_dim;
            double* dx = dX + (size_t)i * in_dim;
            for (int k = 0; k < in_dim; ++k) dx[k] += dy * w[k];
        }
    for (int j = 0; j < out_dim; ++j) {
        double* dw = dW + (size_t)j * in_dim;
        for (int i = 0; i < N; ++i) {
            const double dy = dY[(size_t)i * out_dim + j];
            const double* x = X + (size_t)i * in_dim;
            for (int k = 0; k < in_dim; ++k) dw[k] += dy * x[k];
        }
    }
}

void orc_bmm(const double* A, const double* B, double* C, int Bt, int M, int K, int N) {
    // elementwise.inc:1218-1252: per batch, C[r][c] = sum_k A[r][k] B[k][c] (dot order k).
    for (int bi = 0; bi < Bt; ++bi) {
        const double* a = A + (size_t)bi * M * K;
        const double* b = B + (size_t)bi * K * N;
        double* c = C + (size_t)bi * M * N;
        for (int r = 0; r < M; ++r)
            for (int cc = 0; cc < N; ++cc) {
                double s = 0.0;
                for (int k = 0; k < K; ++k) s += a[(size_t)r * K + k] * b[(size_t)k * N + cc];
                c[(size_t)r * N + cc] = s;
            }
    }
}

void orc_bmm_bwd(const double* A, const double* B, const double* G, double* gA, double* gB,
                 int Bt, int M, int K, int N) {
    // autograd.inc:549-574: gA += G B^T, gB += A^T G per batch, each entry one dot product.
    for (int bi = 0; bi < Bt; ++bi) {
        const double* go = G + (size_t)bi * M * N;
        const double* a = A + (size_t)bi * M * K;
        const double* b = B + (size_t)bi * K * N;
        double* ga = gA + (size_t)bi * M * K;
        double* gb = gB + (size_t)bi * K * N;
        for (int r = 0; r < M; ++r)
            for (int k = 0; k < K; ++k) {
                double s = 0.0;
                for (int c = 0; c < N; ++c) s += go[(size_t)r * N + c] * b[(size_t)k * N + c];
                ga[(size_t)r * K + k] += s;
            }
        for (int k = 0; k < K; ++k)
            for (int c = 0; c < N; ++c) {
                double s = 0.0;
                for (int r = 0; r < M; ++r) s += a[(size_t)r * K + k] * go[(size_t)r * N + c];
                gb[(size_t)k * N + c] += s;
            }
    }
}

// ---------------------------------------------------------------------------
// Convolution (im2col + GEMM)
// ---------------------------------------------------------------------------
namespace {
// im2col with zero padding and stride (im2col.inc:2-13 for pad 0 / stride 1; conv.inc:149-171
// for the padded, strided form): col[r][oh*OW + ow], r = (ci*KH + kh)*KW + kw.
void im2col_ps(const double* inp, double* col, int Cin, int H, int W, int KH, int KW, int OH,
               int OW, int pad, int stride) {
    int r = 0;
    for (int ci = 0; ci < Cin; ++ci)
        for (int kh = 0; kh < KH; ++kh)
            for (int kw = 0; kw < KW; ++kw, ++r)
                for (int oh = 0; oh < OH; ++oh)
                    for (int ow = 0; ow < OW; ++ow) {
                        const int h = oh * stride + kh - pad, w = ow * stride + kw - pad;
                        col[(size_t)r * OH * OW + oh * OW + ow] =
                            (h >= 0 && h < H && w >= 0 && w < W) ? inp[(size_t)ci * H * W + h * W + w] : 0.0;
                    }
}
}  // namespace

void orc_conv2d(const double* X, const double* Kn, const double* bias, double* Y, int N, int Cin,
                int H, int W, int Cout, int KH, int KW, int pad, int stride) {
    // conv.inc:12-55 (pad 0, stride 1) and 119-178: per image im2col, then kernel (Cout x
    // Cin*KH*KW) @ col with the blocked dgemm (cpu_gemm = dream_gemm_d), then + bias[co].
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const int K = Cin * KH * KW, P = OH * OW;
    std::vector<double> col((size_t)K * P);
    for (int n = 0; n < N; ++n) {
        im2col_ps(X + (size_t)n * Cin * H * W, col.data(), Cin, H, W, KH, KW, OH, OW, pad, stride);
        double* y = Y + (size_t)n * Cout * P;
        orc_gemm_d(Kn, col.data(), y, Cout, K, P);
        if (bias)
            for (int co = 0; co < Cout; ++co)
                for (int j = 0; j < P; ++j) y[(size_t)co * P + j] += bias[co];
    }
}

void orc_conv2d_bwd(const double* X, const double* Kn, const double* G, double* gX, double* gK,
                    int N, int Cin, int H, int W, int Cout, int KH, int KW, int pad, int stride) {
    // autograd.inc:507-535 (pad 0, stride 1): per image gK += G col^T (dot products over the
    // output positions), dcol = K^T G, gX += col2im(dcol).  No bias gradient (the reference's
    // conv node has none).  With pad > 0 or stride > 1 the same algebra over the padded,
    // strided im2col -- the exact gradient, which the reference's node (reusing the unpadded
    // shapes) does not compute.
    const int OH = (H + 2 * pad - KH) / stride + 1, OW = (W + 2 * pad - KW) / stride + 1;
    const int K = Cin * KH * KW, P = OH * OW;
    std::vector<double> col((size_t)K * P), dcol((size_t)K * P);
    for (int n = 0; n < N; ++n) {
        im2col_ps(X + (size_t)n * Cin * H * W, col.data(), Cin, H, W, KH, KW, OH, OW, pad, stride);
        const double* go = G + (size_t)n * Cout * P;
        for (int co = 0; co < Cout; ++co)
            for (int cr = 0; cr < K; ++cr) {
                double s = 0.0;
                for (int j = 0; j < P; ++j) s += go[(size_t)co * P + j] * col[(size_t)cr * P + j];
                gK[(size_t)co * K + cr] += s;
            }
        for (int cr = 0; cr < K; ++cr)
            for (int j = 0; j < P; ++j) {
                double s = 0.0;
                for (int co = 0; co < Cout; ++co) s += Kn[(size_t)co * K + cr] * go[(size_t)co * P + j];
                dcol[(size_t)cr * P + j] = s;
            }
        double* gx = gX + (size_t)n * Cin * H * W;
        int r = 0;   // col2im (im2col.inc:14-25), scattering into the unpadded input
        for (int ci = 0; ci < Cin; ++ci)
            for (int kh = 0; kh < KH; ++kh)
                for (int kw = 0; kw < KW; ++kw, ++r)
                    for (int oh = 0; oh < OH; ++oh)
                        for (int ow = 0; ow < OW; ++ow) {
                            const int h = oh * stride + kh - pad, w = ow * stride + kw - pad;
                            if (h >= 0 && h < H && w >= 0 && w < W)
                                gx[(size_t)ci * H * W + h * W + w] += dcol[(size_t)r * P + oh * OW + ow];
                        }
    }
}

// ---------------------------------------------------------------------------
// Elementwise ops (runCPUBinary / runCPUUnary, runtime/backend/gpu.inc:443-598) and their
// backward branches (autograd.inc:58-90, 284-288, 342-378, 491-506)
// ---------------------------------------------------------------------------
namespace {

double bin_op(int op, double a, double b) {
    switch (op) {   // BinopCode order, gpu.inc:455-460; expressions of gpu.inc:511-527
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        case 3: return a / b;
        case 4: return std::fmod(a, b);
        case 5: return a > b ? 1.0 : 0.0;
        case 6: return a < b ? 1.0 : 0.0;
        case 7: return a >= b ? 1.0 : 0.0;
        case 8: return a <= b ? 1.0 : 0.0;
        case 9: return std::fabs(a - b) < 1e-6 ? 1.0 : 0.0;
        case 10: return std::fabs(a - b) >= 1e-6 ? 1.0 : 0.0;
        case 11: return (a > 0 && b > 0) ? 1.0 : 0.0;
        case 12: return (a > 0 || b > 0) ? 1.0 : 0.0;
        case 13: return std::atan2(a, b);
        case 14: return std::pow(a, b);
        case 15: return a < b ? a : b;
        default: return a > b ? a : b;
    }
}

// bcastStrides (gpu.inc:443-449): contiguous strides of the operand's own dims, 0 where the
// dim is 1.
void bcast_strides(const int* d, long long* s) {
    s[0] = d[0] > 1 ? (long long)d[1] * d[2] * d[3] : 0;
    s[1] = d[1] > 1 ? (long long)d[2] * d[3] : 0;
    s[2] = d[2] > 1 ? d[3] : 0;
    s[3] = d[3] > 1 ? 1 : 0;
}

}  // namespace

void orc_binary(int op, const double* A, const int* a_dims, const double* B, const int* b_dims,
                double* C, const int* c_dims) {
    const long long sz = (long long)c_dims[0] * c_dims[1] * c_dims[2] * c_dims[3];
    const long long asz = (long long)a_dims[0] * a_dims[1] * a_dims[2] * a_dims[3];
    const long long bsz = (long long)b_dims[0] * b_dims[1] * b_dims[2] * b_dims[3];
    if (asz == sz && bsz == sz) {   // same-shape path, gpu.inc:504-528
        for (long long i = 0; i < sz; ++i) C[i] = bin_op(op, A[i], B[i]);
        return;
    }
    long long as[4], bs[4];   // broadcasting path, gpu.inc:530-564
    bcast_strides(a_dims, as);
    bcast_strides(b_dims, bs);
    const long long cd3 = c_dims[3], cd2 = c_dims[2], cd1 = c_dims[1];
    for (long long i = 0; i < sz; ++i) {
        const long long i3 = i % cd3, i2 = (i / cd3) % cd2, i1 = (i / (cd3 * cd2)) % cd1,
                        i0 = i / (cd3 * cd2 * cd1);
        const long long ai = i0 * as[0] + i1 * as[1] + i2 * as[2] + i3 * as[3];
        const long long bi = i0 * bs[0] + i1 * bs[1] + i2 * bs[2] + i3 * bs[3];
        C[i] = bin_op(op, A[ai], B[bi]);
    }
}

void orc_unary(int op, const double* A, double* C, long long n, double lo, double hi) {
    for (long long i = 0; i < n; ++i) {
        const double a = A[i];
        double c;
        switch (op) {   // UnopCode order, gpu.inc:571-577; expressions of gpu.inc:614-629
            case 0: c = a > 0.0 ? a : 0.0; break;
            case 1: c = std::exp(a); break;
            case 2: c = std::log(a); break;
            case 3: c = std::sqrt(a); break;
            case 4: c = std::fabs(a); break;
            case 5: c = 1.0 / (1.0 + std::exp(-a)); break;
            case 6: c = std::tanh(a); break;
            case 7: c = a == 0.0 ? 1.0 : 0.0; break;
            case 8: c = std::sin(a); break;
            case 9: c = std::cos(a); break;
            case 10: c = std::tan(a); break;
            case 11: c = std::atan(a); break;
            case 12: c = std::floor(a); break;
            case 13: c = std::ceil(a); break;
            case 14: c = std::round(a); break;
            default: c = std::fmax(lo, std::fmin(hi, a)); break;   // clip's expression
        }
        C[i] = c;
    }
}

void orc_binary_bwd(int op, const double* A, long long a_size, const double* B, long long b_size,
                    const double* Y, const double* G, long long n, double* gA, double* gB) {
    // Operands are indexed j % size (autograd.inc:58-90), not by the forward's strides.
    switch (op) {
        case 0:   // add
            for (long long j = 0; j < n; ++j) {
                gA[j % a_size] += G[j];
                gB[j % b_size] += G[j];
            }
            break;
        case 1:   // sub
            for (long long j = 0; j < n; ++j) {
                gA[j % a_size] += G[j];
                gB[j % b_size] -= G[j];
            }
            break;
        case 2:   // mul
            for (long long j = 0; j < n; ++j) {
                gA[j % a_size] += G[j] * B[j % b_size];
                gB[j % b_size] += G[j] * A[j % a_size];
            }
            break;
        case 3:   // div
            for (long long j = 0; j < n; ++j) {
                const double r = B[j % b_size], g = G[j];
                gA[j % a_size] += g / r;
                gB[j % b_size] -= g * A[j % a_size] / (r * r);
            }
            break;
        case 14:   // pow: over the base's elements, autograd.inc:491-506
            for (long long j = 0; j < a_size; ++j) {
                const double x = A[j], e = B[j % b_size], y = Y[j % n], g = G[j % n];
                if (x != 0.0) gA[j] += g * e * y / x;
                if (x > 0.0) gB[j % b_size] += g * y * std::log(x);
            }
            break;
        case 15:   // minimum / maximum: all to the chosen side, ties to lhs (autograd.inc:68-79)
        case 16:
            for (long long j = 0; j < n; ++j) {
                const double av = A[j % a_size], bv = B[j % b_size];
                const bool lhs = op == 16 ? av >= bv : av <= bv;
                if (lhs) gA[j % a_size] += G[j];
                else gB[j % b_size] += G[j];
            }
            break;
        default:   // the comparisons, mod, and / or, atan2: no backward branch
            break;
    }
}

void orc_unary_bwd(int op, const double* X, const double* Y, const double* G, double* GX,
                   long long n) {
    for (long long j = 0; j < n; ++j) {
        const double x = X[j], y = Y[j], g = G[j];
        switch (op) {
            case 0: GX[j] += (x > 0 ? 1.0 : 0.0) * g; break;   // relu, autograd.inc:284-288
            case 1: GX[j] += y * g; break;                      // exp, 342-344
            case 2: GX[j] += g / x; break;                      // log
            case 3: GX[j] += g / (2.0 * y); break;              // sqrt
            case 4: GX[j] += (x >= 0 ? 1.0 : -1.0) * g; break;  // abs
            case 5: GX[j] += y * (1 - y) * g; break;            // sigmoid
            case 6: GX[j] += (1 - y * y) * g; break;            // tanh
            case 8: GX[j] += std::cos(x) * g; break;            // sin, 363-365
            case 9: GX[j] += -std::sin(x) * g; break;           // cos
            case 10: {                                          // tan
                const double c = std::cos(x);
                GX[j] += g / (c * c);
                break;
            }
            case 11: GX[j] += g / (1.0 + x * x); break;         // atan, 375-378
            default: break;   // lnot, floor, ceil, round, clip: no backward branch
        }
    }
}

// ---------------------------------------------------------------------------
// bf16 (training.inc:1969-1976)
// ---------------------------------------------------------------------------
float orc_to_bf16(float x) {
    uint32_t u;
    std::memcpy(&u, &x, 4);
    u += 0x7FFFu + ((u >> 16) & 1u);   // bias so truncation rounds to nearest, ties to even
    u &= 0xFFFF0000u;
    float r;
    std::memcpy(&r, &u, 4);
    return r;
}

void orc_bf16_bits(const float* x, uint16_t* out, long long n) {
    for (long long i = 0; i < n; ++i) {
        const float r = orc_to_bf16(x[i]);
        uint32_t u;
        std::memcpy(&u, &r, 4);
        out[i] = (uint16_t)(u >> 16);
    }
}

