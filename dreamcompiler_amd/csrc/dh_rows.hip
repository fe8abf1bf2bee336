// dh_rows.hip -- row-wise kernels on gfx950: softmax / log_softmax and layer norm, forward and
// backward, fp32, rows of C contiguous values.
//
// Replaces the reference's scalar per-row loops: dream_softmax (runtime/ops/elementwise.inc:
// 338-358), dream_log_softmax (elementwise.inc:1550-1570), dream_layer_norm
// (runtime/io/builtins.inc:167-188) and their backward branches (runtime/ops/autograd.inc:
// 212-233, 396-409, 453-471).  All four are HBM-bound: each reads its inputs once and writes
// its output once.
//
// Rows of up to 1024 values: a segment of G lanes (G = 4, 16 or 64, the smallest that holds
// the row in at most 16 values per lane) owns one row and keeps it in registers, so every
// statistic (max, sums, mean, variance) is a segment reduction over registers and no value is
// read twice.  Lane s of a segment holds chunks s, s + G, s + 2G, ... of the row (a chunk is 4
// values with 16-byte loads when C % 4 == 0 and the pointers are 16-byte aligned, else 1), so
// one load instruction covers G consecutive chunks of every row in the wave.
// Longer rows: one 256-thread work-group per row, streaming the row from L2 once per pass.
#include "dh_common.hpp"

namespace dh {
namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

template <int G>
__device__ inline float seg_sum(float v) {
#pragma unroll
    for (int m = 1; m < G; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}
template <int G>
__device__ inline float seg_max(float v) {
#pragma unroll
    for (int m = 1; m < G; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}

// NV chunks of VEC values of one row, chunk t of lane s at element VEC (t G + s).
template <int G, int NV, int VEC>
struct Row {
    float v[NV][VEC];
    __device__ void load(const float* __restrict__ p, int C, int s, float fill) {
#pragma unroll
        for (int t = 0; t < NV; ++t) {
            const int e = VEC * (t * G + s);
            if (VEC == 4) {
                if (e < C) {
                    const f4 x = *reinterpret_cast<const f4*>(p + e);
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[t][q] = x[q];
                } else {
#pragma unroll
                    for (int q = 0; q < 4; ++q) v[t][q] = fill;
                }
            } else {
                v[t][0] = e < C ? p[e] : fill;
            }
        }
    }
    // Non-temporal: the output row is streamed out and not read again here, and keeping it
    // out of the caches leaves them to the inputs.
    __device__ void store(float* __restrict__ p, int C, int s) const {
#pragma unroll
        for (int t = 0; t < NV; ++t) {
            const int e = VEC * (t * G + s);
            if (e >= C) continue;
            if (VEC == 4) {
                __builtin_nontemporal_store(f4{v[t][0], v[t][1], v[t][2], v[t][3]},
                                            reinterpret_cast<f4*>(p + e));
            } else {
                __builtin_nontemporal_store(v[t][0], p + e);
            }
        }
    }
};

#define ROW_LOOP(stmt)                              \
    _Pragma("unroll") for (int t = 0; t < NV; ++t)  \
        _Pragma("unroll") for (int q = 0; q < VEC; ++q) { stmt; }

// Common prologue: 256 threads = 256 / G rows per work-group; a row index past R exits the
// whole segment (segments never straddle a wave, so the reductions stay within live lanes).
#define SEG_PROLOGUE()                                                    \
    const int s = threadIdx.x & (G - 1);                                  \
    const int row = blockIdx.x * (256 / G) + threadIdx.x / G;             \
    if (row >= R) return;                                                 \
    const size_t off = (size_t)row * C;

template <int G, int NV, int VEC>
__global__ void __launch_bounds__(256) softmax_seg(const float* __restrict__ X,
                                                   float* __restrict__ Y, int R, int C, int logsm) {
    SEG_PROLOGUE();
    Row<G, NV, VEC> x;
    x.load(X + off, C, s, -INFINITY);
    float mx = -INFINITY;
    ROW_LOOP(mx = fmaxf(mx, x.v[t][q]));
    mx = seg_max<G>(mx);
    float sum = 0.f;
    ROW_LOOP(sum += __expf(x.v[t][q] - mx));
    sum = seg_sum<G>(sum);
    if (logsm) {
        const float lse = mx + __logf(sum);
        ROW_LOOP(x.v[t][q] -= lse);
    } else {
        const float inv = 1.f / sum;
        ROW_LOOP(x.v[t][q] = __expf(x.v[t][q] - mx) * inv);
    }
    x.store(Y + off, C, s);
}

// softmax:     gx (+)= y (g - sum(g y))
// log_softmax: gx (+)= g - exp(y) sum(g)      (y = log_softmax(x), so exp(y) = softmax(x))
template <int G, int NV, int VEC>
__global__ void __launch_bounds__(256) softmax_bwd_seg(const float* __restrict__ Yf,
                                                       const float* __restrict__ Gr,
                                                       float* __restrict__ GX, int R, int C,
                                                       int logsm, int acc) {
    SEG_PROLOGUE();
    Row<G, NV, VEC> y, g;
    y.load(Yf + off, C, s, 0.f);
    g.load(Gr + off, C, s, 0.f);
    float red = 0.f;
    if (logsm) {
        ROW_LOOP(red += g.v[t][q]);
    } else {
        ROW_LOOP(red += g.v[t][q] * y.v[t][q]);
    }
    red = seg_sum<G>(red);
    if (logsm) {
        ROW_LOOP(y.v[t][q] = g.v[t][q] - __expf(y.v[t][q]) * red);
    } else {
        ROW_LOOP(y.v[t][q] = y.v[t][q] * (g.v[t][q] - red));
    }
    if (acc) {
        Row<G, NV, VEC> o;
        o.load(GX + off, C, s, 0.f);
        ROW_LOOP(y.v[t][q] += o.v[t][q]);
    }
    y.store(GX + off, C, s);
}

// Per-row mean and inverse standard deviation (biased variance, eps 1e-5) from registers;
// padding chunks hold 0 and are excluded from the variance by the element count.
template <int G, int NV, int VEC>
__device__ inline void row_stats(const Row<G, NV, VEC>& x, int C, int s, float& mu,
                                 float& inv_std) {
    float sum = 0.f;
    ROW_LOOP(sum += x.v[t][q]);
    mu = seg_sum<G>(sum) / (float)C;
    float var = 0.f;
#pragma unroll
    for (int t = 0; t < NV; ++t)
#pragma unroll
        for (int q = 0; q < VEC; ++q) {
            const float d = VEC * (t * G + s) + q < C ? x.v[t][q] - mu : 0.f;
            var += d * d;
        }
    var = seg_sum<G>(var) / (float)C;
    inv_std = rsqrtf(var + 1e-5f);
}

template <int G, int NV, int VEC>
__global__ void __launch_bounds__(256) layer_norm_seg(const float* __restrict__ X,
                                                      float* __restrict__ Y, int R, int C) {
    SEG_PROLOGUE();
    Row<G, NV, VEC> x;
    x.load(X + off, C, s, 0.f);
    float mu, inv_std;
    row_stats(x, C, s, mu, inv_std);
    ROW_LOOP(x.v[t][q] = (x.v[t][q] - mu) * inv_std);
    x.store(Y + off, C, s);
}

// gx (+)= inv_std / C (C dy - sum(dy) - y sum(dy y)), inv_std recomputed from x.
template <int G, int NV, int VEC>
__global__ void __launch_bounds__(256) layer_norm_bwd_seg(const float* __restrict__ X,
                                                          const float* __restrict__ Yf,
                                                          const float* __restrict__ DY,
                                                          float* __restrict__ GX, int R, int C,
                                                          int acc) {
    SEG_PROLOGUE();
    float mu, inv_std;
    {
        Row<G, NV, VEC> x;
        x.load(X + off, C, s, 0.f);
        row_stats(x, C, s, mu, inv_std);
    }
    Row<G, NV, VEC> y, dy;
    y.load(Yf + off, C, s, 0.f);
    dy.load(DY + off, C, s, 0.f);
    float sdy = 0.f, sdyy = 0.f;
    ROW_LOOP(sdy += dy.v[t][q]; sdyy += dy.v[t][q] * y.v[t][q]);
    sdy = seg_sum<G>(sdy);
    sdyy = seg_sum<G>(sdyy);
    const float k = inv_std / (float)C, fc = (float)C;
    ROW_LOOP(y.v[t][q] = k * (fc * dy.v[t][q] - sdy - y.v[t][q] * sdyy));
    if (acc) {
        Row<G, NV, VEC> o;
        o.load(GX + off, C, s, 0.f);
        ROW_LOOP(y.v[t][q] += o.v[t][q]);
    }
    y.store(GX + off, C, s);
}

// ---- long rows: one work-group of 256 threads per row, streaming ---------------------------
template <typename Op>
__device__ inline float block_reduce(float v, Op op, float* red) {
    v = wave_reduce(v, op);
    const int w = threadIdx.x >> 6;
    __syncthreads();   // red[] may still be read from a previous reduction
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    return op(op(red[0], red[1]), op(red[2], red[3]));
}

__global__ void __launch_bounds__(256) softmax_blk(const float* __restrict__ X,
                                                   float* __restrict__ Y, int C, int logsm) {
    __shared__ float red[4];
    const float* x = X + (size_t)blockIdx.x * C;
    float* y = Y + (size_t)blockIdx.x * C;
    float mx = -INFINITY;
    for (int j = threadIdx.x; j < C; j += 256) mx = fmaxf(mx, x[j]);
    mx = block_reduce(mx, OpMax(), red);
    float sum = 0.f;
    for (int j = threadIdx.x; j < C; j += 256) sum += __expf(x[j] - mx);
    sum = block_reduce(sum, OpSum(), red);
    if (logsm) {
        const float lse = mx + __logf(sum);
        for (int j = threadIdx.x; j < C; j += 256) y[j] = x[j] - lse;
    } else {
        const float inv = 1.f / sum;
        for (int j = threadIdx.x; j < C; j += 256) y[j] = __expf(x[j] - mx) * inv;
    }
}

__global__ void __launch_bounds__(256) softmax_bwd_blk(const float* __restrict__ Yf,
                                                       const float* __restrict__ Gr,
                                                       float* __restrict__ GX, int C, int logsm,
                                                       int acc) {
    __shared__ float red[4];
    const size_t off = (size_t)blockIdx.x * C;
    const float *y = Yf + off, *g = Gr + off;
    float* gx = GX + off;
    float r = 0.f;
    for (int j = threadIdx.x; j < C; j += 256) r += logsm ? g[j] : g[j] * y[j];
    r = block_reduce(r, OpSum(), red);
    for (int j = threadIdx.x; j < C; j += 256) {
        const float v = logsm ? g[j] - __expf(y[j]) * r : y[j] * (g[j] - r);
        gx[j] = acc ? gx[j] + v : v;
    }
}

__device__ inline void blk_stats(const float* x, int C, float* red, float& mu, float& inv_std) {
    float sum = 0.f;
    for (int j = threadIdx.x; j < C; j += 256) sum += x[j];
    mu = block_reduce(sum, OpSum(), red) / (float)C;
    float var = 0.f;
    for (int j = threadIdx.x; j < C; j += 256) {
        const float d = x[j] - mu;
        var += d * d;
    }
    inv_std = rsqrtf(block_reduce(var, OpSum(), red) / (float)C + 1e-5f);
}

__global__ void __launch_bounds__(256) layer_norm_blk(const float* __restrict__ X,
                                                      float* __restrict__ Y, int C) {
    __shared__ float red[4];
    const float* x = X + (size_t)blockIdx.x * C;
    float* y = Y + (size_t)blockIdx.x * C;
    float mu, inv_std;
    blk_stats(x, C, red, mu, inv_std);
    for (int j = threadIdx.x; j < C; j += 256) y[j] = (x[j] - mu) * inv_std;
}

__global__ void __launch_bounds__(256) layer_norm_bwd_blk(const float* __restrict__ X,
                                                          const float* __restrict__ Yf,
                                                          const float* __restrict__ DY,
                                                          float* __restrict__ GX, int C, int acc) {
    __shared__ float red[4];
    const size_t off = (size_t)blockIdx.x * C;
    const float *x = X + off, *y = Yf + off, *dy = DY + off;
    float* gx = GX + off;
    float mu, inv_std;
    blk_stats(x, C, red, mu, inv_std);
    float sdy = 0.f, sdyy = 0.f;
    for (int j = threadIdx.x; j < C; j += 256) {
        sdy += dy[j];
        sdyy += dy[j] * y[j];
    }
    sdy = block_reduce(sdy, OpSum(), red);
    sdyy = block_reduce(sdyy, OpSum(), red);
    const float k = inv_std / (float)C, fc = (float)C;
    for (int j = threadIdx.x; j < C; j += 256) {
        const float v = k * (fc * dy[j] - sdy - y[j] * sdyy);
        gx[j] = acc ? gx[j] + v : v;
    }
}

// ---- linear backward: ReLU mask and bias gradient ------------------------------------------
// Work-group (bx, by): 64 columns (one per lane, so each row's piece is one coalesced load) and
// the rows by, by + P, by + 2P, ... split over its 4 waves.  Partial column sums go to
// part[by][col] and a second pass adds the P partials in a fixed order: no atomics, so reruns
// are bit-identical.
__global__ void __launch_bounds__(256) bias_grad_partial(const float* __restrict__ Y,
                                                         float* __restrict__ dY,
                                                         float* __restrict__ part, int N,
                                                         int out, int relu) {
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    const int P = gridDim.y;
    float s = 0.f;
    if (col < out) {
        for (int i = blockIdx.y + P * w; i < N; i += 4 * P) {
            const size_t e = (size_t)i * out + col;
            float g = dY[e];
            if (relu && !(Y[e] > 0.f)) {   // the reference zeroes dY where Y <= 0, in place
                g = 0.f;
                dY[e] = 0.f;
            }
            s += g;
        }
    }
    red[w][lane] = s;
    __syncthreads();
    if (w == 0 && col < out)
        part[(size_t)blockIdx.y * out + col] = (red[0][lane] + red[1][lane]) + (red[2][lane] + red[3][lane]);
}

__global__ void __launch_bounds__(256) bias_grad_final(const float* __restrict__ part,
                                                       float* __restrict__ db, int P, int out,
                                                       int acc) {
    const int col = blockIdx.x * 256 + threadIdx.x;
    if (col >= out) return;
    float s = 0.f;
    for (int p = 0; p < P; ++p) s += part[(size_t)p * out + col];
    db[col] = acc ? db[col] + s : s;
}

// ---- dispatch --------------------------------------------------------------------------------
constexpr int SEG_MAX_C = 1024;

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

template <int G>
constexpr unsigned seg_grid(int R) { return (unsigned)((R + 256 / G - 1) / (256 / G)); }

template <int G, int NV, int VEC>
int launch_softmax(const float* X, float* Y, int R, int C, int lg) {
    softmax_seg<G, NV, VEC><<<seg_grid<G>(R), 256, 0, stream()>>>(X, Y, R, C, lg);
    return check_launch("dh_row_softmax");
}
template <int G, int NV, int VEC>
int launch_softmax_bwd(const float* Y, const float* Gr, float* GX, int R, int C, int lg, int acc) {
    softmax_bwd_seg<G, NV, VEC><<<seg_grid<G>(R), 256, 0, stream()>>>(Y, Gr, GX, R, C, lg, acc);
    return check_launch("dh_row_softmax_bwd");
}
template <int G, int NV, int VEC>
int launch_layer_norm(const float* X, float* Y, int R, int C) {
    layer_norm_seg<G, NV, VEC><<<seg_grid<G>(R), 256, 0, stream()>>>(X, Y, R, C);
    return check_launch("dh_layer_norm");
}
template <int G, int NV, int VEC>
int launch_layer_norm_bwd(const float* X, const float* Y, const float* DY, float* GX, int R, int C,
                          int acc) {
    layer_norm_bwd_seg<G, NV, VEC><<<seg_grid<G>(R), 256, 0, stream()>>>(X, Y, DY, GX, R, C, acc);
    return check_launch("dh_layer_norm_bwd");
}

// The smallest segment that holds a row of C values in at most 16 values per lane (chunks of 4
// when `vec`).
#define SEG_DISPATCH(C, vec, FN, ...)                                                      \
    ((vec) ? ((C) / 4 <= 16 ? FN<4, 4, 4>(__VA_ARGS__)                                     \
                            : (C) / 4 <= 64 ? FN<16, 4, 4>(__VA_ARGS__) : FN<64, 4, 4>(__VA_ARGS__)) \
           : ((C) <= 64 ? FN<4, 16, 1>(__VA_ARGS__)                                        \
                        : (C) <= 256 ? FN<16, 16, 1>(__VA_ARGS__) : FN<64, 16, 1>(__VA_ARGS__)))

int check_rows(const char* op, int R, int C) {
    if (R < 0 || C < 0) return set_error(DH_ERR_INVALID, "%s: negative shape", op);
    return DH_OK;
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" {

int dh_row_softmax(const float* X, float* Y, int R, int C, int log_softmax) {
    DH_TRY(ensure_init());
    DH_TRY(check_rows("dh_row_softmax", R, C));
    if (R == 0 || C == 0) return DH_OK;
    if (!X || !Y) return set_error(DH_ERR_INVALID, "dh_row_softmax: null pointer");
    if (C > SEG_MAX_C) {
        softmax_blk<<<R, 256, 0, stream()>>>(X, Y, C, log_softmax);
        return check_launch("dh_row_softmax");
    }
    return SEG_DISPATCH(C, C % 4 == 0 && aligned16(X) && aligned16(Y), launch_softmax, X, Y, R, C,
                        log_softmax);
}

int dh_row_softmax_bwd(const float* Y, const float* G, float* GX, int R, int C, int log_softmax,
                       int accumulate) {
    DH_TRY(ensure_init());
    DH_TRY(check_rows("dh_row_softmax_bwd", R, C));
    if (R == 0 || C == 0) return DH_OK;
    if (!Y || !G || !GX) return set_error(DH_ERR_INVALID, "dh_row_softmax_bwd: null pointer");
    if (C > SEG_MAX_C) {
        softmax_bwd_blk<<<R, 256, 0, stream()>>>(Y, G, GX, C, log_softmax, accumulate);
        return check_launch("dh_row_softmax_bwd");
    }
    return SEG_DISPATCH(C, C % 4 == 0 && aligned16(Y) && aligned16(G) && aligned16(GX),
                        launch_softmax_bwd, Y, G, GX, R, C, log_softmax, accumulate);
}

int dh_layer_norm(const float* X, float* Y, int R, int C) {
    DH_TRY(ensure_init());
    DH_TRY(check_rows("dh_layer_norm", R, C));
    if (R == 0 || C == 0) return DH_OK;
    if (!X || !Y) return set_error(DH_ERR_INVALID, "dh_layer_norm: null pointer");
    if (C > SEG_MAX_C) {
        layer_norm_blk<<<R, 256, 0, stream()>>>(X, Y, C);
        return check_launch("dh_layer_norm");
    }
    return SEG_DISPATCH(C, C % 4 == 0 && aligned16(X) && aligned16(Y), launch_layer_norm, X, Y, R,
                        C);
}

int dh_layer_norm_bwd(const float* X, const float* Y, const float* DY, float* GX, int R, int C,
                      int accumulate) {
    DH_TRY(ensure_init());
    DH_TRY(check_rows("dh_layer_norm_bwd", R, C));
    if (R == 0 || C == 0) return DH_OK;
    if (!X || !Y || !DY || !GX) return set_error(DH_ERR_INVALID, "dh_layer_norm_bwd: null pointer");
    if (C > SEG_MAX_C) {
        layer_norm_bwd_blk<<<R, 256, 0, stream()>>>(X, Y, DY, GX, C, accumulate);
        return check_launch("dh_layer_norm_bwd");
    }
    return SEG_DISPATCH(C, C % 4 == 0 && aligned16(X) && aligned16(Y) && aligned16(DY) &&
                               aligned16(GX),
                        launch_layer_norm_bwd, X, Y, DY, GX, R, C, accumulate);
}

int dh_linear_bias_grad(const float* Y, float* dY, float* db, int N, int out, int relu,
                        int accumulate) {
    DH_TRY(ensure_init());
    if (N < 0 || out < 0) return set_error(DH_ERR_INVALID, "dh_linear_bias_grad: negative shape");
    if (out == 0) return DH_OK;
    if (!dY || !db || (relu && !Y))
        return set_error(DH_ERR_INVALID, "dh_linear_bias_grad: null pointer");
    const int cgroups = (out + 63) / 64;
    int P = 1024 / cgroups;                       // enough work-groups to cover the chip
    P = P < 1 ? 1 : P;
    P = P > (N + 63) / 64 ? (N + 63) / 64 : P;    // at least 64 rows per partial
    if (P < 1) P = 1;
    float* part = static_cast<float*>(dh_malloc((size_t)P * out * sizeof(float)));
    if (!part) return set_error(DH_ERR_OOM, "dh_linear_bias_grad: scratch of %d x %d", P, out);
    bias_grad_partial<<<dim3(cgroups, P), 256, 0, stream()>>>(Y, dY, part, N, out, relu);
    int st = check_launch("dh_linear_bias_grad");
    if (st == DH_OK) {
        bias_grad_final<<<(out + 255) / 256, 256, 0, stream()>>>(part, db, P, out, accumulate);
        st = check_launch("dh_linear_bias_grad");
    }
    dh_free(part);   // pooled: the buffer returns to its bucket, stream order keeps it safe
    return st;
}

}  // extern "C"
