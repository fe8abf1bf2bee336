// dh_conv.hip -- the data-movement kernels of conv2d on gfx950: im2col, col2im and a channel
// permute, fp32.  The products themselves are dh_gemm_f32_ex calls.
//
// Replaces the reference's per-image host loops around cpu_gemm (runtime/nn/conv.inc:12-55,
// 119-178; im2col / col2im, runtime/nn/im2col.inc:2-25; the conv2d backward,
// runtime/ops/autograd.inc:507-535).  Layout chosen so that every product is one launch:
//   col  (Cin*KH*KW) x (N*OH*OW): row r = (ci*KH + kh)*KW + kw, column n*OH*OW + oh*OW + ow --
//        all images side by side, so the forward is one batched NN GEMM (the kernel shared by
//        a zero stride, B member n at column offset n*OH*OW) and the weight gradient one NT GEMM
//        with contraction length N*OH*OW;
//   go'  Cout x (N*OH*OW): the output gradient with its channel axis first (dh_nct_to_cnt),
//        the other operand of both backward products.
// All three kernels are HBM-bound gathers/scatters with one thread per output element;
// col2im gathers (each input element sums its KH*KW contributions in a fixed order), so it
// needs no atomics and reruns are bit-identical.
#include "dh_common.hpp"

namespace dh {
namespace {

struct ConvShape {
    int N, Cin, H, W, KH, KW, pad, stride, OH, OW;
};

__global__ void __launch_bounds__(256) im2col_kernel(const float* __restrict__ X,
                                                     float* __restrict__ col, ConvShape s) {
    const size_t P = (size_t)s.OH * s.OW, cols = (size_t)s.N * P;
    const size_t total = (size_t)s.Cin * s.KH * s.KW * cols;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (size_t)gridDim.x * 256) {
        const size_t r = e / cols, c = e % cols;
        const int kw = (int)(r % s.KW), kh = (int)((r / s.KW) % s.KH), ci = (int)(r / s.KW / s.KH);
        const int n = (int)(c / P), p = (int)(c % P), oh = p / s.OW, ow = p % s.OW;
        const int h = oh * s.stride + kh - s.pad, w = ow * s.stride + kw - s.pad;
        col[e] = (h >= 0 && h < s.H && w >= 0 && w < s.W)
                     ? X[(((size_t)n * s.Cin + ci) * s.H + h) * s.W + w]
                     : 0.f;
    }
}

// dX[n][ci][h][w] (+)= sum over (kh, kw) with h = oh*stride + kh - pad, w = ow*stride + kw - pad.
__global__ void __launch_bounds__(256) col2im_kernel(const float* __restrict__ dcol,
                                                     float* __restrict__ dX, ConvShape s, int acc) {
    const size_t P = (size_t)s.OH * s.OW, cols = (size_t)s.N * P;
    const size_t total = (size_t)s.N * s.Cin * s.H * s.W;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (size_t)gridDim.x * 256) {
        const int w = (int)(e % s.W), h = (int)((e / s.W) % s.H);
        const int ci = (int)((e / ((size_t)s.W * s.H)) % s.Cin), n = (int)(e / ((size_t)s.W * s.H * s.Cin));
        float v = 0.f;
        for (int kh = 0; kh < s.KH; ++kh) {
            const int th = h + s.pad - kh;
            if (th < 0 || th % s.stride) continue;
            const int oh = th / s.stride;
            if (oh >= s.OH) continue;
            for (int kw = 0; kw < s.KW; ++kw) {
                const int tw = w + s.pad - kw;
                if (tw < 0 || tw % s.stride) continue;
                const int ow = tw / s.stride;
                if (ow >= s.OW) continue;
                const size_t r = ((size_t)ci * s.KH + kh) * s.KW + kw;
                v += dcol[r * cols + (size_t)n * P + (size_t)oh * s.OW + ow];
            }
        }
        dX[e] = acc ? dX[e] + v : v;
    }
}

// (N, C, T) -> (C, N*T)
__global__ void __launch_bounds__(256) nct_to_cnt_kernel(const float* __restrict__ src,
                                                         float* __restrict__ dst, int N, int C,
                                                         size_t T) {
    const size_t total = (size_t)N * C * T;
    for (size_t e = (size_t)blockIdx.x * 256 + threadIdx.x; e < total;
         e += (size_t)gridDim.x * 256) {
        const size_t t = e % T, c = (e / T) % C, n = e / (T * C);
        dst[(c * N + n) * T + t] = src[e];
    }
}

unsigned grid_for(size_t total) {
    size_t b = (total + 255) / 256;
    const size_t cap = (size_t)num_cus() * 32;
    return (unsigned)(b < cap ? (b ? b : 1) : cap);
}

int make_shape(const char* op, int N, int Cin, int H, int W, int KH, int KW, int pad, int stride,
               ConvShape& s) {
    if (N < 0 || Cin < 1 || H < 1 || W < 1 || KH < 1 || KW < 1 || pad < 0 || stride < 1)
        return set_error(DH_ERR_INVALID, "%s: invalid shape", op);
    s = {N, Cin, H, W, KH, KW, pad, stride, (H + 2 * pad - KH) / stride + 1,
         (W + 2 * pad - KW) / stride + 1};
    if (H + 2 * pad < KH || W + 2 * pad < KW)
        return set_error(DH_ERR_INVALID, "%s: kernel larger than the padded input", op);
    return DH_OK;
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" {

int dh_im2col(const float* X, float* col, int N, int Cin, int H, int W, int KH, int KW, int pad,
              int stride) {
    DH_TRY(ensure_init());
    ConvShape s;
    DH_TRY(make_shape("dh_im2col", N, Cin, H, W, KH, KW, pad, stride, s));
    const size_t total = (size_t)Cin * KH * KW * N * s.OH * s.OW;
    if (total == 0) return DH_OK;
    if (!X || !col) return set_error(DH_ERR_INVALID, "dh_im2col: null pointer");
    im2col_kernel<<<grid_for(total), 256, 0, stream()>>>(X, col, s);
    return check_launch("dh_im2col");
}

int dh_col2im(const float* dcol, float* dX, int N, int Cin, int H, int W, int KH, int KW, int pad,
              int stride, int accumulate) {
    DH_TRY(ensure_init());
    ConvShape s;
    DH_TRY(make_shape("dh_col2im", N, Cin, H, W, KH, KW, pad, stride, s));
    const size_t total = (size_t)N * Cin * H * W;
    if (total == 0) return DH_OK;
    if (!dcol || !dX) return set_error(DH_ERR_INVALID, "dh_col2im: null pointer");
    col2im_kernel<<<grid_for(total), 256, 0, stream()>>>(dcol, dX, s, accumulate);
    return check_launch("dh_col2im");
}

int dh_nct_to_cnt(const float* src, float* dst, int N, int C, size_t T) {
    DH_TRY(ensure_init());
    if (N < 0 || C < 0) return set_error(DH_ERR_INVALID, "dh_nct_to_cnt: negative shape");
    const size_t total = (size_t)N * C * T;
    if (total == 0) return DH_OK;
    if (!src || !dst) return set_error(DH_ERR_INVALID, "dh_nct_to_cnt: null pointer");
    nct_to_cnt_kernel<<<grid_for(total), 256, 0, stream()>>>(src, dst, N, C, T);
    return check_launch("dh_nct_to_cnt");
}

}  // extern "C"
