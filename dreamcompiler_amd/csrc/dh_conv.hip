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
// All three kernels are HBM-bound gathers / permutes; col2im gathers (each input element sums its KH*KW contributions in a fixed order), so it
// needs no atomics and reruns are bit-identical.
#include <algorithm>

#include "dh_common.hpp"

namespace dh {
namespace {

struct ConvShape {
    int N, Cin, H, W, KH, KW, pad, stride, OH, OW;
};

// Grids are 3-D: x = a chunk of one row's columns (or of one image plane), y = the col row
// (or channel), z = the image, so every per-row / per-plane index is decomposed once per
// work-group and a thread's own index with one multiply-shift division (32-bit: planes and
// rows of fewer than 2^31 elements, checked on the host).  y and z are launched in chunks of
// at most 65535 (y0, z0 the chunk's first row / image).  Outputs are streamed with
// non-temporal stores.

// col[r][n*P + p] for p = oh*OW + ow.  A work-group covers up to IM_SPAN columns of one
// (row, image); thread t takes columns t, t + 256, ... so every load and store instruction of
// a wave touches 64 consecutive columns (consecutive input elements where stride is 1).
constexpr uint32_t IM_SPAN = 4096, IM_UNROLL = 4;

__global__ void __launch_bounds__(256) im2col_kernel(const float* __restrict__ X,
                                                     float* __restrict__ col, ConvShape s,
                                                     FastDiv f_ow, int y0, int z0) {
    const int r = y0 + blockIdx.y, n = z0 + blockIdx.z;
    const int kw = r % s.KW, kh = (r / s.KW) % s.KH, ci = r / (s.KW * s.KH);
    const uint32_t P = (uint32_t)s.OH * (uint32_t)s.OW;
    const uint32_t end = min(P, (blockIdx.x + 1u) * IM_SPAN);
    const float* Xc = X + ((size_t)n * s.Cin + ci) * s.H * s.W;
    float* dst = col + (size_t)r * ((size_t)s.N * P) + (size_t)n * P;
    for (uint32_t p0 = blockIdx.x * IM_SPAN + threadIdx.x; p0 < end; p0 += 256u * IM_UNROLL) {
        float v[IM_UNROLL];
#pragma unroll
        for (uint32_t u = 0; u < IM_UNROLL; ++u) {
            const uint32_t p = p0 + 256u * u;
            float x = 0.f;
            if (p < end) {
                const uint32_t oh = fdiv(p, f_ow), ow = p - oh * (uint32_t)s.OW;
                const int h = (int)oh * s.stride + kh - s.pad, w = (int)ow * s.stride + kw - s.pad;
                if (h >= 0 && h < s.H && w >= 0 && w < s.W) x = Xc[h * s.W + w];
            }
            v[u] = x;
        }
#pragma unroll
        for (uint32_t u = 0; u < IM_UNROLL; ++u) {
            const uint32_t p = p0 + 256u * u;
            if (p < end) __builtin_nontemporal_store(v[u], dst + p);
        }
    }
}

// dX[n][ci][h][w] (+)= sum over (kh, kw) with h = oh*stride + kh - pad, w = ow*stride + kw - pad,
// in the order kh, then kw.
__global__ void __launch_bounds__(256) col2im_kernel(const float* __restrict__ dcol,
                                                     float* __restrict__ dX, ConvShape s,
                                                     FastDiv f_w, int acc, int y0, int z0) {
    const int ci = y0 + blockIdx.y, n = z0 + blockIdx.z;
    const uint32_t HW = (uint32_t)s.H * (uint32_t)s.W;
    const uint32_t hw = blockIdx.x * 256u + threadIdx.x;
    if (hw >= HW) return;
    const int h = (int)fdiv(hw, f_w), w = (int)(hw - (uint32_t)h * (uint32_t)s.W);
    const size_t P = (size_t)s.OH * s.OW, cols = (size_t)s.N * P;
    const float* src = dcol + (size_t)n * P;
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
            v += src[r * cols + (size_t)oh * s.OW + ow];
        }
    }
    float* o = dX + ((size_t)n * s.Cin + ci) * HW + hw;
    if (acc) *o += v;
    else __builtin_nontemporal_store(v, o);
}

// (N, C, T) -> (C, N*T): dst[(c*N + n)*T + t] = src[(n*C + c)*T + t], 4 values per thread.
template <bool VEC>
__global__ void __launch_bounds__(256) nct_to_cnt_kernel(const float* __restrict__ src,
                                                         float* __restrict__ dst, int N, int C,
                                                         uint32_t T, int y0, int z0) {
    const int c = y0 + blockIdx.y, n = z0 + blockIdx.z;
    const uint32_t t0 = (blockIdx.x * 256u + threadIdx.x) * 4u;
    if (t0 >= T) return;
    const float* a = src + ((size_t)n * C + c) * T + t0;
    float* b = dst + ((size_t)c * N + n) * T + t0;
    if (VEC) {
        __builtin_nontemporal_store(*reinterpret_cast<const f32x4*>(a), reinterpret_cast<f32x4*>(b));
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (t0 + e < T) __builtin_nontemporal_store(a[e], b + e);
    }
}

// Launch kern over a (gx, Y, Z) grid in y / z chunks of at most 65535.
template <typename Launch>
void launch_yz(unsigned gx, int Y, int Z, Launch launch) {
    for (int z0 = 0; z0 < Z; z0 += 65535)
        for (int y0 = 0; y0 < Y; y0 += 65535)
            launch(dim3(gx, (unsigned)std::min(65535, Y - y0), (unsigned)std::min(65535, Z - z0)),
                   y0, z0);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

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
    const size_t P = (size_t)s.OH * s.OW, R = (size_t)Cin * KH * KW;
    if (R * N * P == 0) return DH_OK;
    if (!X || !col) return set_error(DH_ERR_INVALID, "dh_im2col: null pointer");
    if (P >= (1u << 31) || R >= (1u << 31))
        return set_error(DH_ERR_UNSUPPORTED, "dh_im2col: %zu output positions x %zu rows", P, R);
    const FastDiv f_ow = make_fastdiv((uint32_t)s.OW);
    launch_yz((unsigned)((P + IM_SPAN - 1) / IM_SPAN), (int)R, N, [&](dim3 g, int y0, int z0) {
        im2col_kernel<<<g, 256, 0, stream()>>>(X, col, s, f_ow, y0, z0);
    });
    return check_launch("dh_im2col");
}

int dh_col2im(const float* dcol, float* dX, int N, int Cin, int H, int W, int KH, int KW, int pad,
              int stride, int accumulate) {
    DH_TRY(ensure_init());
    ConvShape s;
    DH_TRY(make_shape("dh_col2im", N, Cin, H, W, KH, KW, pad, stride, s));
    const size_t HW = (size_t)H * W;
    if ((size_t)N * Cin * HW == 0) return DH_OK;
    if (!dcol || !dX) return set_error(DH_ERR_INVALID, "dh_col2im: null pointer");
    if (HW >= (1u << 31)) return set_error(DH_ERR_UNSUPPORTED, "dh_col2im: %zu-element planes", HW);
    const FastDiv f_w = make_fastdiv((uint32_t)W);
    launch_yz((unsigned)((HW + 255) / 256), Cin, N, [&](dim3 g, int y0, int z0) {
        col2im_kernel<<<g, 256, 0, stream()>>>(dcol, dX, s, f_w, accumulate, y0, z0);
    });
    return check_launch("dh_col2im");
}

int dh_nct_to_cnt(const float* src, float* dst, int N, int C, size_t T) {
    DH_TRY(ensure_init());
    if (N < 0 || C < 0) return set_error(DH_ERR_INVALID, "dh_nct_to_cnt: negative shape");
    if ((size_t)N * C * T == 0) return DH_OK;
    if (!src || !dst) return set_error(DH_ERR_INVALID, "dh_nct_to_cnt: null pointer");
    if (T >= (1u << 31)) return set_error(DH_ERR_UNSUPPORTED, "dh_nct_to_cnt: T = %zu", T);
    const bool vec = T % 4 == 0 && aligned16(src) && aligned16(dst);
    launch_yz((unsigned)((T + 1023) / 1024), C, N, [&](dim3 g, int y0, int z0) {
        if (vec) nct_to_cnt_kernel<true><<<g, 256, 0, stream()>>>(src, dst, N, C, (uint32_t)T, y0, z0);
        else nct_to_cnt_kernel<false><<<g, 256, 0, stream()>>>(src, dst, N, C, (uint32_t)T, y0, z0);
    });
    return check_launch("dh_nct_to_cnt");
}

}  // extern "C"
