// dh_elementwise.hip -- elementwise binary ops over broadcast strides and unary ops, fp32 or
// fp64 (replaces runGPU / runGPUUnary, runtime/backend/gpu.inc:637-716, whose OpenCL kernels
// index C's flat position i as (i0, i1, i2, i3) over C's dims and read A, B at
// i0*s0 + i1*s1 + i2*s2 + i3*s3 with zero strides on broadcast dims, bcastStrides at
// gpu.inc:443-449).
//
// HBM-bound streaming: one pass over A, B and C.  On the host the 4 dims are collapsed (size-1
// dims dropped, neighbours merged where both operands stay linear across them), so the
// common cases -- same shape, a scalar operand, a row or column broadcast -- reach the kernel
// with one or two dims.  Same-shape contiguous operands take a 16-byte vector path; the rest
// decompose i with multiply-shift division by the launch-invariant dims.
#include <cmath>

#include "dh_common.hpp"

namespace dh {
namespace {

constexpr int EW_THREADS = 256;
constexpr int EW_UNROLL = 4;

// Binary op codes in the order of the reference's BinopCode (gpu.inc:455-460).
template <int OP, typename T>
__device__ inline T bin(T a, T b) {
    constexpr T one = T(1), zero = T(0);
    constexpr T eps = T(1e-6);   // eq / ne tolerance: 1e-6f in the kernels, 1e-6 on the CPU path
    if constexpr (OP == DH_BOP_ADD) return a + b;
    else if constexpr (OP == DH_BOP_SUB) return a - b;
    else if constexpr (OP == DH_BOP_MUL) return a * b;
    else if constexpr (OP == DH_BOP_DIV) return a / b;
    else if constexpr (OP == DH_BOP_MOD) return std::fmod(a, b);
    else if constexpr (OP == DH_BOP_GT) return a > b ? one : zero;
    else if constexpr (OP == DH_BOP_LT) return a < b ? one : zero;
    else if constexpr (OP == DH_BOP_GE) return a >= b ? one : zero;
    else if constexpr (OP == DH_BOP_LE) return a <= b ? one : zero;
    else if constexpr (OP == DH_BOP_EQ) return std::fabs(a - b) < eps ? one : zero;
    else if constexpr (OP == DH_BOP_NE) return std::fabs(a - b) >= eps ? one : zero;
    else if constexpr (OP == DH_BOP_AND) return (a > zero && b > zero) ? one : zero;
    else if constexpr (OP == DH_BOP_OR) return (a > zero || b > zero) ? one : zero;
    else if constexpr (OP == DH_BOP_ATAN2) return std::atan2(a, b);
    else if constexpr (OP == DH_BOP_POW) return std::pow(a, b);
    else if constexpr (OP == DH_BOP_MIN) return a < b ? a : b;
    else return a > b ? a : b;   // DH_BOP_MAX
}

// Unary op codes in the order of the reference's UnopCode (gpu.inc:571-577), then clip.
template <int OP, typename T>
__device__ inline T un(T a, T lo, T hi) {
    constexpr T one = T(1), zero = T(0);
    if constexpr (OP == DH_UOP_RELU) return a > zero ? a : zero;
    else if constexpr (OP == DH_UOP_EXP) return std::exp(a);
    else if constexpr (OP == DH_UOP_LOG) return std::log(a);
    else if constexpr (OP == DH_UOP_SQRT) return std::sqrt(a);
    else if constexpr (OP == DH_UOP_ABS) return std::fabs(a);
    else if constexpr (OP == DH_UOP_SIGMOID) return one / (one + std::exp(-a));
    else if constexpr (OP == DH_UOP_TANH) return std::tanh(a);
    else if constexpr (OP == DH_UOP_LNOT) return a == zero ? one : zero;
    else if constexpr (OP == DH_UOP_SIN) return std::sin(a);
    else if constexpr (OP == DH_UOP_COS) return std::cos(a);
    else if constexpr (OP == DH_UOP_TAN) return std::tan(a);
    else if constexpr (OP == DH_UOP_ATAN) return std::atan(a);
    else if constexpr (OP == DH_UOP_FLOOR) return std::floor(a);
    else if constexpr (OP == DH_UOP_CEIL) return std::ceil(a);
    else if constexpr (OP == DH_UOP_ROUND) return std::round(a);
    else return std::fmax(lo, std::fmin(hi, a));   // DH_UOP_CLIP (dream_clip, elementwise.inc:329-336)
}

// 16-byte vectors: 4 floats or 2 doubles.
template <typename T>
struct V16 {
    static constexpr int N = 16 / sizeof(T);
    typedef T type __attribute__((ext_vector_type(N)));
};

// Results are written with non-temporal stores: a streamed output is not read again by this
// kernel, and keeping it out of the caches leaves them to the inputs (measured: a same-shape
// fp64 add at 4096 x 4096 goes from 5.1 to 7.9 TB/s).
template <typename V>
__device__ inline void st_nt(V* p, const V& v) {
    __builtin_nontemporal_store(v, p);
}

template <typename T>
__device__ inline void store32(float* c32, size_t i, const typename V16<T>::type& v) {
    if constexpr (V16<T>::N == 2) {
        typedef float f32x2 __attribute__((ext_vector_type(2)));
        f32x2 w = {(float)v[0], (float)v[1]};
        st_nt(reinterpret_cast<f32x2*>(c32 + i), w);
    } else {
        st_nt(reinterpret_cast<f32x4*>(c32 + i), v);
    }
}

// Same-shape contiguous operands.  Vector part: UNROLL 16-byte vectors per thread per step,
// loads first; the tail (< one vector per thread) is done element by element by block 0.
template <int OP, typename T>
__global__ void __launch_bounds__(EW_THREADS)
binary_contig_kernel(const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C,
                     float* __restrict__ C32, size_t n) {
    using VT = typename V16<T>::type;
    constexpr int NV = V16<T>::N;
    const size_t nvec = n / NV;
    const size_t stride = (size_t)gridDim.x * EW_THREADS;
    const VT* Av = reinterpret_cast<const VT*>(A);
    const VT* Bv = reinterpret_cast<const VT*>(B);
    VT* Cv = reinterpret_cast<VT*>(C);
    for (size_t v0 = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; v0 < nvec;
         v0 += stride * EW_UNROLL) {
        VT a[EW_UNROLL], b[EW_UNROLL];
#pragma unroll
        for (int u = 0; u < EW_UNROLL; ++u) {
            const size_t v = v0 + u * stride;
            if (v < nvec) {
                a[u] = Av[v];
                b[u] = Bv[v];
            }
        }
#pragma unroll
        for (int u = 0; u < EW_UNROLL; ++u) {
            const size_t v = v0 + u * stride;
            if (v < nvec) {
                VT c;
#pragma unroll
                for (int e = 0; e < NV; ++e) c[e] = bin<OP, T>(a[u][e], b[u][e]);
                st_nt(&Cv[v], c);
                if (C32) store32<T>(C32, v * NV, c);
            }
        }
    }
    if (blockIdx.x == 0) {
        for (size_t i = nvec * NV + threadIdx.x; i < n; i += EW_THREADS) {
            const T c = bin<OP, T>(A[i], B[i]);
            st_nt(&C[i], c);
            if (C32) st_nt(&C32[i], (float)c);
        }
    }
}

// Collapsed broadcast shape: dims[0..3] (outermost first, padded with 1s in front),
// element strides of A and B per dim (0 where broadcast).
struct BcastShape {
    FastDiv div[4];
    int sa[4], sb[4];
};

template <int OP, typename T>
__global__ void __launch_bounds__(EW_THREADS)
binary_bcast_kernel(const T* __restrict__ A, const T* __restrict__ B, T* __restrict__ C,
                    float* __restrict__ C32, uint32_t n, BcastShape sh) {
    const uint32_t stride = gridDim.x * EW_THREADS;
    for (uint32_t i = blockIdx.x * EW_THREADS + threadIdx.x; i < n; i += stride) {
        uint32_t r = i, ia = 0, ib = 0;
#pragma unroll
        for (int k = 3; k >= 1; --k) {
            const uint32_t q = fdiv(r, sh.div[k]);
            const uint32_t x = r - q * sh.div[k].d;
            ia += x * (uint32_t)sh.sa[k];
            ib += x * (uint32_t)sh.sb[k];
            r = q;
        }
        ia += r * (uint32_t)sh.sa[0];
        ib += r * (uint32_t)sh.sb[0];
        const T c = bin<OP, T>(A[ia], B[ib]);
        st_nt(&C[i], c);
        if (C32) st_nt(&C32[i], (float)c);
    }
}

template <int OP, typename T>
__global__ void __launch_bounds__(EW_THREADS)
unary_kernel(const T* __restrict__ A, T* __restrict__ C, float* __restrict__ C32, size_t n, T lo,
             T hi) {
    using VT = typename V16<T>::type;
    constexpr int NV = V16<T>::N;
    const size_t nvec = n / NV;
    const size_t stride = (size_t)gridDim.x * EW_THREADS;
    const VT* Av = reinterpret_cast<const VT*>(A);
    VT* Cv = reinterpret_cast<VT*>(C);
    for (size_t v0 = (size_t)blockIdx.x * EW_THREADS + threadIdx.x; v0 < nvec;
         v0 += stride * EW_UNROLL) {
        VT a[EW_UNROLL];
#pragma unroll
        for (int u = 0; u < EW_UNROLL; ++u) {
            const size_t v = v0 + u * stride;
            if (v < nvec) a[u] = Av[v];
        }
#pragma unroll
        for (int u = 0; u < EW_UNROLL; ++u) {
            const size_t v = v0 + u * stride;
            if (v < nvec) {
                VT c;
#pragma unroll
                for (int e = 0; e < NV; ++e) c[e] = un<OP, T>(a[u][e], lo, hi);
                st_nt(&Cv[v], c);
                if (C32) store32<T>(C32, v * NV, c);
            }
        }
    }
    if (blockIdx.x == 0) {
        for (size_t i = nvec * NV + threadIdx.x; i < n; i += EW_THREADS) {
            const T c = un<OP, T>(A[i], lo, hi);
            st_nt(&C[i], c);
            if (C32) st_nt(&C32[i], (float)c);
        }
    }
}

unsigned grid_for(size_t work_items) {
    size_t blocks = (work_items + EW_THREADS - 1) / EW_THREADS;
    const size_t cap = (size_t)num_cus() * 8;   // 8 work-groups of 4 waves per CU
    if (blocks > cap) blocks = cap;
    return (unsigned)(blocks ? blocks : 1);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <typename T>
int launch_binary(int op, const T* A, const T* B, T* C, float* C32, size_t n, bool contig,
                  const BcastShape& sh) {
    constexpr int NV = V16<T>::N;
    const unsigned gc = grid_for((n / NV + EW_UNROLL - 1) / EW_UNROLL);
    const unsigned gb = grid_for(n);
    switch (op) {
#define DH_BIN_CASE(OP)                                                                      \
    case OP:                                                                                 \
        if (contig)                                                                          \
            binary_contig_kernel<OP, T><<<gc, EW_THREADS, 0, stream()>>>(A, B, C, C32, n);   \
        else                                                                                 \
            binary_bcast_kernel<OP, T><<<gb, EW_THREADS, 0, stream()>>>(A, B, C, C32,        \
                                                                        (uint32_t)n, sh);    \
        break;
        DH_BIN_CASE(DH_BOP_ADD) DH_BIN_CASE(DH_BOP_SUB) DH_BIN_CASE(DH_BOP_MUL)
        DH_BIN_CASE(DH_BOP_DIV) DH_BIN_CASE(DH_BOP_MOD) DH_BIN_CASE(DH_BOP_GT)
        DH_BIN_CASE(DH_BOP_LT) DH_BIN_CASE(DH_BOP_GE) DH_BIN_CASE(DH_BOP_LE)
        DH_BIN_CASE(DH_BOP_EQ) DH_BIN_CASE(DH_BOP_NE) DH_BIN_CASE(DH_BOP_AND)
        DH_BIN_CASE(DH_BOP_OR) DH_BIN_CASE(DH_BOP_ATAN2) DH_BIN_CASE(DH_BOP_POW)
        DH_BIN_CASE(DH_BOP_MIN) DH_BIN_CASE(DH_BOP_MAX)
#undef DH_BIN_CASE
        default:
            return set_error(DH_ERR_INVALID, "dh_binary: unknown op %d", op);
    }
    return check_launch("dh_binary");
}

template <typename T>
int launch_unary(int op, const T* A, T* C, float* C32, size_t n, T lo, T hi) {
    constexpr int NV = V16<T>::N;
    const unsigned g = grid_for((n / NV + EW_UNROLL - 1) / EW_UNROLL);
    switch (op) {
#define DH_UN_CASE(OP)                                                                   \
    case OP:                                                                             \
        unary_kernel<OP, T><<<g, EW_THREADS, 0, stream()>>>(A, C, C32, n, lo, hi);      \
        break;
        DH_UN_CASE(DH_UOP_RELU) DH_UN_CASE(DH_UOP_EXP) DH_UN_CASE(DH_UOP_LOG)
        DH_UN_CASE(DH_UOP_SQRT) DH_UN_CASE(DH_UOP_ABS) DH_UN_CASE(DH_UOP_SIGMOID)
        DH_UN_CASE(DH_UOP_TANH) DH_UN_CASE(DH_UOP_LNOT) DH_UN_CASE(DH_UOP_SIN)
        DH_UN_CASE(DH_UOP_COS) DH_UN_CASE(DH_UOP_TAN) DH_UN_CASE(DH_UOP_ATAN)
        DH_UN_CASE(DH_UOP_FLOOR) DH_UN_CASE(DH_UOP_CEIL) DH_UN_CASE(DH_UOP_ROUND)
        DH_UN_CASE(DH_UOP_CLIP)
#undef DH_UN_CASE
        default:
            return set_error(DH_ERR_INVALID, "dh_unary: unknown op %d", op);
    }
    return check_launch("dh_unary");
}

}  // namespace
}  // namespace dh

using namespace dh;

extern "C" {

int dh_binary(int op, int dtype, const void* d_A, size_t a_len, const int* a_strides,
              const void* d_B, size_t b_len, const int* b_strides, void* d_C, const int* c_dims,
              float* d_C32) {
    DH_TRY(ensure_init());
    if (dtype != DH_F32 && dtype != DH_F64)
        return set_error(DH_ERR_INVALID, "dh_binary: dtype must be DH_F32 or DH_F64");
    if (op < 0 || op >= DH_BOP_COUNT) return set_error(DH_ERR_INVALID, "dh_binary: unknown op %d", op);
    if (!c_dims || !a_strides || !b_strides)
        return set_error(DH_ERR_INVALID, "dh_binary: null dims / strides");
    unsigned long long n = 1;
    for (int k = 0; k < 4; ++k) {
        if (c_dims[k] < 0) return set_error(DH_ERR_INVALID, "dh_binary: negative dim");
        n *= (unsigned long long)c_dims[k];
    }
    if (n == 0) return DH_OK;
    if (n >= (1ull << 31))
        return set_error(DH_ERR_INVALID, "dh_binary: %llu elements (limit 2^31 - 1)", n);
    if (!d_A || !d_B || !d_C) return set_error(DH_ERR_INVALID, "dh_binary: null operand");
    // every read stays inside its operand: the largest offset is sum (dim - 1) * stride
    unsigned long long amax = 0, bmax = 0;
    for (int k = 0; k < 4; ++k) {
        if (a_strides[k] < 0 || b_strides[k] < 0)
            return set_error(DH_ERR_INVALID, "dh_binary: negative stride");
        amax += (unsigned long long)(c_dims[k] - 1) * (unsigned)a_strides[k];
        bmax += (unsigned long long)(c_dims[k] - 1) * (unsigned)b_strides[k];
    }
    if (amax >= (1ull << 32) || bmax >= (1ull << 32))
        return set_error(DH_ERR_INVALID, "dh_binary: operand offsets beyond 2^32 elements");
    if (amax >= a_len || bmax >= b_len)
        return set_error(DH_ERR_INVALID,
                         "dh_binary: strides reach element %llu / %llu of operands of %zu / %zu",
                         amax, bmax, a_len, b_len);
    // collapse: drop size-1 dims, merge a dim into its inner neighbour where both operands
    // are linear across the pair
    int d[4], sa[4], sb[4], nd = 0;
    for (int k = 3; k >= 0; --k) {   // innermost first
        if (c_dims[k] == 1) continue;
        if (nd > 0 && a_strides[k] == sa[nd - 1] * d[nd - 1] &&
            b_strides[k] == sb[nd - 1] * d[nd - 1]) {
            d[nd - 1] *= c_dims[k];
            continue;
        }
        d[nd] = c_dims[k];
        sa[nd] = a_strides[k];
        sb[nd] = b_strides[k];
        ++nd;
    }
    const bool contig = nd == 1 && sa[0] == 1 && sb[0] == 1 && aligned16(d_A) &&
                        aligned16(d_B) && aligned16(d_C) && (!d_C32 || aligned16(d_C32));
    BcastShape sh;
    for (int k = 0; k < 4; ++k) {   // kernel order: outermost first, padded with 1s
        const int src = 3 - k;        // d[0] is the innermost collapsed dim
        const bool have = src < nd;
        sh.div[k] = make_fastdiv(have ? (uint32_t)d[src] : 1u);
        sh.sa[k] = have ? sa[src] : 0;
        sh.sb[k] = have ? sb[src] : 0;
    }
    if (dtype == DH_F32) {
        if (d_C32) return set_error(DH_ERR_INVALID, "dh_binary: C32 side output is for DH_F64");
        return launch_binary<float>(op, (const float*)d_A, (const float*)d_B, (float*)d_C,
                                    nullptr, (size_t)n, contig, sh);
    }
    return launch_binary<double>(op, (const double*)d_A, (const double*)d_B, (double*)d_C, d_C32,
                                 (size_t)n, contig, sh);
}

int dh_unary(int op, int dtype, const void* d_A, void* d_C, size_t n, double lo, double hi,
             float* d_C32) {
    DH_TRY(ensure_init());
    if (dtype != DH_F32 && dtype != DH_F64)
        return set_error(DH_ERR_INVALID, "dh_unary: dtype must be DH_F32 or DH_F64");
    if (op < 0 || op >= DH_UOP_COUNT) return set_error(DH_ERR_INVALID, "dh_unary: unknown op %d", op);
    if (n == 0) return DH_OK;
    if (!d_A || !d_C) return set_error(DH_ERR_INVALID, "dh_unary: null operand");
    if (!aligned16(d_A) || !aligned16(d_C) || (d_C32 && !aligned16(d_C32)))
        return set_error(DH_ERR_INVALID, "dh_unary: operands must be 16-byte aligned");
    if (dtype == DH_F32) {
        if (d_C32) return set_error(DH_ERR_INVALID, "dh_unary: C32 side output is for DH_F64");
        return launch_unary<float>(op, (const float*)d_A, (float*)d_C, nullptr, n, (float)lo,
                                   (float)hi);
    }
    return launch_unary<double>(op, (const double*)d_A, (double*)d_C, d_C32, n, lo, hi);
}

}  // extern "C"
