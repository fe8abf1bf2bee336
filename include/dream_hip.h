/*
 * dream_hip.h -- C ABI of the MI355X (gfx950) backend for Dream's dense-tensor hot path.
 *
 * This library replaces the GPU half of the reference runtime's backend
 * (runtime/backend/gpu.inc: the OpenCL/CUDA/cuBLAS loaders, DeviceMemPool, HostBuf
 * staging and the OpenCL/cuBLAS GEMM and flash kernels).  Plain pointers and sizes
 * only; no C++ or framework types cross this boundary.
 *
 * Conventions
 *  - Every entry point returns an int status: DH_OK (0) or a DH_ERR_* code, with a
 *    human-readable reason from dh_last_error().  Nothing here exits or throws; on
 *    an error the caller decides what to do (the integrated runtime prints
 *    "RUNTIME ERROR in <op>: ..." and keeps going, runtime/ops/elementwise.inc:972-989).
 *  - Pointers named d_* are device pointers (from dh_malloc or any hipMalloc'd
 *    buffer in the same process).  Pointers named h_* are host pointers.
 *  - Matrices are row-major.  Leading dimensions are in elements.
 *  - All work is enqueued on the library stream (dh_get_stream); calls return once
 *    the work is queued, except where "synchronous" is stated.
 *  - bf16 buffers hold the upper 16 bits of an IEEE fp32 value (uint16_t storage).
 *  - Single device: the backend drives device 0 of the process (one process per GPU).
 */
#ifndef DREAM_HIP_H
#define DREAM_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    DH_OK = 0,
    DH_ERR_NO_DEVICE = 1,   /* no usable HIP device / init failed      */
    DH_ERR_INVALID = 2,     /* bad argument (shape, pointer, dtype)     */
    DH_ERR_OOM = 3,         /* device allocation failed                 */
    DH_ERR_HIP = 4,         /* a HIP runtime call or launch failed      */
    DH_ERR_UNSUPPORTED = 5  /* valid request this build does not cover  */
};

enum { DH_F32 = 0, DH_BF16 = 1, DH_F64 = 2 };

/* ---- device / init --------------------------------------------------------
 * Replaces initBackend() (runtime/backend/gpu.inc:313-361): lazy, idempotent, logs
 * "[dream] backend: HIP (device: ...)" once to stderr.  dh_init is also called
 * implicitly by every other entry point. */
int dh_init(void);
/* 1 when a HIP device is usable (the replacement of the OpenCL/CUDA probe,
 * gpu.inc:271-273, for the GEMM and flash builtins). */
int dh_available(void);
/* Device name, compute units, XCDs, max shader clock (MHz), HBM bytes. */
int dh_device_info(char* name, int name_len, int* cus, int* xcds, int* sclk_mhz,
                   long long* hbm_bytes);
const char* dh_last_error(void);

/* ---- dispatch policy (kept from the reference) -----------------------------
 * gpu_dispatch_threshold() (gpu.inc:293-307): 262144 elements of M*N unless env
 * DREAM_GPU_THRESHOLD overrides it.  dh_matmul_eligible: M*N >= threshold
 * (elementwise.inc:1033).  dh_flash_eligible: B*S*S >= 262144 and dk <= 128
 * (runtime/nn/training.inc:308, 336). */
size_t dh_dispatch_threshold(void);
int dh_matmul_eligible(int M, int N);
int dh_flash_eligible(int B, int S, int dk);

/* ---- memory (replaces DeviceMemPool, gpu.inc:372-420) ----------------------
 * Exact-size buckets, at most 64 cached buffers per size; dh_free returns the
 * buffer to its bucket.  dh_pool_release frees every cached buffer. */
void* dh_malloc(size_t bytes);
int dh_free(void* d_ptr);
int dh_pool_release(void);
/* Pinned (page-locked) host buffers for staging tensors, pooled by exact size (at most 16 per
 * size); copies to and from them run at full PCIe rate and are truly asynchronous -- a caller
 * must not modify a buffer that a queued H2D copy still reads (dh_sync first).  dh_host_free
 * drains the stream before the buffer can be reused; dh_pool_release frees the cached ones.
 * dh_host_alloc returns NULL (with dh_last_error) when pinning fails. */
void* dh_host_alloc(size_t bytes);
int dh_host_free(void* h_ptr);
int dh_memcpy_h2d(void* d_dst, const void* h_src, size_t bytes);
int dh_memcpy_d2h(void* h_dst, const void* d_src, size_t bytes);   /* returns when the data is home */
/* D2H copy queued on the stream without waiting (HostBuf's download, gpu.inc:177-196, made
 * asynchronous): the data is home after the next dh_sync.  Several of them into one pinned
 * buffer cost one wait instead of one each. */
int dh_memcpy_d2h_async(void* h_dst, const void* d_src, size_t bytes);
int dh_memcpy_d2d(void* d_dst, const void* d_src, size_t bytes);
int dh_memset(void* d_dst, int value, size_t bytes);
int dh_sync(void);                         /* synchronous: waits for the stream */
void* dh_get_stream(void);                 /* hipStream_t of the library        */
int dh_set_stream(void* hip_stream);       /* NULL restores the library stream  */

/* ---- timing on the library stream ----------------------------------------- */
int dh_timer_start(void);
int dh_timer_stop(float* ms);              /* synchronous */
/* Events on the library stream, so a host thread can wait for part of the queued work (one
 * copy of several) instead of all of it: the copies home of a backward overlap the host's
 * widening of the ones already landed. */
void* dh_event_create(void);               /* NULL on failure (dh_last_error) */
int dh_event_record(void* event);          /* marks the work queued so far */
int dh_event_wait(void* event);            /* host waits until that work is done */
int dh_event_destroy(void* event);

/* ---- conversions (replaces HostBuf fromDouble/toDouble, gpu.inc:177-196) ----
 * dst[i] = convert(src[i]) for n elements.  Supported pairs: F64->F32, F32->F64,
 * F64->BF16 (through fp32, then round to nearest even exactly as
 * dream_to_bf16, runtime/nn/training.inc:1969-1976), F32->BF16, BF16->F32, and F32->F32
 * (a plain device copy). */
int dh_convert(void* d_dst, int dst_type, const void* d_src, int src_type, size_t n);
/* y[i] += alpha * x[i] for n fp32 values: merges gradient contributions on the device (the
 * reference's host "+=" accumulation of a node's gradient, runtime/ops/autograd.inc:26-887). */
int dh_axpy(float* d_y, const float* d_x, float alpha, size_t n);

/* ---- GEMM -------------------------------------------------------------------
 * C[M x N] = op(A) @ op(B) + beta * C, fp32 accumulate, fp32 C.
 * op(X) = X (trans = 0) or X^T (trans = 1) of the stored row-major matrix:
 *   transA = 0: A is M x K (lda >= K);  transA = 1: A is stored K x M (lda >= M)
 *   transB = 0: B is K x N (ldb >= N);  transB = 1: B is stored N x K (ldb >= K)
 * NN is tensor_matmul's C = A @ B (elementwise.inc:971-1213, replacing the
 * OpenCL matmul_tiled_wpt4 kernel and the cublasSgemm/GemmEx branch 1042-1212);
 * NT with beta = 1 is the matmul backward's dA += dY @ B^T and TN with beta = 1
 * its dB += A^T @ dY (runtime/ops/autograd.inc:91-125).
 * beta = 0 never reads C.  M, N or K of 0 is a valid no-op (K = 0 scales C by beta). */
int dh_gemm_f32(int transA, int transB, int M, int N, int K,
                const float* d_A, int lda, const float* d_B, int ldb,
                float beta, float* d_C, int ldc);
/* Same contract with bf16 A and B (replaces the fp16 cublasGemmEx path,
 * elementwise.inc:1046-1071; inputs are bf16 rather than truncated fp16). */
int dh_gemm_bf16(int transA, int transB, int M, int N, int K,
                 const uint16_t* d_A, int lda, const uint16_t* d_B, int ldb,
                 float beta, float* d_C, int ldc);
/* Batched GEMM with a fused epilogue, for every member b < batch:
 *   C_b = op(A_b) @ op(B_b) + beta * C_b + bias,  then C_b = max(C_b, 0) with DH_EPI_RELU
 * with X_b = d_X + b * strideX (strides in elements; a zero stride for A or B shares one
 * operand across the batch; C members must not overlap: strideC >= (M-1)*ldc + N when
 * batch > 1).  bias (fp32, may be NULL) holds N values added to every row, or with
 * DH_EPI_ROW_BIAS M values added to every column; NaN passes the ReLU as in the reference's
 * `y < 0 ? 0 : y`.
 * NT with a column bias (+ relu) is dream_linear / linear_relu's Y = X W^T + b with W stored
 * out x in (runtime/ops/elementwise.inc:1432-1516); batched NN is dream_bmm
 * (elementwise.inc:1218-1252), and its backward's G B^T and A^T G are batched NT and TN
 * with beta = 1 (runtime/ops/autograd.inc:549-574); NN with a row bias per image is
 * dream_conv2d's kernel @ im2col + bias (runtime/nn/conv.inc:12-55).  dh_gemm_f32 /
 * dh_gemm_bf16 are the batch = 1, bias = NULL, epilogue = 0 case.  The fp32 form splits a
 * skinny product's long K over idle CUs by itself (deterministic ordered reduction). */
enum { DH_EPI_RELU = 1, DH_EPI_ROW_BIAS = 2 };
int dh_gemm_f32_ex(int transA, int transB, int M, int N, int K,
                   const float* d_A, int lda, long long strideA,
                   const float* d_B, int ldb, long long strideB,
                   float beta, float* d_C, int ldc, long long strideC,
                   int batch, const float* d_bias, int epilogue);
int dh_gemm_bf16_ex(int transA, int transB, int M, int N, int K,
                    const uint16_t* d_A, int lda, long long strideA,
                    const uint16_t* d_B, int ldb, long long strideB,
                    float beta, float* d_C, int ldc, long long strideC,
                    int batch, const float* d_bias, int epilogue);

/* ---- fp64 (the reference's double-precision results) ---------------------------
 * C[M x N] = alpha * (op(A) @ op(B)) + beta * C in fp64, same op / leading-dimension rules
 * as dh_gemm_f32.  Replaces dream_gemm_d (runtime/ops/elementwise.inc:593-638), which the
 * reference's `@` runs when M*N is below the dispatch threshold (elementwise.inc:1033-1040):
 * every element is summed in the reference's order -- per 256-deep block of k (its KC) one
 * fused multiply-add chain in k order started from zero, the blocks' sums added in k order
 * -- so NN with alpha = 1, beta = 0 is bit-identical to the reference's fp64 `@`.  NT / TN
 * with beta = 1 are the fp64 matmul backward (autograd.inc:91-125).  beta = 0 never reads C.
 * _ex: batched, X_b = d_X + b * strideX (elements; zero shares an operand), batch <= 65535,
 * C members must not overlap. */
int dh_gemm_f64(int transA, int transB, int M, int N, int K,
                const double* d_A, int lda, const double* d_B, int ldb,
                double beta, double* d_C, int ldc);
int dh_gemm_f64_ex(int transA, int transB, int M, int N, int K, double alpha,
                   const double* d_A, int lda, long long strideA,
                   const double* d_B, int ldb, long long strideB,
                   double beta, double* d_C, int ldc, long long strideC, int batch);
/* fp64 scaled dot-product attention in the reference layout (B, S*D), any head dim D:
 * O = softmax(scale * Q K^T, causal mask j <= i when causal) V per slice -- the reference's
 * dream_attention / dream_attention_causal (runtime/nn/training.inc:178-263), which it always
 * computes in fp64, and its flash_attention outside B*S*S >= 262144 && dk <= 128 (the fp64
 * loop of training.inc:366-399; same values up to rounding).  The backward
 * (autograd.inc:675-778) recomputes the probabilities and adds (accumulate = 1) or writes
 * dQ, dK, dV; any two of them may be one buffer, which then receives the sum of its
 * gradients.  Score buffers come from the pool, at most 256 MB each: whole S x S blocks
 * by chunks of slices while one slice fits, else blocks of query rows of one slice
 * (rows x S); the backward takes two.  S <= 46340.  scale must be positive. */
int dh_attention_f64_fwd(int BH, int S, int D, double scale, int causal,
                         const double* d_Q, const double* d_K, const double* d_V, double* d_O);
int dh_attention_f64_bwd(int BH, int S, int D, double scale, int causal,
                         const double* d_Q, const double* d_K, const double* d_V,
                         const double* d_dO, double* d_dQ, double* d_dK, double* d_dV,
                         int accumulate);

/* ---- FlashAttention -----------------------------------------------------------
 * Q, K, V, O in the reference layout (B, S*dk): slice b (a batch x head pair)
 * starts at b*S*D, rows of D contiguous.  dtype DH_F32 or DH_BF16 for Q/K/V/dO;
 * O is written in the same dtype; LSE (fp32, B*S) receives m_i + ln(l_i) of the
 * scaled scores (natural log).  Causal keeps key j <= query i
 * (runtime/nn/training.inc:284-401, which replaces the OpenCL flash_attention_v1
 * kernel 310-363).  D in {32, 64, 128} (callers zero-pad other head dims: zero columns
 * of Q and K leave Q K^T unchanged and zero columns of V give zero columns of O).
 * scale is usually 1/sqrt(dk) of the unpadded head dim (the reference always passes
 * that, training.inc:292); it must be finite and > 0, else DH_ERR_INVALID. */
int dh_flash_fwd(int dtype, int BH, int S, int D, float scale, int causal,
                 const void* d_Q, const void* d_K, const void* d_V,
                 void* d_O, float* d_LSE);
/* Backward of dh_flash_fwd given its O and LSE (runtime/ops/autograd.inc:779-840).
 * dQ, dK, dV are fp32 (B, S*D).  accumulate = 1 adds into them (the reference
 * backward's "+="), 0 overwrites.  Any two of dQ, dK, dV may be the same buffer (one
 * tensor passed as several of Q, K, V): that buffer then receives the sum of the
 * gradients aimed at it, as the reference's per-input "+=" leaves it
 * (autograd.inc:693-728); buffers that overlap without being equal are DH_ERR_INVALID.
 * Deterministic: no floating-point atomics.  Scratch (BH*S floats, twice that for bf16)
 * comes from the pool. */
int dh_flash_bwd(int dtype, int BH, int S, int D, float scale, int causal,
                 const void* d_Q, const void* d_K, const void* d_V,
                 const void* d_O, const void* d_dO, const float* d_LSE,
                 float* d_dQ, float* d_dK, float* d_dV, int accumulate);
/* dh_flash_bwd without any allocation.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops, harnesses
 * that forbid hipMalloc).  Same arguments and errors as dh_flash_bwd, and the same results bit
 * for bit, except fp32 at D = 64 or 128 with BH*ceil(S/128) at least the GPU's CU count, where
 * dh_flash_bwd forms dQ from a stored dS in pool memory and this one recomputes it (equal to
 * fp32 rounding); the scratch is a fixed 8 MB device array per GPU (held until the process ends), so BH*S must be at most
 * 1048576 rows, else DH_ERR_INVALID.  Every call on one GPU shares that array: calls that
 * overlap in time on one GPU (other host threads, or another stream set with dh_set_stream)
 * race; calls ordered on one stream do not. */
int dh_flash_bwd_noalloc(int dtype, int BH, int S, int D, float scale, int causal,
                         const void* d_Q, const void* d_K, const void* d_V,
                         const void* d_O, const void* d_dO, const float* d_LSE,
                         float* d_dQ, float* d_dK, float* d_dV, int accumulate);

/* ---- row-wise ops: fp32, R rows of C contiguous values -------------------------
 * accumulate = 1 adds into GX (the reference backward's "+="), 0 overwrites it.
 * Y = softmax or log_softmax of every row (dream_softmax, elementwise.inc:338-358;
 * dream_log_softmax, elementwise.inc:1550-1570). */
int dh_row_softmax(const float* d_X, float* d_Y, int R, int C, int log_softmax);
/* Their backward from the forward OUTPUT Y: softmax GX (+)= Y (G - rowsum(G Y))
 * (autograd.inc:396-409); log_softmax GX (+)= G - exp(Y) rowsum(G), exp(Y) being the softmax
 * the reference recomputes from its input (autograd.inc:212-233). */
int dh_row_softmax_bwd(const float* d_Y, const float* d_G, float* d_GX, int R, int C,
                       int log_softmax, int accumulate);
/* Row layer norm without affine terms: Y = (X - mean) / sqrt(var + 1e-5), biased variance
 * (dream_layer_norm, runtime/io/builtins.inc:167-188). */
int dh_layer_norm(const float* d_X, float* d_Y, int R, int C);
/* Its backward, inv_std recomputed from X (autograd.inc:453-471):
 * GX (+)= inv_std / C (C DY - rowsum(DY) - Y rowsum(DY Y)). */
int dh_layer_norm_bwd(const float* d_X, const float* d_Y, const float* d_DY, float* d_GX,
                      int R, int C, int accumulate);
/* Bias gradient of a linear layer Y (N x out): db (+)= column sums of dY.  With relu != 0
 * dY is first zeroed where Y <= 0, in place -- the linear_relu backward, which masks the
 * node's own gradient the same way (runtime/ops/autograd.inc:156-183).  Deterministic (no
 * floating-point atomics).  Y may be NULL when relu == 0. */
int dh_linear_bias_grad(const float* d_Y, float* d_dY, float* d_db, int N, int out, int relu,
                        int accumulate);

/* ---- conv2d data movement (runtime/nn/conv.inc:12-55, 119-178; im2col.inc:2-25;
 *      autograd.inc:507-535) ------------------------------------------------------------
 * Input X is (N, Cin, H, W) fp32; OH = (H + 2 pad - KH) / stride + 1, likewise OW.
 * dh_im2col writes col, (Cin*KH*KW) x (N*OH*OW): row (ci*KH + kh)*KW + kw, column
 * n*OH*OW + oh*OW + ow, zero where the window covers padding.  With it the forward is one
 * dh_gemm_f32_ex (kernel @ col per image, the kernel shared by a zero stride, the per-channel
 * bias as DH_EPI_ROW_BIAS).  dh_col2im is its adjoint: dX (+)= the sum, for every input
 * element, of the dcol entries that read it (a gather in a fixed order: deterministic).
 * dh_nct_to_cnt permutes (N, C, T) to (C, N*T), the channel-first output gradient both
 * backward products take. */
int dh_im2col(const float* d_X, float* d_col, int N, int Cin, int H, int W, int KH, int KW,
              int pad, int stride);
int dh_col2im(const float* d_dcol, float* d_dX, int N, int Cin, int H, int W, int KH, int KW,
              int pad, int stride, int accumulate);
int dh_nct_to_cnt(const float* d_src, float* d_dst, int N, int C, size_t T);
/* The forward in one launch, as an implicit GEMM: Y (N, Cout, OH*OW) = kernel (Cout x
 * Cin*KH*KW) @ col_n + bias[co] per image, the im2col matrix gathered inside the GEMM's operand
 * loader and never stored (dream_conv2d / dream_conv2d_padded, conv.inc:12-55, 119-178).
 * bias may be NULL; otherwise it holds Cout values. */
int dh_conv2d_fwd(const float* d_X, const float* d_kernel, const float* d_bias, float* d_Y,
                  int N, int Cin, int H, int W, int Cout, int KH, int KW, int pad, int stride);
/* The input gradient of a stride-1 convolution in one implicit-GEMM launch (after a small
 * kernel-flip launch): dX (N, Cin*H*W) (+)= col2im(kernel^T dY) per image, the dX half of the
 * conv node's backward (autograd.inc:507-535, the cpu_gemm of conv.inc:175), computed as the
 * convolution of dY (N, Cout, OH*OW) with the flipped, channel-swapped kernel padded by
 * KH-1-pad / KW-1-pad.  accumulate = 1 adds into dX.  Stride > 1 or pad > KH-1 / KW-1 is
 * DH_ERR_UNSUPPORTED: those take dh_gemm_f32 + dh_col2im. */
int dh_conv2d_bwd_data(const float* d_dY, const float* d_kernel, float* d_dX, int N, int Cin,
                       int H, int W, int Cout, int KH, int KW, int pad, int stride,
                       int accumulate);
/* The kernel gradient of a convolution (any pad and stride): dK (Cout x Cin*KH*KW) (+)= sum
 * over images of dY_n (Cout x OH*OW) col_n^T, the gK half of the conv node's backward
 * (autograd.inc:507-535), as an implicit GEMM: col_n is gathered from X inside the operand
 * loader and dY is read in its (N, Cout, OH*OW) layout (no im2col matrix, no channel-first
 * copy).  The (image, position) contraction is split over work-groups and the fp32 partials
 * (at most 256 MB of pool memory) are summed in a fixed order: reruns are bit-identical.
 * accumulate = 1 adds into dK. */
int dh_conv2d_bwd_filter(const float* d_dY, const float* d_X, float* d_dK, int N, int Cin,
                         int H, int W, int Cout, int KH, int KW, int pad, int stride,
                         int accumulate);

/* ---- elementwise ops (runGPU / runGPUUnary, runtime/backend/gpu.inc:637-716) ---------------
 * Op codes follow the reference's BinopCode / UnopCode (gpu.inc:455-460, 571-577); each
 * computes, in the operand type, what the reference's CPU loop (runCPUBinary / runCPUUnary,
 * gpu.inc:484-598) computes in fp64: eq / ne compare |a - b| against 1e-6, and / or test
 * a > 0, b > 0, min / max pick a on ties of the other test, clip is fmax(lo, fmin(hi, a))
 * (the OpenCL expression of dream_clip, elementwise.inc:329-336). */
enum {
    DH_BOP_ADD = 0, DH_BOP_SUB, DH_BOP_MUL, DH_BOP_DIV, DH_BOP_MOD,
    DH_BOP_GT, DH_BOP_LT, DH_BOP_GE, DH_BOP_LE, DH_BOP_EQ, DH_BOP_NE,
    DH_BOP_AND, DH_BOP_OR, DH_BOP_ATAN2, DH_BOP_POW, DH_BOP_MIN, DH_BOP_MAX, DH_BOP_COUNT
};
enum {
    DH_UOP_RELU = 0, DH_UOP_EXP, DH_UOP_LOG, DH_UOP_SQRT, DH_UOP_ABS,
    DH_UOP_SIGMOID, DH_UOP_TANH, DH_UOP_LNOT,
    DH_UOP_SIN, DH_UOP_COS, DH_UOP_TAN, DH_UOP_ATAN,
    DH_UOP_FLOOR, DH_UOP_CEIL, DH_UOP_ROUND, DH_UOP_CLIP, DH_UOP_COUNT
};
/* C[i] = op(A[ia], B[ib]) over C's dims c_dims[0..3] (d0 outermost, row-major), where i's
 * indices (i0, i1, i2, i3) give ia = sum ik * a_strides[k] (element strides, 0 on a broadcast
 * dim: the bcastStrides rule, gpu.inc:443-449) and likewise ib.  dtype DH_F32 or DH_F64 for
 * A, B, C.  a_len / b_len are the operands' element counts: a stride pattern that would read
 * past them is DH_ERR_INVALID.  C holds at most 2^31 - 1 elements.  d_C32, DH_F64 only and
 * may be NULL: also receives C rounded to fp32 (the device copy of the result for fp32
 * consumers). */
int dh_binary(int op, int dtype, const void* d_A, size_t a_len, const int* a_strides,
              const void* d_B, size_t b_len, const int* b_strides, void* d_C, const int* c_dims,
              float* d_C32);
/* C[i] = op(A[i]) for n contiguous values; lo / hi are clip's bounds (ignored otherwise).
 * Pointers 16-byte aligned (every dh_malloc block is).  d_C32 as for dh_binary. */
int dh_unary(int op, int dtype, const void* d_A, void* d_C, size_t n, double lo, double hi,
             float* d_C32);

#ifdef __cplusplus
}
#endif
#endif
