/*
 * dream_rt.h -- Dream runtime builtins of the dense-tensor hot path, over the HIP backend.
 *
 * Same names, argument meaning, ownership and error behaviour as the reference runtime's
 * builtins (runtime/runtime.h, runtime/ops/elementwise.inc, runtime/ops/autograd.inc,
 * runtime/nn/training.inc), so compiled .dream programs and C callers bind unchanged:
 *   - every Tensor* returned is a +1 reference owned by the caller; arguments are never
 *     stolen (interop/dream.h:13-16);
 *   - errors print "RUNTIME ERROR in <op>: ..." to stderr and return a fresh 1x1 tensor
 *     (runtime/ops/elementwise.inc:972-989); nothing exits.
 * The GEMM and attention builtins compute on the GPU through include/dream_hip.h, in fp64
 * where the reference's dispatch computes fp64; this runtime has no CPU GEMM or CPU
 * attention.  Host-side builtins kept only to build
 * programs around the hot path (ones, randn, sum, tensor_mul, ...) run on the host, as
 * the reference's own elementwise ops do.
 *
 * Tensor: fields 0-6 (data, grad, size, d0..d3) are the layout generated code reads
 * (runtime/runtime.h:49-55); all later fields belong to this runtime.
 */
#ifndef DREAM_RT_H
#define DREAM_RT_H

#ifdef __cplusplus
extern "C" {
#endif

typedef struct Tensor {
    /* ---- IR-visible, fixed order (runtime/runtime.h:49-55) ---- */
    double* data;
    double* grad;
    int size;
    int d0, d1, d2, d3;
    /* ---- runtime-only ---- */
    int refcount;
    int is_leaf;
    int op;                    /* graph node kind (DREAM_OP_*)                     */
    struct Tensor* lhs;
    struct Tensor* rhs;
    struct Tensor* parents[3];
    int num_parents;
    int attn_B, attn_S, attn_dk;   /* "B,S,dk" of an attention node (bwd_name)    */
    int bmm_B, bmm_M, bmm_K, bmm_N;   /* "B,M,K,N" of a bmm node (bwd_name)       */
    int conv[8];               /* H, W, KH, KW, Cin, Cout, pad, stride of a conv2d node */
    int dtype;                 /* 0 = fp64 storage, 1 = live fp32 mirror (as f32)  */
    float* fdata;              /* fp32 mirror when dtype == 1                      */
    float* fgrad;
    /* Device residency.  `data` is always current (generated code reads it directly,
     * src/AST.cpp:160-172, 862-870), so results are copied home before a builtin returns;
     * `dev` is a device fp32 copy of `data` that later GPU ops reuse instead of uploading
     * again.  It is valid while dev_version == version: every in-place mutation of `data`
     * increments `version` (the reference's own mutation counter, runtime/runtime.h:76,
     * bumped by its mutating builtins, runtime/io/builtins.inc:295-445). */
    int version;
    float* dev;                /* device fp32 copy of data, or NULL                */
    int dev_version;
    float* dgrad;              /* device fp32 gradient during backward(), or NULL  */
    int grad_zero;             /* 1 while every host grad value is known to be 0   */
    float* dlse;               /* attention nodes: device per-row log-sum-exp (B*S) */
    int host_pinned;           /* bit 0: data, bit 1: grad are pinned pool buffers   */
    int f64_node;              /* 1: the node's forward ran in fp64 (below the GPU
                                * threshold), so its backward does too               */
    double keep;               /* dropout nodes: the keep rate (bwd_name)            */
    int dev_exact;             /* 1: data is exactly the widened `dev` (a GPU result), so
                                * the fp64 values can be rebuilt on the device from it  */
    double* dev64;             /* device fp64 copy of data (elementwise operands), or NULL */
    int dev64_version;
} Tensor;

enum {
    DREAM_OP_LEAF = 0, DREAM_OP_MATMUL, DREAM_OP_FLASH, DREAM_OP_ATTN, DREAM_OP_ATTN_CAUSAL,
    DREAM_OP_SUM, DREAM_OP_MUL, DREAM_OP_ADD, DREAM_OP_LINEAR, DREAM_OP_LINEAR_RELU,
    DREAM_OP_BMM, DREAM_OP_SOFTMAX, DREAM_OP_LOG_SOFTMAX, DREAM_OP_LAYER_NORM, DREAM_OP_CONV2D,
    /* elementwise nodes with a backward branch (autograd.inc:58-90, 284-288, 342-378,
     * 491-506), and the elementwise nodes without one (comparisons, mod, and/or, atan2,
     * logical not, floor/ceil/round, clip) */
    DREAM_OP_SUB, DREAM_OP_DIV, DREAM_OP_MINIMUM, DREAM_OP_MAXIMUM, DREAM_OP_POW,
    DREAM_OP_RELU, DREAM_OP_EXP, DREAM_OP_LOG, DREAM_OP_SQRT, DREAM_OP_ABS, DREAM_OP_SIGMOID,
    DREAM_OP_TANH, DREAM_OP_SIN, DREAM_OP_COS, DREAM_OP_TAN, DREAM_OP_ATAN, DREAM_OP_NO_GRAD,
    DREAM_OP_DROPOUT
};

/* ---- tensors (runtime/core/tensor.inc:143-303) ---- */
Tensor* alloc_tensor(int d0, int d1, int d2, int d3);
Tensor* create_scalar(double v);
Tensor* tensor_incref(Tensor* t);
Tensor* tensor_decref(Tensor* t);
Tensor* ones(Tensor* d0, Tensor* d1);                      /* elementwise.inc:2     */
Tensor* dream_set_seed(Tensor* seed);                      /* elementwise.inc:35-40 */
Tensor* dream_randn(Tensor* d0, Tensor* d1);               /* elementwise.inc:48-54 */
Tensor* sum(Tensor* a);                                    /* elementwise.inc:56    */
Tensor* dream_dropout(Tensor* t, Tensor* keep_rate);       /* builtins.inc:151-163  */
/* ---- elementwise ops (elementwise.inc:276-336, 1254-1270; math_extra.inc:1-10;
 * builtins.inc:85-87), the reference's runGPU / runGPUUnary path (backend/gpu.inc:637-716).
 * Binary: C's dims are the per-dim maxima of the operands', each operand read through
 * bcastStrides (its own contiguous strides, 0 on a dim of 1); operands that do not broadcast
 * (which the reference reads out of bounds after a warning) are an error.  Outputs of at
 * most 4194304 elements are computed on the host, larger ones on the GPU in fp64
 * (DREAM_ELEMWISE_CPU_MAX overrides the bound).  The error text names the operator symbol
 * ('+', '-', '*', '/', '%', '>', ..., 'min', 'max', 'atan2', '**') or the unary op. */
Tensor* tensor_add(Tensor* a, Tensor* b);
Tensor* tensor_sub(Tensor* a, Tensor* b);
Tensor* tensor_mul(Tensor* a, Tensor* b);
Tensor* tensor_div(Tensor* a, Tensor* b);
Tensor* tensor_mod(Tensor* a, Tensor* b);
Tensor* tensor_gt(Tensor* a, Tensor* b);
Tensor* tensor_lt(Tensor* a, Tensor* b);
Tensor* tensor_ge(Tensor* a, Tensor* b);
Tensor* tensor_le(Tensor* a, Tensor* b);
Tensor* tensor_eq(Tensor* a, Tensor* b);
Tensor* tensor_ne(Tensor* a, Tensor* b);
Tensor* tensor_and(Tensor* a, Tensor* b);
Tensor* tensor_or(Tensor* a, Tensor* b);
Tensor* dream_minimum(Tensor* a, Tensor* b);
Tensor* dream_maximum(Tensor* a, Tensor* b);
Tensor* dream_atan2(Tensor* y, Tensor* x);
Tensor* dream_pow(Tensor* base, Tensor* exp_t);            /* C is (max d0, max d1) */
Tensor* relu(Tensor* a);
Tensor* dream_exp(Tensor* a);
Tensor* dream_log(Tensor* a);
Tensor* dream_sqrt(Tensor* a);
Tensor* dream_abs(Tensor* a);
Tensor* dream_sigmoid(Tensor* a);
Tensor* dream_tanh(Tensor* a);
Tensor* dream_logical_not(Tensor* a);
Tensor* dream_sin(Tensor* a);
Tensor* dream_cos(Tensor* a);
Tensor* dream_tan(Tensor* a);
Tensor* dream_atan(Tensor* a);
Tensor* dream_floor(Tensor* a);
Tensor* dream_ceil(Tensor* a);
Tensor* dream_round(Tensor* a);
/* fmax(lo, fmin(hi, a)) with lo, hi the bounds' first values: the OpenCL expression of the
 * reference (elementwise.inc:329-336), whose CPU interpreter has no form of it. */
Tensor* dream_clip(Tensor* a, Tensor* lo, Tensor* hi);
Tensor* tensor_get_grad(Tensor* t);                        /* autograd.inc:1-14     */
Tensor* zero_grad(Tensor* t);                              /* autograd.inc:15-24    */
/* t[i] = v and t[i][j] = v (runtime/io/builtins.inc:286-317): the in-place writes of
 * generated code (src/AST.cpp:1702-1740); they bump `version`. */
Tensor* tensor_set_element(Tensor* t, Tensor* idx, Tensor* v);
Tensor* tensor_set_element_2d(Tensor* t, Tensor* i, Tensor* j, Tensor* v);

/* ---- precision (runtime/io/builtins.inc:1168-1184, 380-394, 465-475) ---- */
Tensor* dream_set_precision(Tensor* t, int code);          /* `as f32` (1) / `as f64` (0) */
Tensor* dream_to_float32(Tensor* t);
Tensor* dream_enable_fp16(void);   /* reduced-precision `@`: bf16 operands, fp32 accumulate */
Tensor* dream_disable_fp16(void);

/* ---- the hot path ---- */
/* C = A @ B (runtime/ops/elementwise.inc:971-1213), graph node "matmul", with the
 * reference's dispatch (elementwise.inc:1000-1040): both operands `as f32` -> fp32 GEMM;
 * else M*N below the dispatch threshold (DREAM_GPU_THRESHOLD, default 262144) -> fp64 GEMM,
 * bit-identical to the reference's dream_gemm_d; else the fp32 (bf16 after
 * dream_enable_fp16) matrix-core GEMM, the reference's GPU branch.  All three run on the GPU;
 * the node's backward runs in the precision of its forward. */
Tensor* tensor_matmul(Tensor* a, Tensor* b);
/* Causal FlashAttention (runtime/nn/training.inc:284-401); block_t may be NULL.  The
 * reference's GPU rule B*S*S >= 262144 && dk <= 128 (training.inc:308, 336) selects the fp32
 * (bf16) FlashAttention kernels; any other shape -- every dk > 128 included -- is computed in
 * fp64, as the reference's CPU loop computes it. */
Tensor* dream_flash_attention(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq,
                              Tensor* dk, Tensor* block);
/* Standard attention, non-causal and causal (training.inc:178-263).  The reference computes
 * it in fp64 for every shape; here shapes under the flash rule above run on the FlashAttention
 * kernels (no S x S scores), every other shape in fp64. */
Tensor* dream_attention(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq, Tensor* dk);
Tensor* dream_attention_causal(Tensor* Q, Tensor* K, Tensor* V, Tensor* batch, Tensor* seq,
                               Tensor* dk);
/* The other GEMM callers and the row-wise ops, on the GPU with their backward:
 *   Y = x W^T + b, W stored out x in; linear_relu clamps Y < 0 to 0 (one GEMM with a fused
 *   bias / ReLU epilogue; runtime/ops/elementwise.inc:1432-1516, autograd.inc:156-205);
 *   batched C[b] = A[b] B[b] with A (B, M*K), B (B, K*N), scalars as 1x1 tensors
 *   (elementwise.inc:1218-1252, autograd.inc:549-574);
 *   row softmax over d0 rows (elementwise.inc:338-358, autograd.inc:396-409), log_softmax over
 *   d0 x d1 (elementwise.inc:1550-1570, autograd.inc:212-233), row layer norm without affine
 *   terms, eps 1e-5 (runtime/io/builtins.inc:167-188, autograd.inc:453-471). */
Tensor* dream_linear(Tensor* x, Tensor* W, Tensor* b);
Tensor* dream_linear_relu(Tensor* x, Tensor* W, Tensor* b);
Tensor* linear(Tensor* x, Tensor* W, Tensor* b);          /* aliases, elementwise.inc:1520 */
Tensor* linear_relu(Tensor* x, Tensor* W, Tensor* b);
Tensor* dream_bmm(Tensor* a, Tensor* b, Tensor* batch, Tensor* m, Tensor* k, Tensor* n);
Tensor* dream_softmax(Tensor* a);
Tensor* dream_log_softmax(Tensor* x);
Tensor* dream_layer_norm(Tensor* t);
/* 2-D convolution of input (N, Cin*H*W) with kernel (Cout, Cin*KH*KW) plus a per-channel bias
 * (may be NULL) -> (N, Cout*OH*OW), scalars as 1x1 tensors: valid (runtime/nn/conv.inc:12-55)
 * and zero-padded / strided (conv.inc:119-178).  Implicit-GEMM kernels; backward dX, dK
 * (autograd.inc:507-535; the reference computes no bias gradient, and neither does this).
 * Divergence from the reference, on purpose: the reference's padded / strided node reuses the
 * valid-convolution backward (autograd.inc:507-535 reads H, W, KH, KW only), which is correct
 * for pad 0 and stride 1 alone; for pad > 0 or stride > 1 this backward computes the exact
 * gradient of the padded / strided forward instead (pinned by finite differences), so dX and
 * dK differ from the reference's values on the same inputs for those shapes. */
Tensor* dream_conv2d(Tensor* input, Tensor* kernel, Tensor* bias, Tensor* h, Tensor* w,
                     Tensor* kh, Tensor* kw);
Tensor* dream_conv2d_padded(Tensor* input, Tensor* kernel, Tensor* bias, Tensor* h, Tensor* w,
                            Tensor* kh, Tensor* kw, Tensor* pad, Tensor* stride);
/* Reverse sweep from root (runtime/ops/autograd.inc:26-887) for the node kinds above;
 * gradients accumulate ("+=") into grad buffers like the reference.  Between two GPU ops a
 * gradient stays on the device; every grad buffer is current on the host when it returns. */
Tensor* backward(Tensor* root);

/* ---- backend queries, selftests (runtime/backend/gpu.inc:271-273,
 *      runtime/ops/elementwise.inc:759-875, runtime/nn/training.inc:405-435) ---- */
/* 0: the OpenCL fused-expression path does not exist, so generated code keeps fused
 * elementwise expressions on its CPU branch (src/AST.cpp:1053-1076). */
int dream_gpu_available(void);
/* 1 when the HIP backend can run the GEMM and attention builtins. */
int dream_hip_available(void);
/* gemm_selftest (elementwise.inc:888-968): the reference's 17 shapes, seed and draws; the 11
 * fp64 shapes through the fp64 GEMM (dh_gemm_f64, what `@` runs below the threshold) against
 * the naive fp64 product under the reference's gate (max relative error < 1e-11), the 6 f32
 * shapes through the fp32 GEMM under its 2e-4; prints "GEMM: 17/17 PASS" like the
 * reference. */
Tensor* gemm_selftest(void);
/* bf16_selftest (runtime/nn/training.inc:1978-2025): bf16 range and precision through the
 * device rounding (dh_convert), and the mixed-precision convergence check; prints
 * "BF16_MIXED: 3/3 PASS" like the reference. */
Tensor* bf16_selftest(void);
Tensor* gpu_selftest(void);
Tensor* dream_gpu_warmup(void);
/* flash_attention_selftest (training.inc:405-435): the reference's four configurations and
 * seed; flash_attention (fp64 at these sizes) against the naive fp64 causal attention under
 * the reference's gate (max relative error < 1e-9). */
Tensor* flash_attention_selftest(void);

#ifdef __cplusplus
}
#endif
#endif
