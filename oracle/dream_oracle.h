/*
 * dream_oracle.h -- CPU restatement of the Dream reference hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Nothing in the product (dreamcompiler_amd/, include/)
 * links, loads or calls this library.  Only tests/, __graft_entry__.smoke() and
 * bench.py's cpu_baseline leg may use it, and only as the checker / the timed
 * CPU comparison, never as the thing measured on the GPU.
 *
 * Every function restates one reference function (file:line into
 * heellowdsf/DreamCompiler).  All matrices are row-major and contiguous.
 * Functions documented as "+=" accumulate into the output buffers exactly
 * like the reference backward branches do.
 *
 * Pinning status (what checks each function, see tests/test_oracle.py):
 *   orc_set_seed/orc_randn/orc_kaiming   golden vectors from the reference build
 *   orc_uniform(_f32)   bit-exact vs an independent mt19937 stream through libstdc++'s
 *                       generate_canonical; range and moments
 *   orc_gemm_ref_d      closed forms (all-ones -> K), identity, brute-force fp64 sums via numpy
 *   orc_gemm_d          golden vectors + gemm_ref_d (1e-11, the reference gate)
 *   orc_gemm_f32        golden vectors + fp64 on the same fp32 inputs (2e-4, the reference gate)
 *   orc_gemm_general_d  numpy fp64 einsum on random transposes / beta (independent code)
 *   orc_matmul_bwd      golden vectors (reference backward) + finite differences
 *   orc_attention*, orc_flash_fwd, orc_flash_bwd      golden vectors + special cases
 *                       (S=1 -> O=V, constant K -> causal running mean) + finite differences
 *   orc_flash_lse       closed form log-sum-exp (scipy.special.logsumexp)
 *   orc_attention_rows  the rows of orc_attention(_causal) / orc_attention_bwd's dQ
 *   orc_softmax_rows, orc_log_softmax_rows   golden vectors, scipy softmax / log_softmax, rows sum to 1
 *   orc_softmax_bwd, orc_log_softmax_bwd, orc_layer_norm(_bwd)   golden vectors + finite
 *                       differences + invariants (zero row sums, mean 0 / variance of layer norm)
 *   orc_linear(_bwd), orc_bmm(_bwd)   golden vectors + independent numpy + finite differences
 *   orc_conv2d(_bwd)    golden vectors (pad 0 / stride 1 forward and backward, padded strided
 *                       forward) + finite differences (all, incl. the padded backward)
 *   orc_binary, orc_unary   golden vectors (every op, same shape and 2-D broadcasts) + numpy
 *                       broadcasting on 4-D shapes (independent code)
 *   orc_binary_bwd, orc_unary_bwd   golden vectors (reference backward, incl. its j % size
 *                       broadcast rule) + finite differences on same-shape operands
 *   orc_to_bf16         IEEE round-to-nearest-even (torch.bfloat16 cast) + hand-picked ties
 */
#ifndef DREAM_ORACLE_H
#define DREAM_ORACLE_H
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* RNG (runtime/ops/elementwise.inc:30-54, runtime/io/builtins.inc:511-519).
 * One global std::mt19937, seeded like set_seed(); draws are std::normal_distribution<double>
 * (randn), std::uniform_real_distribution<double>(lo,hi) (selftests) and kaiming(rows, cols)
 * = normal(0, sqrt(2/cols)). */
void orc_set_seed(unsigned int seed);
void orc_randn(double* out, long long n);
void orc_uniform(double* out, long long n, double lo, double hi);
void orc_uniform_f32(float* out, long long n, float lo, float hi);
void orc_kaiming(double* out, int rows, int cols);

/* GEMM, C = A(MxK) @ B(KxN).
 * orc_gemm_ref_d : naive triple loop        (elementwise.inc:878-886)
 * orc_gemm_d     : blocked fp64 4x8 kernel  (elementwise.inc:513-638)
 * orc_gemm_f32   : blocked fp32 8x16 kernel (elementwise.inc:644-738) */
void orc_gemm_ref_d(const double* A, const double* B, double* C, int M, int K, int N);
void orc_gemm_d(const double* A, const double* B, double* C, int M, int K, int N);
void orc_gemm_f32(const float* A, const float* B, float* C, int M, int K, int N);

/* General fp64 GEMM used to check the GPU's transposed variants:
 * C = op(A) @ op(B) + beta*C with op(X) = X or X^T (trans flags), leading dims in elements.
 * The NT and TN shapes are the two matmul-backward products of autograd.inc:91-125. */
void orc_gemm_general_d(int transA, int transB, int M, int N, int K,
                        const double* A, int lda, const double* B, int ldb,
                        double beta, double* C, int ldc);

/* Matmul backward (autograd.inc:91-125): dA += dY @ B^T, dB += A^T @ dY. */
void orc_matmul_bwd(const double* A, const double* B, const double* dY,
                    double* dA, double* dB, int M, int K, int N);

/* Attention forward; layout (B, S*dk): slice b starts at b*S*dk, scale 1/sqrt(dk).
 * orc_attention        : training.inc:178-220 (non-causal)
 * orc_attention_causal : training.inc:225-263
 * orc_flash_fwd        : training.inc:284-401 CPU path (block Bc, online softmax) */
void orc_attention(const double* Q, const double* K, const double* V, double* O,
                   int B, int S, int dk);
void orc_attention_causal(const double* Q, const double* K, const double* V, double* O,
                          int B, int S, int dk);
void orc_flash_fwd(const double* Q, const double* K, const double* V, double* O,
                   int B, int S, int dk, int Bc);

/* Attention backward, "+=" into dQ/dK/dV.
 * orc_attention_bwd : autograd.inc:675-778 (causal selects the attention_causal branch)
 * orc_flash_bwd     : autograd.inc:779-840 (3 passes, Bc = 64) */
void orc_attention_bwd(const double* Q, const double* K, const double* V, const double* dO,
                       double* dQ, double* dK, double* dV, int B, int S, int dk, int causal);
void orc_flash_bwd(const double* Q, const double* K, const double* V, const double* dO,
                   double* dQ, double* dK, double* dV, int B, int S, int dk);
/* orc_attention_rows : O and dQ of selected query rows, standard attention (causal or not):
 * rows[b * nrows + r] is the r-th row taken from slice b; O_rows, dQ_rows are
 * (B, nrows * dk).  The same operations as orc_attention(_causal) / orc_attention_bwd for
 * those rows (training.inc:178-263, autograd.inc:675-778), O(S * dk) per row. */
void orc_attention_rows(const double* Q, const double* K, const double* V, const double* dO,
                        const int* rows, int nrows, double* O_rows, double* dQ_rows, int B,
                        int S, int dk, int causal);

/* Per-row natural-log log-sum-exp of the scaled scores, lse[b*S+i] = m_i + log(l_i),
 * from the (m, l) recurrence of pass 1 in autograd.inc:799-812 (causal) or the full row
 * (non-causal).  This is the statistic the GPU forward saves for its backward. */
void orc_flash_lse(const double* Q, const double* K, double* lse, int B, int S, int dk,
                   int causal);

/* Row reductions (elementwise.inc:338-358, 1550-1570): rows = R, cols = C. */
void orc_softmax_rows(const double* X, double* Y, int R, int C);
void orc_log_softmax_rows(const double* X, double* Y, int R, int C);
/* Their backward, "+=" into GX: softmax from its output Y (autograd.inc:396-409),
 * log_softmax from its input X (autograd.inc:212-233). */
void orc_softmax_bwd(const double* Y, const double* G, double* GX, int R, int C);
void orc_log_softmax_bwd(const double* X, const double* G, double* GX, int N, int C);
/* Row-wise layer norm without affine terms, eps 1e-5 (builtins.inc:167-188), and its
 * backward "+=" into GX (autograd.inc:453-471). */
void orc_layer_norm(const double* X, double* Y, int R, int C);
void orc_layer_norm_bwd(const double* X, const double* Y, const double* DY, double* GX, int R,
                        int C);

/* Fused linear layer Y = X W^T + b (W stored out_dim x in_dim), relu != 0 for
 * linear_relu (elementwise.inc:1432-1510), and its backward (autograd.inc:156-205):
 * relu masks dY in place (Y <= 0 -> 0), then db, dX, dW "+=". */
void orc_linear(const double* X, const double* W, const double* b, double* Y, int N, int in_dim,
                int out_dim, int relu);
void orc_linear_bwd(const double* X, const double* W, const double* Y, double* dY, double* dX,
                    double* dW, double* db, int N, int in_dim, int out_dim, int relu);
/* Batched matmul C[b] = A[b] B[b] (elementwise.inc:1218-1252) and its backward
 * gA += G B^T, gB += A^T G (autograd.inc:549-574); A is (Bt, M*K), B (Bt, K*N). */
void orc_bmm(const double* A, const double* B, double* C, int Bt, int M, int K, int N);
void orc_bmm_bwd(const double* A, const double* B, const double* G, double* gA, double* gB,
                 int Bt, int M, int K, int N);

/* Conv2d, input (N, Cin*H*W), kernel (Cout, Cin*KH*KW), output (N, Cout*OH*OW),
 * OH = (H + 2 pad - KH) / stride + 1: im2col + blocked dgemm + per-channel bias
 * (runtime/nn/conv.inc:12-55 for pad 0 / stride 1, 119-178 padded and strided), and the
 * backward "+=" into gX, gK (autograd.inc:507-535; no bias gradient).  For pad > 0 or
 * stride > 1 the backward is the exact gradient, not the reference's node (which reuses the
 * unpadded shapes); it is pinned by finite differences only. */
void orc_conv2d(const double* X, const double* Kn, const double* bias, double* Y, int N, int Cin,
                int H, int W, int Cout, int KH, int KW, int pad, int stride);
void orc_conv2d_bwd(const double* X, const double* Kn, const double* G, double* gX, double* gK,
                    int N, int Cin, int H, int W, int Cout, int KH, int KW, int pad, int stride);

/* Elementwise ops in fp64.  orc_binary: runCPUBinary (runtime/backend/gpu.inc:484-565) --
 * same-shape operands element by element, otherwise C's flat index i split over c_dims and
 * each operand read through bcastStrides (gpu.inc:443-449: its own contiguous strides, 0 on
 * a dim of 1).  op in BinopCode order (gpu.inc:455-460): add sub mul div mod gt lt ge le eq
 * ne and or atan2 pow min max = 0..16.  orc_unary: runCPUUnary (gpu.inc:599-634) in UnopCode
 * order (relu exp log sqrt abs sigmoid tanh lnot sin cos tan atan floor ceil round = 0..14),
 * 15 = clip, fmax(lo, fmin(hi, a)) (the expression of dream_clip, elementwise.inc:329-336).
 * Their backward "+=": orc_binary_bwd (autograd.inc:58-90 add, sub, minimum/maximum, mul,
 * div with operands indexed j % size; 491-506 pow over the base's elements; Y = the forward
 * output, n = its size) and orc_unary_bwd (autograd.inc:284-288, 342-378). */
void orc_binary(int op, const double* A, const int* a_dims, const double* B, const int* b_dims,
                double* C, const int* c_dims);
void orc_unary(int op, const double* A, double* C, long long n, double lo, double hi);
void orc_binary_bwd(int op, const double* A, long long a_size, const double* B, long long b_size,
                    const double* Y, const double* G, long long n, double* gA, double* gB);
void orc_unary_bwd(int op, const double* X, const double* Y, const double* G, double* GX,
                   long long n);

/* bf16 rounding (training.inc:1969-1976): fp32 -> bf16 -> fp32, round to nearest even
 * by the bias-and-truncate rule.  orc_bf16_bits returns the upper 16 bits. */
float orc_to_bf16(float x);
void orc_bf16_bits(const float* x, uint16_t* out, long long n);

#ifdef __cplusplus
}
#endif
#endif
