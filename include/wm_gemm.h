/*
 * wm_gemm.h -- C ABI of libwm_hip's fp32 matrix products on the MFMA
 * matrix cores: Tensor::matmul and Tensor::bmm (reference
 * core/tensor.cpp:783-895) with their backward, Tensor::transpose
 * (:2223-2248), and the general strided product the drop-in Linear and
 * MultiHeadAttention modules are built on (core/layer.cpp:13-15,
 * :1103-1437).
 *
 * Conventions are those of wm_hip.h: status codes, wm_last_error(), device
 * pointers to row-major fp32, one library stream.  Gradient outputs take an
 * `accumulate` flag (1 = "+=", 0 = overwrite) and may be NULL when that
 * input does not require grad.
 *
 * Arithmetic: products and sums in fp32 on the matrix cores (no
 * reduced-precision inputs): this library's v_mfma_f32_32x32x2_f32 kernels
 * (for products whose tiles are all interior, operands staged straight
 * into LDS; for the rest, through registers), or, for the plain large
 * products (wm_gemm_library), rocBLAS's fp32 kernels with atomics off.  The
 * reference adds each product to its fp32 accumulator in k order; the
 * matrix cores add them in another order (and a product with fewer output
 * tiles than CUs and a long k adds the partial
 * products of its k slices in a second pass, in fixed slice order), so the
 * results agree with the reference within fp32 summation error (tested
 * against an fp64 restatement relative to sum_k |a_ik * b_kj|), not bit for
 * bit; each route gives the same bits on every run.  Products of small
 * integers, whose partial sums are exact in fp32, are bit-exact.
 */
#ifndef WM_GEMM_H
#define WM_GEMM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The general product, for `batch` problems:
 *   C_p = alpha * op(A_p) * op(B_p)  [+ C_p if accumulate]  [+ bias]
 * op(A_p) is m x k: A_p row-major m x k with row stride lda (trans_a = 0) or
 * A_p row-major k x m (trans_a = 1, i.e. A_p^T is used); op(B_p) is k x n
 * likewise (trans_b = 1: B_p stored n x k).  C_p is m x n with row stride
 * ldc.  bias (NULL or [n]) is added to every row after the product (and
 * after the accumulation), as Linear's matmul-then-add does.
 * Problem p = (o, i) with o = p / batch_inner, i = p % batch_inner starts at
 *   A + o * strides[0] + i * strides[1],  B + o * strides[2] + i * strides[3],
 *   C + o * strides[4] + i * strides[5]
 * (elements).  strides may be NULL only when batch == 1.  Two batch levels
 * express per-head slices of [batch, seq, heads * head_dim] activations
 * without copies.  Output problems must not overlap each other or the
 * inputs.  No counterpart function in the reference: it is the loop nest
 * the reference repeats inline in matmul_blocked (core/tensor.cpp:281-331),
 * matmul/bmm's closures (:797-815, :857-893) and MultiHeadAttention
 * (core/layer.cpp:1133-1260, :1310-1400).                                   */
int wm_gemm(int trans_a, int trans_b, int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda,
            const float* b, int64_t ldb, float* c, int64_t ldc, int accumulate, const float* bias, int64_t batch,
            int64_t batch_inner, const int64_t* strides);

/* The route of the plain large products (unbatched, m, n >= 128, k >= 256,
 * not both bias and accumulate) and of the one-level batches of
 * untransposed products with m, n >= 128, k <= 256 and no bias that this
 * library's interior-tile kernel does not take (m or n not a multiple of
 * 128, k not of 64, rows not 16-byte aligned): 1 (default) = rocBLAS's
 * tuned fp32 kernels (sgemm / sgemm_strided_batched, atomics off), which
 * are faster there; 0 = this library's MFMA kernels for every product.  mode 0 or 1 sets it, any other value only queries; returns the
 * route now in force.  The results agree with the reference within the same
 * fp32 summation error either way (both deterministic run to run).  No
 * counterpart in the reference (a routing switch, for tests and
 * measurements of each kernel).                                              */
int wm_gemm_library(int mode);

/* Tensor::matmul, core/tensor.cpp:783-795: c[m, n] = a[m, k] @ b[k, n]. */
int wm_matmul(const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* c);

/* matmul's closure, core/tensor.cpp:797-815, given g = dL/dc [m, n]:
 *   ga [m, k] (+)= g @ b^T;  gb [k, n] (+)= a^T @ g                          */
int wm_matmul_bwd(const float* g, const float* a, const float* b, int64_t m, int64_t k, int64_t n, float* ga,
                  int accumulate_a, float* gb, int accumulate_b);

/* Tensor::bmm, core/tensor.cpp:827-852: c[p] = a[p] @ b[p] for
 * p < batch; a [batch, m, k], b [batch, k, n], c [batch, m, n].             */
int wm_bmm(const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n, float* c);

/* bmm's closure, core/tensor.cpp:854-893: per p, ga[p] (+)= g[p] @ b[p]^T,
 * gb[p] (+)= a[p]^T @ g[p].                                                  */
int wm_bmm_bwd(const float* g, const float* a, const float* b, int64_t batch, int64_t m, int64_t k, int64_t n,
               float* ga, int accumulate_a, float* gb, int accumulate_b);

/* Tensor::transpose, core/tensor.cpp:2223-2248, and its closure:
 *   out[c][r] (+)= x[r][c]  for x [rows, cols], out [cols, rows].
 * The forward writes (accumulate 0); the closure adds the transposed
 * gradient (accumulate 1).  x and out must not overlap.                      */
int wm_transpose2d(const float* x, int64_t rows, int64_t cols, float* out, int accumulate);

#ifdef __cplusplus
}
#endif

#endif /* WM_GEMM_H */
