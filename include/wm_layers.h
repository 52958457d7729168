/*
 * wm_layers.h -- C ABI of libwm_hip's normalisation and attention kernels:
 * the reduction / softmax work inside whitematter's LayerNorm, BatchNorm2d
 * and MultiHeadAttention modules (reference core/layer.cpp), which the
 * reference writes as raw host loops that bypass its Tensor ops, and the
 * whole MultiHeadAttention forward and closure on top of them.
 *
 * Conventions are those of wm_hip.h: status codes, wm_last_error(), device
 * pointers to contiguous row-major fp32, one library stream, and for every
 * gradient output an `accumulate` flag (1 = "+=", 0 = the buffer is known to
 * be zero and is overwritten).  A NULL gradient pointer means that input does
 * not require grad (the reference's `if (x->requires_grad)` branches).
 *
 * Statistics the backward needs (per-row / per-channel mean and 1/std) are
 * written by the forward into caller-provided device arrays, as the
 * reference's closures capture them; the backward reads the input again
 * (the reference recomputes x_norm from input->data in its closure).
 */
#ifndef WM_LAYERS_H
#define WM_LAYERS_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* LayerNorm::forward, core/layer.cpp:395-446, over the trailing n elements
 * of each of `rows` instances:
 *   mean_r = sum(x_r) / n;  var_r = sum((x_r - mean_r)^2) / n
 *   inv_std_r = 1 / sqrt(var_r + eps)
 *   y = gamma * ((x - mean_r) * inv_std_r) + beta
 * gamma, beta [n]; mean, inv_std [rows] (written).                         */
int wm_layernorm_fwd(const float* x, const float* gamma, const float* beta, int64_t rows, int64_t n, float eps,
                     float* y, float* mean, float* inv_std);

/* LayerNorm's closure, core/layer.cpp:447-504:
 *   x_norm = (x - mean_r) * inv_std_r
 *   dgamma (+)= sum_r g * x_norm;  dbeta (+)= sum_r g
 *   gx (+)= inv_std_r * (g*gamma - mean_i(g*gamma) - x_norm * mean_i(g*gamma*x_norm))   */
int wm_layernorm_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                     int64_t rows, int64_t n, float* gx, int acc_x, float* dgamma, int acc_gamma, float* dbeta,
                     int acc_beta);

/* BatchNorm2d::forward, core/layer.cpp:202-280, x [batch, channels, spatial]
 * (spatial = H * W), per channel over batch * spatial elements.
 * training != 0: batch statistics (biased variance), and the running
 * statistics are updated in place:
 *   running_mean = (1 - momentum) * running_mean + momentum * mean
 *   running_var  = (1 - momentum) * running_var  + momentum * var
 * training == 0: mean / var are running_mean / running_var (not updated).
 *   inv_std = 1 / sqrt(var + eps);  y = gamma * ((x - mean) * inv_std) + beta
 * mean, inv_std [channels] (written: what the closure captures).            */
int wm_batchnorm2d_fwd(const float* x, const float* gamma, const float* beta, float* running_mean,
                       float* running_var, int64_t batch, int64_t channels, int64_t spatial, float eps,
                       float momentum, int training, float* y, float* mean, float* inv_std);

/* BatchNorm2d's closure, core/layer.cpp:281-374 (the same formula in both
 * modes, with the captured mean / inv_std), n = batch * spatial:
 *   dgamma (+)= sum g * x_norm;  dbeta (+)= sum g
 *   dvar  = sum (g*gamma) * (x - mean) * -0.5 * inv_std^3
 *   dmean = sum (g*gamma) * (-inv_std) + dvar * sum(-2 (x - mean)) / n
 *   gx (+)= (g*gamma) * inv_std + dvar * 2 (x - mean) / n + dmean / n       */
int wm_batchnorm2d_bwd(const float* g, const float* x, const float* gamma, const float* mean, const float* inv_std,
                       int64_t batch, int64_t channels, int64_t spatial, float* gx, int acc_x, float* dgamma,
                       int acc_gamma, float* dbeta, int acc_beta);

/* MultiHeadAttention's softmax over the keys, core/layer.cpp:1210-1237, with
 * the mask add of :1198-1204 fused in front of it.  scores [batch, heads,
 * tq, tk] are the scaled dot products (Q K^T / sqrt(head_dim)); mask is NULL
 * or [mask_batches, 1, tq, tk] with mask_batches 1 (broadcast over the
 * batch) or batch; it is added to the scores before the softmax:
 *   s = scores + mask;  m = max(-FLT_MAX, max_j s_j)
 *   attn_j = exp(s_j - m) / sum_k exp(s_k - m)
 * (the quotient taken as a product with the row sum's reciprocal).         */
int wm_attention_softmax_fwd(const float* scores, const float* mask, int64_t mask_batches, int64_t batch,
                             int64_t heads, int64_t tq, int64_t tk, float* attn);

/* Its backward, core/layer.cpp:1343-1360, over rows = batch*heads*tq rows:
 *   d_scores_j = attn_j * (d_attn_j - sum_k attn_k d_attn_k)
 * d_scores is written (the reference assigns a fresh tensor).              */
int wm_attention_softmax_bwd(const float* attn, const float* d_attn, int64_t rows, int64_t tk, float* d_scores);

/* Dropout's mask, core/layer.cpp:47-73: mask_i = u_i > p ? 1 / (1 - p) : 0,
 * with u_i in [0, 1) the top 24 bits of splitmix64(seed + i) (a counter-
 * based generator, so any element can be drawn independently; the
 * reference draws from a sequential std::mt19937, whose stream a device
 * cannot reproduce -- the distribution is the same, the bits are not).
 * The drop-in multiplies the input by this mask.                           */
int wm_dropout_mask(float* mask, int64_t n, float p, uint64_t seed);

/* MultiHeadAttention::forward(query, key, value, mask), core/layer.cpp:
 * 1103-1280, with heads = num_heads, hd = embed / heads:
 *   Q = q Wq^T + bq;  K = k Wk^T + bk;  V = v Wv^T + bv
 *   attn[b, h] = softmax(Q_h K_h^T * (1 / sqrt(hd)) + mask[b or 0])
 *   ctx[b, :, h] = attn[b, h] V_h;  out = ctx Wo^T + bo
 * where X_h is the h-th hd-wide column block of X.  q [B, Sq, E]; k, v
 * [B, Sk, E]; W* [E, E] (row = output feature); b* [E]; mask NULL or
 * [mask_batches, 1, Sq, Sk] with mask_batches 1 or B.  Writes out [B, Sq, E]
 * and the values the reference's closure captures: Q [B, Sq, E], K, V
 * [B, Sk, E], attn [B, H, Sq, Sk] (the module's attn_weights), ctx
 * [B, Sq, E].  Products on the matrix cores (include/wm_gemm.h).  For
 * Sk <= 1024 and hd <= 128 with hd and E multiples of 4 (16-byte aligned
 * operands) the score product, mask and softmax are one kernel that writes
 * only attn (the scores stay in registers; the softmax's arithmetic is
 * wm_attention_softmax_fwd's, its sums in another order); otherwise the
 * scores go to a buffer and wm_attention_softmax_fwd takes them.           */
int wm_mha_fwd(const float* q, const float* k, const float* v, const float* mask, int64_t mask_batches,
               const float* Wq, const float* Wk, const float* Wv, const float* Wo, const float* bq, const float* bk,
               const float* bv, const float* bo, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed,
               int64_t heads, float* out, float* attn, float* Q, float* K, float* V, float* ctx);

/* Its closure, core/layer.cpp:1299-1433, given dout = dL/dout and the
 * captured Q, K, V, attn, ctx.  Every gradient is added to (+=), as the
 * reference's loops do; the eight parameter gradients are always written
 * (the reference does not test their requires_grad); gq, gk, gv may be NULL
 * (that input does not require grad) and may be the same buffer (self
 * attention: the V, K and Q projections add into it in that order).  On the
 * fused route (hd <= 128 with hd and E multiples of 4, 16-byte aligned
 * operands; any key length) dattn = dctx_h V_h^T and the
 * softmax backward are one kernel, whose row dot sum_j attn_ij dattn_ij is
 * taken as dctx_i . ctx_i over the head's columns -- the same value in exact
 * arithmetic since ctx_h = attn_h V_h, so ctx must be the forward's.        */
int wm_mha_bwd(const float* dout, const float* q, const float* k, const float* v, const float* Wq, const float* Wk,
               const float* Wv, const float* Wo, const float* Q, const float* K, const float* V, const float* attn,
               const float* ctx, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed, int64_t heads,
               float* gWq, float* gWk, float* gWv, float* gWo, float* gbq, float* gbk, float* gbv, float* gbo,
               float* gq, float* gk, float* gv);

/* The route of the attention's per-head score products: 1 (default) = the
 * fused kernels above where the shape fits; 0 = always the two-pass route
 * (wm_gemm's product into a scores buffer, then the attention-softmax
 * kernels).  mode 0 or 1 sets it, any other value only queries; returns the
 * route now in force.  No counterpart in the reference (a routing switch,
 * for tests and measurements of each route).                               */
int wm_mha_fused(int mode);

#ifdef __cplusplus
}
#endif

#endif /* WM_LAYERS_H */
