// wm_attention.hip -- MultiHeadAttention's forward and closure
// (include/wm_layers.h: wm_mha_fwd / wm_mha_bwd; reference core/layer.cpp:
// 1103-1437) as a sequence of library kernels on the one library stream:
// projections and per-head products on the matrix cores (wm_gemm, with the
// heads addressed as column blocks of the [B, S, E] activations through its
// two-level batch, so nothing is copied or permuted), the mask and softmax
// by the attention-softmax kernels, bias gradients by the broadcast
// backward's column sums.  Host code only.
#include "wm_common.hpp"

#include "../../include/wm_gemm.h"
#include "../../include/wm_layers.h"

#include <cmath>

namespace wm {
namespace {

struct MhaDims {
    int64_t B, Sq, Sk, E, H, hd;
};

int check_dims(const MhaDims& d, const char* who) {
    if (d.B < 0 || d.Sq < 0 || d.Sk < 0 || d.E < 0 || d.H < 1)
        return set_error(WM_ERR_INVALID, std::string(who) + ": negative extent or no heads");
    if (d.E % d.H != 0) return set_error(WM_ERR_INVALID, std::string(who) + ": embed_dim % num_heads != 0");
    return WM_OK;
}

// y [rows, E] = x [rows, E] W^T + bias (W [E, E], row = output feature).
int project(const float* x, const float* W, const float* bias, int64_t rows, int64_t E, float* y) {
    return wm_gemm(0, 1, rows, E, E, 1.0f, x, E, W, E, y, E, 0, bias, 1, 1, nullptr);
}

// gb [E] += column sums of dy [rows, E] (the broadcast add's backward).
int bias_grad(const float* dy, int64_t rows, int64_t E, float* gb) {
    const int64_t ys[2] = {rows, E}, bs[1] = {E};
    return wm_binary_bwd(WM_ADD, dy, dy, ys, 2, gb, bs, 1, nullptr, nullptr, 0, gb, 1);
}

}  // namespace
}  // namespace wm

using namespace wm;

int wm_mha_fwd(const float* q, const float* k, const float* v, const float* mask, int64_t mask_batches,
               const float* Wq, const float* Wk, const float* Wv, const float* Wo, const float* bq, const float* bk,
               const float* bv, const float* bo, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed,
               int64_t heads, float* out, float* attn, float* Q, float* K, float* V, float* ctx) {
    const MhaDims d{batch, seq_q, seq_k, embed, heads, heads > 0 ? embed / heads : 0};
    WM_TRY(check_dims(d, "wm_mha_fwd"));
    if (d.B == 0 || d.Sq == 0 || d.E == 0) return WM_OK;
    if (mask && mask_batches != 1 && mask_batches != d.B)
        return set_error(WM_ERR_INVALID, "wm_mha_fwd: mask batch must be 1 or the batch size");
    if (!q || !k || !v || !Wq || !Wk || !Wv || !Wo || !bq || !bk || !bv || !bo || !out || !attn || !Q || !K || !V ||
        !ctx)
        return set_error(WM_ERR_INVALID, "wm_mha_fwd: null pointer");
    WM_CHECK_INIT();
    const float scale = 1.0f / std::sqrt((float)d.hd);  // layer.cpp:1178
    WM_TRY(project(q, Wq, bq, d.B * d.Sq, d.E, Q));
    WM_TRY(project(k, Wk, bk, d.B * d.Sk, d.E, K));
    WM_TRY(project(v, Wv, bv, d.B * d.Sk, d.E, V));
    if (d.Sk > 0) {
        // scores[b, h] = Q_h K_h^T * scale, one problem per (b, h)
        Workspace scores((size_t)(d.B * d.H * d.Sq * d.Sk) * sizeof(float));
        const int64_t st[6] = {d.Sq * d.E, d.hd, d.Sk * d.E, d.hd, d.H * d.Sq * d.Sk, d.Sq * d.Sk};
        WM_TRY(wm_gemm(0, 1, d.Sq, d.Sk, d.hd, scale, Q, d.E, K, d.E, scores.as<float>(), d.Sk, 0, nullptr,
                       d.B * d.H, d.H, st));
        WM_TRY(wm_attention_softmax_fwd(scores.as<float>(), mask, mask ? mask_batches : 0, d.B, d.H, d.Sq, d.Sk,
                                        attn));
    }
    // ctx[b, :, h] = attn[b, h] V_h
    const int64_t sc[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sk * d.E, d.hd, d.Sq * d.E, d.hd};
    WM_TRY(wm_gemm(0, 0, d.Sq, d.hd, d.Sk, 1.0f, attn, std::max<int64_t>(d.Sk, 1), V, d.E, ctx, d.E, 0, nullptr,
                   d.B * d.H, d.H, sc));
    return project(ctx, Wo, bo, d.B * d.Sq, d.E, out);
}

int wm_mha_bwd(const float* dout, const float* q, const float* k, const float* v, const float* Wq, const float* Wk,
               const float* Wv, const float* Wo, const float* Q, const float* K, const float* V, const float* attn,
               const float* ctx, int64_t batch, int64_t seq_q, int64_t seq_k, int64_t embed, int64_t heads,
               float* gWq, float* gWk, float* gWv, float* gWo, float* gbq, float* gbk, float* gbv, float* gbo,
               float* gq, float* gk, float* gv) {
    const MhaDims d{batch, seq_q, seq_k, embed, heads, heads > 0 ? embed / heads : 0};
    WM_TRY(check_dims(d, "wm_mha_bwd"));
    if (d.B == 0 || d.Sq == 0 || d.E == 0) return WM_OK;
    if (!dout || !q || !k || !v || !Wq || !Wk || !Wv || !Wo || !Q || !K || !V || !attn || !ctx || !gWq || !gWk ||
        !gWv || !gWo || !gbq || !gbk || !gbv || !gbo)
        return set_error(WM_ERR_INVALID, "wm_mha_bwd: null pointer");
    WM_CHECK_INIT();
    const float scale = 1.0f / std::sqrt((float)d.hd);
    const int64_t Rq = d.B * d.Sq, Rk = d.B * d.Sk, E = d.E;
    // output projection (:1305-1318): gbo += sum dout; gWo += dout^T ctx; dctx = dout Wo
    WM_TRY(bias_grad(dout, Rq, E, gbo));
    WM_TRY(wm_gemm(1, 0, E, E, Rq, 1.0f, dout, E, ctx, E, gWo, E, 1, nullptr, 1, 1, nullptr));
    Workspace dctx((size_t)(Rq * E) * sizeof(float));
    WM_TRY(wm_gemm(0, 0, Rq, E, E, 1.0f, dout, E, Wo, E, dctx.as<float>(), E, 0, nullptr, 1, 1, nullptr));
    Workspace dV((size_t)(Rk * E) * sizeof(float));
    Workspace dK((size_t)(Rk * E) * sizeof(float));
    Workspace dQ((size_t)(Rq * E) * sizeof(float));
    if (d.Sk > 0) {
        const size_t n_att = (size_t)(d.B * d.H * d.Sq * d.Sk);
        Workspace dattn(n_att * sizeof(float));
        Workspace ds(n_att * sizeof(float));
        // attn @ V (:1320-1339): dattn_h = dctx_h V_h^T; dV_h = attn_h^T dctx_h
        const int64_t s1[6] = {d.Sq * E, d.hd, d.Sk * E, d.hd, d.H * d.Sq * d.Sk, d.Sq * d.Sk};
        WM_TRY(wm_gemm(0, 1, d.Sq, d.Sk, d.hd, 1.0f, dctx.as<float>(), E, V, E, dattn.as<float>(), d.Sk, 0, nullptr,
                       d.B * d.H, d.H, s1));
        const int64_t s2[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sq * E, d.hd, d.Sk * E, d.hd};
        WM_TRY(wm_gemm(1, 0, d.Sk, d.hd, d.Sq, 1.0f, attn, d.Sk, dctx.as<float>(), E, dV.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s2));
        // softmax (:1341-1360)
        WM_TRY(wm_attention_softmax_bwd(attn, dattn.as<float>(), d.B * d.H * d.Sq, d.Sk, ds.as<float>()));
        // Q K^T (:1362-1383): dQ_h = scale ds_h K_h; dK_h = scale ds_h^T Q_h
        const int64_t s3[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sk * E, d.hd, d.Sq * E, d.hd};
        WM_TRY(wm_gemm(0, 0, d.Sq, d.hd, d.Sk, scale, ds.as<float>(), d.Sk, K, E, dQ.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s3));
        const int64_t s4[6] = {d.H * d.Sq * d.Sk, d.Sq * d.Sk, d.Sq * E, d.hd, d.Sk * E, d.hd};
        WM_TRY(wm_gemm(1, 0, d.Sk, d.hd, d.Sq, scale, ds.as<float>(), d.Sk, Q, E, dK.as<float>(), E, 0, nullptr,
                       d.B * d.H, d.H, s4));
    } else {
        // no keys: the context is zero and so are dV, dK and dQ
        WM_TRY(wm_fill(dQ.as<float>(), 0.0f, Rq * E));
    }
    // V, K, Q projections (:1385-1433): gb += sum dY; gW += dY^T x; gx += dY W
    struct Proj {
        const float* dY;
        const float* x;
        const float* W;
        float *gW, *gb, *gx;
        int64_t rows;
    };
    const Proj proj[3] = {{dV.as<float>(), v, Wv, gWv, gbv, gv, Rk},
                          {dK.as<float>(), k, Wk, gWk, gbk, gk, Rk},
                          {dQ.as<float>(), q, Wq, gWq, gbq, gq, Rq}};
    for (const Proj& p : proj) {
        if (p.rows == 0) continue;
        WM_TRY(bias_grad(p.dY, p.rows, E, p.gb));
        WM_TRY(wm_gemm(1, 0, E, E, p.rows, 1.0f, p.dY, E, p.x, E, p.gW, E, 1, nullptr, 1, 1, nullptr));
        if (p.gx) WM_TRY(wm_gemm(0, 0, p.rows, E, E, 1.0f, p.dY, E, p.W, E, p.gx, E, 1, nullptr, 1, 1, nullptr));
    }
    return WM_OK;
}
