// hk_moe15.hip -- one MoE decode layer of the reference's mixed-1p5-v1
// artifact (moe_suffix of model/qwen80_mixed_hybrid_decode.rs:3636-3752 with
// routed_wave, 2192-2386): routed experts with an HGRAVB01 gate, an HGRAVR02
// up (binary base + Rice residual) and an HGRAVS01 down (y = L (R act));
// router, shared-expert gate and shared expert as HGRAVU01 q8 organs.
//
// The layer is composed from the organ GEMVs on device-resident tables, no
// host round trip:
//   norm -> router, shared-gate logit and shared gate/up GEMVs -> one wave
//   runs softmax / top-k / renormalise and copies the selected experts'
//   descriptors into launch tables -> routed gate+up bases (one launch over
//   2k organs) -> up residuals -> SwiGLU (routed and shared) -> down right
//   factors -> down left factors -> shared down -> combine
//   out = h + sum_r w_r y_r (slot order) + sigmoid(g) * shared.
#include <cmath>
#include <memory>
#include <vector>

#include "hk_internal.h"
#include "hk_router.h"
#include "hk_router_dev.h"

namespace hk {

// xn = h * (1 / sqrt(mean(h^2) + eps)) * (1 + w) (source_qwen80_residual_rms_norm,
// model/qwen80_complete_runtime.rs:6778-6797); one block.
__global__ void __launch_bounds__(1024) moe15_norm_kernel(const float* __restrict__ h, const float* __restrict__ w,
                                                          uint32_t n, float eps, float* __restrict__ xn,
                                                          uint32_t* status) {
    __shared__ float red[16];
    const uint32_t tid = threadIdx.x;
    float s = 0.0f;
    for (uint32_t i = tid; i < n; i += 1024) s += h[i] * h[i];
    s = wave_sum(s);
    if ((tid & 63) == 0) red[tid >> 6] = s;
    __syncthreads();
    float total = 0.0f;
    for (int k = 0; k < 16; ++k) total += red[k];
    const float inv = 1.0f / sqrtf(total / (float)n + eps);
    bool bad = false;
    for (uint32_t i = tid; i < n; i += 1024) {
        const float v = h[i] * inv * (1.0f + w[i]);
        xn[i] = v;
        bad |= !isfinite(v);
    }
    if (bad) atomicOr(status, HK_DEVERR_NONFINITE);
}

struct Moe15Tables {
    const OrganView* gate;  // [E]
    const OrganView* up;    // [E] (the binary bases)
    const ResView* res;     // [E] (the up residuals)
    const OrganView* dr;    // [E] right factors (rank x inter)
    const OrganView* dl;    // [E] left factors (hidden x rank)
    OrganView* sel_gu;      // [2K]: gate views, then up views
    ResView* sel_res;       // [K]
    OrganView* sel_dr;      // [K]
    OrganView* sel_dl;      // [K]
};

// One wave: softmax / top-k / renormalise (source_qwen80_topk_router) over
// the E logits, the weights and ids, and the selected experts' descriptors.
// An id outside [0, E) (only possible on invalid logits, which set the
// status) is replaced by 0 so the launches stay in bounds.
template <int NPL>
__global__ void __launch_bounds__(64) moe15_select_kernel(const float* __restrict__ logits, uint32_t E, uint32_t K,
                                                          Moe15Tables t, int32_t* __restrict__ ids_ws,
                                                          float* __restrict__ w_ws, int32_t* ids_out, float* w_out,
                                                          uint32_t* status) {
    __shared__ TopkLds tk;
    const uint32_t lane = threadIdx.x;
    const ArgBest mine = softmax_topk_wave<NPL>(logits, E, K, 1, nullptr, nullptr, status, &tk);
    if (lane < K) {
        int32_t id = mine.i;
        if (id < 0 || (uint32_t)id >= E) {
            atomicOr(status, HK_DEVERR_ROUTE);
            id = 0;
        }
        ids_ws[lane] = id;
        w_ws[lane] = mine.v;
        if (ids_out) ids_out[lane] = id;
        if (w_out) w_out[lane] = mine.v;
        t.sel_gu[lane] = t.gate[id];
        t.sel_gu[K + lane] = t.up[id];
        t.sel_res[lane] = t.res[id];
        t.sel_dr[lane] = t.dr[id];
        t.sel_dl[lane] = t.dl[id];
    }
}

// act_r = silu(g_r) * u_r for the K routed slots (gu = [g_0..g_{K-1}, u_0..u_{K-1}],
// I each) and act_s = silu(g_s) * u_s for the shared expert (sgu = [g_s, u_s], SI each).
__global__ void moe15_swiglu_kernel(const float* __restrict__ gu, uint32_t K, uint32_t I,
                                    const float* __restrict__ sgu, uint32_t SI, float* __restrict__ act,
                                    float* __restrict__ act_s, uint32_t* status) {
    const uint32_t n = K * I + SI;
    bool bad = false;
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += gridDim.x * blockDim.x) {
        float g, u;
        if (i < K * I) {
            g = gu[i];
            u = gu[K * I + i];
        } else {
            g = sgu[i - K * I];
            u = sgu[SI + (i - K * I)];
        }
        const float a = (g / (1.0f + expf(-g))) * u;
        if (i < K * I) act[i] = a;
        else act_s[i - K * I] = a;
        bad |= !isfinite(a);
    }
    if (bad) atomicOr(status, HK_DEVERR_NONFINITE);
}

// out = h + ((sum_r yd_r * w_r, in slot order from 0) + ys * sigmoid(glogit)).
__global__ void moe15_combine_kernel(const float* __restrict__ h, const float* __restrict__ yd, uint32_t K,
                                     uint32_t H, const float* __restrict__ w, const float* __restrict__ ys,
                                     const float* __restrict__ glogit, float* __restrict__ out, uint32_t* status) {
    const float gate = ys ? 1.0f / (1.0f + expf(-glogit[0])) : 0.0f;
    bool bad = ys && !(isfinite(gate) && gate >= 0.0f && gate <= 1.0f);
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < H; i += gridDim.x * blockDim.x) {
        float c = 0.0f;
        for (uint32_t r = 0; r < K; ++r) c += yd[(size_t)r * H + i] * w[r];
        if (ys) c += ys[i] * gate;
        const float o = h[i] + c;
        out[i] = o;
        bad |= !isfinite(o);
    }
    if (bad) atomicOr(status, HK_DEVERR_NONFINITE);
}

}  // namespace hk

using namespace hk;

struct hk_moe15_layer {
    uint32_t H = 0, I = 0, SI = 0, E = 0, K = 0, rank = 0;
    float eps = 0.0f;
    const hk_organ* router = nullptr;
    const hk_organ* shared_gate = nullptr;
    const hk_organ* s_down = nullptr;
    OrganView gate_view{}, dr_view{}, dl_view{}, sgu_view{};
    void* mem = nullptr;
    float* norm_w = nullptr;
    Moe15Tables t{};
    OrganView* sgu_set = nullptr;  // [2] shared gate, shared up
    float *xn = nullptr, *logits = nullptr, *glogit = nullptr, *gu = nullptr, *sgu = nullptr, *act = nullptr,
          *act_s = nullptr, *mid = nullptr, *yd = nullptr, *ys = nullptr, *w = nullptr;
    float* hbuf = nullptr;  // this layer's output inside a stack
    int32_t* ids = nullptr;
};

static inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

static bool same_shape(const OrganView& a, const OrganView& b) {
    return a.kind == b.kind && a.rows == b.rows && a.cols == b.cols && a.group == b.group;
}

extern "C" int hk_moe15_layer_create(hk_ctx* ctx, const hk_moe15_layer_src* s, hk_moe15_layer** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!s || !s->norm_w || !s->router || !s->gate || !s->up || !s->down_left || !s->down_right)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_layer_create: NULL argument");
    const uint32_t H = s->hidden, I = s->inter, SI = s->shared_inter, E = s->n_experts, K = s->top_k;
    if (!H || !I || !E || !K || K > E || K > 64 || E > 512)
        return set_error(ctx, HK_E_UNSUPPORTED, "mixed-1p5 layer: need 0 < top_k <= min(n_experts, 64), n_experts <= 512");
    if (!(s->eps >= 0.0f) || !std::isfinite(s->eps)) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: bad eps");
    if (s->router->view.rows != E || s->router->view.cols != H)
        return set_error(ctx, HK_E_GEOMETRY, "mixed-1p5 layer: router must be n_experts x hidden");
    if (SI && (!s->shared_gate || !s->shared_gate_proj || !s->shared_up || !s->shared_down))
        return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: shared expert organs are NULL");
    if (SI && (s->shared_gate->view.rows != 1 || s->shared_gate->view.cols != H ||
               s->shared_gate_proj->view.rows != SI || s->shared_gate_proj->view.cols != H ||
               !same_shape(s->shared_gate_proj->view, s->shared_up->view) || s->shared_gate_proj->res_dev ||
               s->shared_up->res_dev || s->shared_down->view.rows != H || s->shared_down->view.cols != SI))
        return set_error(ctx, HK_E_GEOMETRY, "mixed-1p5 layer: shared expert shapes disagree with hidden/shared_inter");
    const hk_organ *g0 = s->gate[0], *u0 = s->up[0], *l0 = s->down_left[0], *r0 = s->down_right[0];
    if (!g0 || !u0 || !l0 || !r0) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: NULL expert organ");
    const uint32_t rank = r0->view.rows;
    if (g0->view.kind != HK_BIN || g0->view.rows != I || g0->view.cols != H || u0->kind != HK_BIN_RICE ||
        !same_shape(g0->view, u0->view) || l0->view.rows != H || l0->view.cols != rank || r0->view.cols != I ||
        rank % 4 || I % 4 || H % 4)
        return set_error(ctx, HK_E_GEOMETRY,
                         "mixed-1p5 layer: experts need a binary gate and an HGRAVR02 up of inter x hidden, and "
                         "down factors hidden x rank, rank x inter");
    std::vector<OrganView> gv(E), uv(E), lv(E), rv(E);
    std::vector<ResView> res(E);
    for (uint32_t e = 0; e < E; ++e) {
        const hk_organ *g = s->gate[e], *u = s->up[e], *l = s->down_left[e], *r = s->down_right[e];
        if (!g || !u || !l || !r) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: NULL expert organ");
        if (!same_shape(g->view, g0->view) || !same_shape(u->view, u0->view) || u->kind != HK_BIN_RICE ||
            !same_shape(l->view, l0->view) || !same_shape(r->view, r0->view) || g->res_dev)
            return set_error(ctx, HK_E_GEOMETRY, "mixed-1p5 layer: experts must share kinds and shapes");
        gv[e] = g->view;
        uv[e] = u->view;
        lv[e] = l->view;
        rv[e] = r->view;
        res[e] = u->res;
    }
    std::unique_ptr<hk_moe15_layer> L(new hk_moe15_layer());
    L->H = H;
    L->I = I;
    L->SI = SI;
    L->E = E;
    L->K = K;
    L->rank = rank;
    L->eps = s->eps;
    L->router = s->router;
    L->shared_gate = SI ? s->shared_gate : nullptr;
    L->s_down = SI ? s->shared_down : nullptr;
    L->gate_view = g0->view;
    L->dr_view = r0->view;
    L->dl_view = l0->view;
    if (SI) L->sgu_view = s->shared_gate_proj->view;
    // one allocation: tables, launch tables, workspace (each section 256-B aligned)
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_norm = take(H * 4), o_gate = take(E * sizeof(OrganView)), o_up = take(E * sizeof(OrganView)),
                 o_res = take(E * sizeof(ResView)), o_dr = take(E * sizeof(OrganView)),
                 o_dl = take(E * sizeof(OrganView)), o_sgu_tab = take(2 * K * sizeof(OrganView)),
                 o_sres = take(K * sizeof(ResView)), o_sdr = take(K * sizeof(OrganView)),
                 o_sdl = take(K * sizeof(OrganView)), o_sset = take(2 * sizeof(OrganView)), o_xn = take(H * 4),
                 o_logits = take(E * 4), o_glogit = take(16), o_gu = take(2 * (size_t)K * I * 4),
                 o_sgu = take(2 * (size_t)SI * 4 + 16), o_act = take((size_t)K * I * 4), o_acts = take(SI * 4 + 16),
                 o_mid = take((size_t)K * rank * 4), o_yd = take((size_t)K * H * 4), o_ys = take(H * 4),
                 o_w = take(K * 4), o_ids = take(K * 4), o_hbuf = take(H * 4);
    if (hipMalloc(&L->mem, off) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "mixed-1p5 layer allocation failed");
    uint8_t* m = static_cast<uint8_t*>(L->mem);
    L->norm_w = reinterpret_cast<float*>(m + o_norm);
    L->t.gate = reinterpret_cast<const OrganView*>(m + o_gate);
    L->t.up = reinterpret_cast<const OrganView*>(m + o_up);
    L->t.res = reinterpret_cast<const ResView*>(m + o_res);
    L->t.dr = reinterpret_cast<const OrganView*>(m + o_dr);
    L->t.dl = reinterpret_cast<const OrganView*>(m + o_dl);
    L->t.sel_gu = reinterpret_cast<OrganView*>(m + o_sgu_tab);
    L->t.sel_res = reinterpret_cast<ResView*>(m + o_sres);
    L->t.sel_dr = reinterpret_cast<OrganView*>(m + o_sdr);
    L->t.sel_dl = reinterpret_cast<OrganView*>(m + o_sdl);
    L->sgu_set = reinterpret_cast<OrganView*>(m + o_sset);
    L->xn = reinterpret_cast<float*>(m + o_xn);
    L->logits = reinterpret_cast<float*>(m + o_logits);
    L->glogit = reinterpret_cast<float*>(m + o_glogit);
    L->gu = reinterpret_cast<float*>(m + o_gu);
    L->sgu = reinterpret_cast<float*>(m + o_sgu);
    L->act = reinterpret_cast<float*>(m + o_act);
    L->act_s = reinterpret_cast<float*>(m + o_acts);
    L->mid = reinterpret_cast<float*>(m + o_mid);
    L->yd = reinterpret_cast<float*>(m + o_yd);
    L->ys = reinterpret_cast<float*>(m + o_ys);
    L->w = reinterpret_cast<float*>(m + o_w);
    L->ids = reinterpret_cast<int32_t*>(m + o_ids);
    L->hbuf = reinterpret_cast<float*>(m + o_hbuf);
    auto up_copy = [&](const void* dst, const void* src, size_t bytes) {
        return check_hip(ctx, hipMemcpy(const_cast<void*>(dst), src, bytes, hipMemcpyDefault), "mixed-1p5 layer upload");
    };
    int rc = up_copy(L->norm_w, s->norm_w, H * 4);
    if (!rc) rc = up_copy(L->t.gate, gv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(L->t.up, uv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(L->t.res, res.data(), E * sizeof(ResView));
    if (!rc) rc = up_copy(L->t.dr, rv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(L->t.dl, lv.data(), E * sizeof(OrganView));
    if (!rc && SI) {
        const OrganView sv[2] = {s->shared_gate_proj->view, s->shared_up->view};
        rc = up_copy(L->sgu_set, sv, sizeof sv);
    }
    if (rc) {
        (void)hipFree(L->mem);
        return rc;
    }
    *out = L.release();
    return HK_OK;
}

extern "C" int hk_moe15_layer_free(hk_ctx* ctx, hk_moe15_layer* L) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!L) return HK_OK;
    int rc = check_hip(ctx, hipFree(L->mem), "hipFree (mixed-1p5 layer)");
    delete L;
    return rc;
}

extern "C" int hk_moe15_decode_layer(hk_ctx* ctx, hk_moe15_layer* L, const float* h, float* out, int32_t* ids,
                                     float* weights, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!L || !h || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_decode_layer: NULL argument");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const uint32_t H = L->H, I = L->I, SI = L->SI, K = L->K;
    uint32_t* st = ctx->dev_status;
    int rc = check_hip(ctx, [&]() {
        hipLaunchKernelGGL(moe15_norm_kernel, dim3(1), dim3(1024), 0, s, h, L->norm_w, H, L->eps, L->xn, st);
        return hipGetLastError();
    }(), "mixed-1p5 norm");
    if (rc) return rc;
    auto gemv = [&](const OrganView* views, uint32_t n, const OrganView& sh, const float* x, size_t xs, float* y,
                    size_t ys, const char* what) {
        return check_hip(ctx, launch_gemv_tiled(views, n, sh, x, xs, y, ys, s), what);
    };
    if ((rc = gemv(static_cast<const OrganView*>(L->router->view_dev), 1, L->router->view, L->xn, 0, L->logits, 0,
                   "mixed-1p5 router")))
        return rc;
    if (SI) {
        if ((rc = gemv(static_cast<const OrganView*>(L->shared_gate->view_dev), 1, L->shared_gate->view, L->xn, 0,
                       L->glogit, 0, "mixed-1p5 shared gate")))
            return rc;
        if ((rc = gemv(L->sgu_set, 2, L->sgu_view, L->xn, 0, L->sgu, SI, "mixed-1p5 shared gate/up"))) return rc;
    }
    rc = check_hip(ctx, [&]() {
        if (L->E <= 64)
            hipLaunchKernelGGL((moe15_select_kernel<1>), dim3(1), dim3(64), 0, s, L->logits, L->E, K, L->t, L->ids, L->w,
                               ids, weights, st);
        else if (L->E <= 256)
            hipLaunchKernelGGL((moe15_select_kernel<4>), dim3(1), dim3(64), 0, s, L->logits, L->E, K, L->t, L->ids, L->w,
                               ids, weights, st);
        else
            hipLaunchKernelGGL((moe15_select_kernel<8>), dim3(1), dim3(64), 0, s, L->logits, L->E, K, L->t, L->ids, L->w,
                               ids, weights, st);
        return hipGetLastError();
    }(), "mixed-1p5 select");
    if (rc) return rc;
    // routed gate and up bases in one launch (x broadcast), then the up residuals
    if ((rc = gemv(L->t.sel_gu, 2 * K, L->gate_view, L->xn, 0, L->gu, I, "mixed-1p5 gate/up"))) return rc;
    if ((rc = check_hip(ctx, launch_rice_apply(L->t.sel_res, K, I, H, L->xn, 0, L->gu + (size_t)K * I, I, s),
                        "mixed-1p5 up residual")))
        return rc;
    rc = check_hip(ctx, [&]() {
        const uint32_t n = K * I + SI;
        hipLaunchKernelGGL(moe15_swiglu_kernel, dim3((n + 255) / 256), dim3(256), 0, s, L->gu, K, I, L->sgu, SI, L->act,
                           L->act_s, st);
        return hipGetLastError();
    }(), "mixed-1p5 swiglu");
    if (rc) return rc;
    if ((rc = gemv(L->t.sel_dr, K, L->dr_view, L->act, I, L->mid, L->rank, "mixed-1p5 down right"))) return rc;
    if ((rc = gemv(L->t.sel_dl, K, L->dl_view, L->mid, L->rank, L->yd, H, "mixed-1p5 down left"))) return rc;
    if (SI && (rc = gemv(static_cast<const OrganView*>(L->s_down->view_dev), 1, L->s_down->view, L->act_s, 0, L->ys, 0,
                         "mixed-1p5 shared down")))
        return rc;
    return check_hip(ctx, [&]() {
        hipLaunchKernelGGL(moe15_combine_kernel, dim3((H + 255) / 256), dim3(256), 0, s, h, L->yd, K, H, L->w,
                           SI ? L->ys : nullptr, L->glogit, out, st);
        return hipGetLastError();
    }(), "mixed-1p5 combine");
}

extern "C" int hk_moe15_decode_stack(hk_ctx* ctx, hk_moe15_layer* const* layers, uint32_t n_layers, const float* h,
                                     float* out, int32_t* ids, float* weights, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!layers || !n_layers || !h || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_decode_stack: NULL argument");
    for (uint32_t l = 0; l < n_layers; ++l)
        if (!layers[l] || layers[l]->H != layers[0]->H || layers[l]->K != layers[0]->K)
            return set_error(ctx, HK_E_GEOMETRY, "hk_moe15_decode_stack: layers must share hidden and top_k");
    const uint32_t K = layers[0]->K;
    const float* cur = h;
    for (uint32_t l = 0; l < n_layers; ++l) {
        float* dst = l + 1 == n_layers ? out : layers[l]->hbuf;
        const int rc = hk_moe15_decode_layer(ctx, layers[l], cur, dst, ids ? ids + (size_t)l * K : nullptr,
                                             weights ? weights + (size_t)l * K : nullptr, stream);
        if (rc) return rc;
        cur = dst;
    }
    return HK_OK;
}
