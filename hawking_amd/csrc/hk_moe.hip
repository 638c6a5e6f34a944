// hk_moe.hip -- one MoE decode layer (moe_suffix) at batch 1 on device data.
//
// Three stream-ordered launches, no host round trip; expert weights live in
// the tiled layout and every packed dot runs on the int8 matrix-core engine
// (hk_mfma.h).  The routed expert ids never leave the device
// (run_qwen80_routed_expert_table,
//  crates/hawking-core/src/model/qwen80_device_expert_table.rs:1204-1247):
//   1. route:   every block recomputes xn = RMSNorm(1+w)(h) in LDS; blocks
//               0..ceil(E/4)-1 compute the router logits (one row per wave),
//               the next block also the shared-gate logit and stores xn.
//   2. gate/up: one workgroup per (16-row tile, slot); each runs softmax /
//               top-k / renormalise over the logits itself to find its
//               slot's expert (slot K = the shared expert) while its other
//               waves build the x image of xn in LDS (fixed-point limb tiles
//               with E = 0; a separate image block in the route kernel was
//               that kernel's last to finish), then its 4 waves
//               split the columns, both organs share each x-image fetch, and
//               the epilogue applies SwiGLU: act = silu(gate.xn) * (up.xn).
//   3. down:    one workgroup per 16-row output tile, one wave per slot; each
//               wave builds the x image of its slot's activations, and the
//               block combines out = h + sum_r w_r y_r (route order)
//               + gate * y_shared  (moe_suffix,
//               model/qwen80_uniform_q4_hybrid_decode.rs:2615-2757).
#include "hk_internal.h"
#include "hk_mfma.h"
#include "hk_moe.h"
#include "hk_router_dev.h"

namespace hk {

size_t moe_img_bytes(int kind, uint32_t H) {
    const uint32_t S = n_steps_for(kind, H);
    return kind == HK_Q4 ? x_lds_bytes<HK_Q4>(S) : x_lds_bytes<HK_MIXED>(S);
}

size_t moe_gate_up_lds_bytes(int kind, uint32_t H) { return moe_img_bytes(kind, H) + 4 * 32 * sizeof(float); }

// Floats of x staging for an image of `cols` columns (cols rounded up to whole steps).
static uint32_t stage_floats(int kind, uint32_t cols) { return n_steps_for(kind, cols) * tile_step_cols(kind); }

// The route kernel's LDS: xn (whole steps).
size_t moe_route_lds_bytes(int kind, uint32_t H) { return (size_t)stage_floats(kind, H) * sizeof(float); }

size_t moe_down_lds_bytes(int kind, uint32_t Imax, uint32_t slots) {
    return (size_t)slots * (moe_img_bytes(kind, Imax) + 16 * sizeof(float) + (size_t)stage_floats(kind, Imax) * sizeof(float));
}

// Float4s of h (per thread) and of a router row (per lane) held in registers:
// every global load of the route kernel is issued before its first reduction.
constexpr int H_PRE = 8;    // 256 threads x 8 float4 = hidden <= 8192
constexpr int ROW_PRE = 8;  // 64 lanes x 8 float4 = 2048 columns, the rest streamed

__device__ __forceinline__ float dot4(const float4& a, const float4& b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

template <int KIND>
__global__ void __launch_bounds__(256) moe_route_kernel(MoeDims d, MoeLayerDev L, const float* __restrict__ h,
                                                        MoeWs ws) {
    extern __shared__ __align__(16) float xn[];  // [H rounded up to whole steps]
    __shared__ float red[4];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t nrb = (d.E + 3u) / 4u, n4 = d.H / 4u;
    // this wave's weight row: a router row, or the shared-expert gate (last block, wave 0)
    const float* wrow = nullptr;
    if (blockIdx.x < nrb) {
        const uint32_t row = blockIdx.x * 4u + wave;
        if (row < d.E) wrow = L.router_w + (size_t)row * d.H;
    } else if (blockIdx.x == nrb && wave == 0) {
        wrow = L.gate_w;
    }
    // every load is unconditional (indices clamped to the vector, values past
    // it dropped afterwards): a load under a per-lane condition makes the
    // compiler wait for it before the next one issues.  h and the norm
    // weight come first, so the RMSNorm waits for them only.
    const float4* h4 = reinterpret_cast<const float4*>(h);
    const float4* g4 = reinterpret_cast<const float4*>(L.norm_w);
    float4 hv[H_PRE], gv[H_PRE];
#pragma unroll
    for (int k = 0; k < H_PRE; ++k) {
        const uint32_t j = min(threadIdx.x + 256u * k, n4 - 1u);
        hv[k] = ldg(h4 + j);
        gv[k] = ldg(g4 + j);
    }
    const float4* w4 = reinterpret_cast<const float4*>(wrow ? wrow : L.router_w);
    float4 wv[ROW_PRE];
#pragma unroll
    for (int k = 0; k < ROW_PRE; ++k) wv[k] = ldg(w4 + min((uint32_t)lane + 64u * k, n4 - 1u));
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < H_PRE; ++k) ss += threadIdx.x + 256u * k < n4 ? dot4(hv[k], hv[k]) : 0.0f;
    // xn = RMSNorm(1+w)(h) = h * (mean(h^2) + eps)^-1/2 * (1 + w)
    const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)d.H + d.eps);
    float4* x4 = reinterpret_cast<float4*>(xn);
#pragma unroll
    for (int k = 0; k < H_PRE; ++k) {
        const uint32_t j = threadIdx.x + 256u * k;
        if (j < n4)
            x4[j] = make_float4(hv[k].x * inv * (1.0f + gv[k].x), hv[k].y * inv * (1.0f + gv[k].y),
                                hv[k].z * inv * (1.0f + gv[k].z), hv[k].w * inv * (1.0f + gv[k].w));
    }
    __syncthreads();
    if (wrow) {
        float acc = 0.f;
#pragma unroll
        for (int k = 0; k < ROW_PRE; ++k) {
            const uint32_t j = (uint32_t)lane + 64u * k;
            if (j < n4) acc += dot4(wv[k], x4[j]);
        }
        for (uint32_t j = (uint32_t)lane + 64u * ROW_PRE; j < n4; j += 64u) acc += dot4(w4[j], x4[j]);
        acc = wave_sum(acc);
        if (lane == 0) {
            if (blockIdx.x < nrb)
                ws.logits[blockIdx.x * 4u + wave] = acc;
            else
                ws.gate[0] = acc;
        }
    }
    if (blockIdx.x == nrb) {
        // xn for the gate/up kernel, which builds its x image from it
        for (uint32_t j = threadIdx.x; j < n4; j += 256u) reinterpret_cast<float4*>(ws.xn)[j] = x4[j];
    }
}

// Gate/up of one (16-row tile, slot).  Every workgroup of a routed slot first
// ranks the router logits itself (softmax, top-k, renormalise:
// source_qwen80_topk_router; one wave, about 2 us) while its other waves
// build the layer's x image of xn (E = 0) in LDS, and takes its slot's
// expert; this saves a launch.  Slot 0's tile 0 publishes the route and the shared-gate value
// for the down kernel.
constexpr int GU_IMG_PT = 2;  // x chunks per thread loaded before the scatter (2,048 columns)

template <int KIND, int D, int NPL>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(MoeDims d, MoeLayerDev L, MoeWs ws, int32_t* ids_out,
                                                          float* w_out) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int32_t sel_id;
    __shared__ TopkLds tk;
    const uint32_t slot = blockIdx.y, T = blockIdx.x;
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool lead = T == 0, routed = slot < d.K;
    const uint32_t S = n_steps_for(KIND, d.H), ib = (uint32_t)x_lds_bytes<KIND>(S);
    // the slot's base views (expert 0's, or the shared expert's), loaded with the logits
    const uint32_t base = routed ? 0u : d.E * 3u;
    const OrganView g0 = L.table[base], u0 = L.table[base + 1u];
    OrganView dn0{};
    if constexpr (KIND == HK_MIXED) dn0 = L.table[base + 2u];
    // the ranking wave: slots 8 apart share CUs when the grid exceeds the
    // CU count (workgroups i and i + 256 of a 32-tile grid), so theirs rank
    // on different SIMDs
    const uint32_t tw = (slot >> 3) & 3u;
    if (routed && wave == tw) {
        const bool pub = lead && slot == 0;
        const ArgBest mine = softmax_topk_wave<NPL>(ws.logits, d.E, d.K, 1, pub ? ws.ids : nullptr,
                                                    pub ? ws.weights : nullptr, pub ? ws.status : nullptr, &tk,
                                                    lane, d.tie_eps);
        if (pub && (uint32_t)lane < d.K) {
            if (ids_out) ids_out[lane] = mine.i;
            if (w_out) w_out[lane] = mine.v;
        }
        if (pub && lane == 0) ws.gate[1] = L.gate_w ? 1.0f / (1.0f + expf(-ws.gate[0])) : 1.0f;
        if ((uint32_t)lane == slot) sel_id = mine.i;
    } else {
        // the x image of xn with E = 0, scattered into LDS by the other waves
        // (the image the GEMV engine builds: the same bits); every chunk's
        // load in flight before the first scatter
        const uint32_t nt = routed ? blockDim.x - 64u : blockDim.x;
        const uint32_t tid = routed && threadIdx.x >= 64u * tw ? threadIdx.x - 64u : threadIdx.x;
        const uint32_t nch = S * tile_step_cols(KIND) / 8u;
        float* sxw = reinterpret_cast<float*>(lds + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
        if (tid < 64u) image_zero_blocks<KIND>(tid, lds, S);
        float4 v[GU_IMG_PT][2];
#pragma unroll
        for (int j = 0; j < GU_IMG_PT; ++j) load_chunk(ws.xn, 8u * (tid + nt * (uint32_t)j), d.H, v[j]);
        bool bad = false;
#pragma unroll
        for (int j = 0; j < GU_IMG_PT; ++j) {
            const uint32_t ch = tid + nt * (uint32_t)j;
            if (ch < nch) bad |= image_chunk<KIND>(ch, v[j], lds, sxw, 0u, 0u);
        }
        for (uint32_t ch = tid + nt * GU_IMG_PT; ch < nch; ch += nt) {
            float4 w[2];
            load_chunk(ws.xn, 8u * ch, d.H, w);
            bad |= image_chunk<KIND>(ch, w, lds, sxw, 0u, 0u);
        }
        if (bad && lead && slot == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);  // every workgroup's image is the same
    }
    __syncthreads();
    const int32_t id = routed ? sel_id : (int32_t)d.E;
    // an invalid route selects no organ (the down kernel skips it too)
    const bool ok = !routed || (id >= 0 && (uint32_t)id < d.E);
    if (!ok) {
        if (lead && threadIdx.x == 0) atomicOr(ws.status, HK_DEVERR_ROUTE);
        return;
    }
    // the slot's organs from the id: no table load between the route and the weights
    const OrganView g = routed ? advance_view(g0, (uint32_t)id, L.stride) : g0;
    // mixed: this workgroup's share of the slot's down-organ step headers,
    // loaded now and stored at the end (for the down kernel, which then
    // needs no route before its weights)
    uint4 dh = make_uint4(0u, 0u, 0u, 0u);
    uint32_t dhi = 0xFFFFFFFFu;
    if constexpr (KIND == HK_MIXED) {
        const OrganView dn = routed ? advance_view(dn0, (uint32_t)id, L.stride) : dn0;
        const uint32_t nh = dn.n_tiles * dn.steps, share = (nh + gridDim.x - 1u) / gridDim.x;
        const uint32_t i = T * share + threadIdx.x;
        if (threadIdx.x < share && i < nh) {
            dh = ldg(dn.hdr + i);
            dhi = slot * moe_dn_hdr_stride(d.H, d.Imax) + i;
        }
    }
    if (T >= g.n_tiles) {
        if (dhi != 0xFFFFFFFFu) ws.dn_hdr[dhi] = dh;
        return;
    }
    const OrganView u = routed ? advance_view(u0, (uint32_t)id, L.stride) : u0;
    const uint32_t per = (S + 3u) / 4u;
    const uint32_t s0 = min(wave * per, S), n = min(s0 + per, S) - s0;
    Frag<KIND, 2> f[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        if ((uint32_t)k < n) {
            fetch_one<KIND, 2>(g, T, s0 + k, lane, f[k], 0);
            fetch_one<KIND, 2>(u, T, s0 + k, lane, f[k], 1);
        }
    }
    const int E = 0;  // the route kernel's image is built with E = 0
    const ImageA A{lds, a_lane_offset(lane)};
    const float* SX = reinterpret_cast<const float*>(lds + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    float acc[2] = {0.0f, 0.0f};
    for (uint32_t it = 0; it < n; it += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            if (it + k >= n) break;
            compute_step<KIND, 2>(f[k], s0 + it + k, A, SX, q, acc);
            const uint32_t nx = it + D + k;
            if (nx < n) {
                fetch_one<KIND, 2>(g, T, s0 + nx, lane, f[k], 0);
                fetch_one<KIND, 2>(u, T, s0 + nx, lane, f[k], 1);
            }
        }
    }
    float* part = reinterpret_cast<float*>(lds + ib);  // [wave][gate 16 | up 16]
    const float gs = tile_row_sum(acc[0]), us = tile_row_sum(acc[1]);
    if (lane < 16) {
        part[wave * 32u + lane] = gs;
        part[wave * 32u + 16u + lane] = us;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        float gv = 0.f, uv = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            gv += part[w * 32 + threadIdx.x];
            uv += part[w * 32 + 16 + threadIdx.x];
        }
        gv = ldexpf(gv, -E);
        uv = ldexpf(uv, -E);
        const uint32_t row = T * 16u + threadIdx.x;
        if (row < g.rows) ws.act[(size_t)slot * d.Imax + row] = (gv / (1.0f + expf(-gv))) * uv;
    }
    if (dhi != 0xFFFFFFFFu) ws.dn_hdr[dhi] = dh;
}

// h_in and h_out may be the same vector (each row is read, then written, by
// one thread); the route (ids, weights) in slot order; slot d.K = the shared
// expert.  A slot with an invalid id contributes nothing.  Each wave owns one
// slot: it stages the slot's activations in LDS (loads issued before the
// route is read), issues its weight steps, and builds the slot's x image with
// E = 0 while they are in flight (image_wave: no barrier, no gather pass).
template <int KIND, int D, bool HDR_WS>
__global__ void __launch_bounds__(1024) moe_down_kernel(MoeDims d, MoeLayerDev L, const float* h_in, float* h_out,
                                                        MoeWs ws, const int32_t* __restrict__ ids,
                                                        const float* __restrict__ wts, uint32_t img_stride) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t T = blockIdx.x, slots = blockDim.x >> 6;
    const uint32_t slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const bool routed = slot < d.K;
    // the route and the slot's base view (scalar loads), the residual this
    // thread adds at the end and the slot's activations (sized from the dims,
    // so they wait for no route) all in flight together
    const OrganView o0 = L.table[routed ? 2u : d.E * 3u + 2u];
    const int32_t idr = __builtin_amdgcn_readfirstlane(ids[min(slot, d.K - 1u)]);  // no branch before the load
    // HDR_WS (mixed, per-layer launches): the slot's step headers as the
    // gate/up kernel copied them (tile T's at T * steps of the slot's own
    // down organ: the routed and shared intermediates may differ in steps),
    // loaded with the route instead of after it
    uint4 hws[D];
    if constexpr (HDR_WS) {
        const uint32_t ns = n_steps_for(HK_MIXED, routed ? d.I : d.SI);
#pragma unroll
        for (int k = 0; k < D; ++k)
            hws[k] = ldg(ws.dn_hdr + (size_t)slot * moe_dn_hdr_stride(d.H, d.Imax) + T * ns + min((uint32_t)k, ns - 1u));
    }
    const int32_t id = routed ? idr : (int32_t)d.E;
    const uint32_t row = T * 16u + threadIdx.x;
    const float hres = h_in[min(row, d.H - 1u)];  // every lane loads (no branch); threads 0-15 use it
    uint8_t* img = lds + (size_t)slot * img_stride;
    const uint32_t kst = x_image_cols<KIND>(n_steps_for(KIND, d.Imax)), acols = routed ? d.I : d.SI;
    float* xs = reinterpret_cast<float*>(lds + (size_t)slots * (img_stride + 64u)) + (size_t)slot * kst;
    copy16_to_lds<4>(reinterpret_cast<uint4*>(xs), reinterpret_cast<const uint4*>(ws.act + (size_t)slot * d.Imax),
                     acols / 4u, (uint32_t)lane, 64u);
    const bool ok = !routed || (id >= 0 && (uint32_t)id < d.E);
    const OrganView o = routed ? advance_view(o0, ok ? (uint32_t)id : 0u, L.stride) : o0;
    const bool active = ok && T < o.n_tiles;
    const uint32_t S = active ? o.steps : 0u;
    Frag<KIND, 1> f[D];
#pragma unroll
    for (int k = 0; k < D; ++k)
        if ((uint32_t)k < S) {
            if constexpr (HDR_WS) fetch_mixed<1>(o, hws[k], lane, f[k], 0);
            else fetch_one<KIND, 1>(o, T, (uint32_t)k, lane, f[k], 0);
        }
    const float wgt = !active ? 0.0f : (slot < d.K ? wts[slot] : ws.gate[1]);
    if (active) {
        bool bad = false;
        image_wave<KIND>((uint32_t)lane, xs, o.cols, img,
                         reinterpret_cast<float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE), 0u,
                         S * tile_step_cols(KIND) / 8u, &bad);
        if (__ballot(bad) != 0 && lane == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
    const ImageA A{img, a_lane_offset(lane)};
    const float* SX = reinterpret_cast<const float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    float acc[1] = {0.0f};
    for (uint32_t it = 0; it < S; it += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            if (it + k >= S) break;
            compute_step<KIND, 1>(f[k], it + k, A, SX, q, acc);
            const uint32_t nx = it + D + k;
            if (nx < S) fetch_one<KIND, 1>(o, T, nx, lane, f[k], 0);
        }
    }
    float* part = reinterpret_cast<float*>(lds + (size_t)slots * img_stride);  // [slots][16]
    const float y = tile_row_sum(acc[0]);
    if (lane < 16) part[slot * 16u + lane] = active ? y * wgt : 0.0f;
    __syncthreads();
    if (threadIdx.x < 16) {
        // combined += out_r * w_r in route order, then += gate * shared; out = h + combined
        float comb = 0.0f;
        for (uint32_t r = 0; r < slots; ++r) comb += part[r * 16u + threadIdx.x];
        if (row < d.H) h_out[row] = hres + comb;
    }
}

// Gate/up of one (16-row tile, slot) of the expert block for caller routes
// (BackendMoe::moe_block): slot r < d.K takes route_ids[r], slot d.K the
// shared expert.  The slot's first weight steps are issued as soon as its id
// is read; the workgroup then builds the x image of x itself (no route
// kernel) and, for the shared slot, tile 0 forms the shared gate
// sigmoid(wg . x) (1 without a gate).
template <int KIND, int D>
__global__ void __launch_bounds__(256) moe_block_gate_up_kernel(MoeDims d, MoeLayerDev L, MoeWs ws,
                                                                const int32_t* __restrict__ route_ids,
                                                                const float* __restrict__ x) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[4];
    const uint32_t slot = blockIdx.y, T = blockIdx.x;
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool routed = slot < d.K;
    const uint32_t base = routed ? 0u : d.E * 3u;
    const OrganView g0 = L.table[base], u0 = L.table[base + 1u];
    const int32_t id = routed ? __builtin_amdgcn_readfirstlane(route_ids[slot]) : (int32_t)d.E;
    // an invalid route selects no organ (the down kernel skips it too)
    const bool ok = !routed || (id >= 0 && (uint32_t)id < d.E);
    if (!ok) {
        if (T == 0 && threadIdx.x == 0) atomicOr(ws.status, HK_DEVERR_ROUTE);
        return;
    }
    const OrganView g = routed ? advance_view(g0, (uint32_t)id, L.stride) : g0;
    if (T >= g.n_tiles) return;
    const OrganView u = routed ? advance_view(u0, (uint32_t)id, L.stride) : u0;
    const uint32_t S = n_steps_for(KIND, d.H), ib = (uint32_t)x_lds_bytes<KIND>(S);
    const uint32_t per = (S + 3u) / 4u;
    const uint32_t s0 = min(wave * per, S), n = min(s0 + per, S) - s0;
    Frag<KIND, 2> f[D];
#pragma unroll
    for (int k = 0; k < D; ++k) {
        if ((uint32_t)k < n) {
            fetch_one<KIND, 2>(g, T, s0 + k, lane, f[k], 0);
            fetch_one<KIND, 2>(u, T, s0 + k, lane, f[k], 1);
        }
    }
    if (!routed && T == 0) {
        // the shared-expert gate: sigmoid(wg . x), a block dot over 8-column chunks
        float acc = 0.0f;
        if (L.gate_w) {
            for (uint32_t c = 8u * threadIdx.x; c < d.H; c += 8u * blockDim.x) {
                float4 xv[2], wv[2];
                load_chunk(x, c, d.H, xv);
                load_chunk(L.gate_w, c, d.H, wv);
                acc += dot4(xv[0], wv[0]) + dot4(xv[1], wv[1]);
            }
        }
        const float lg = block_sum(acc, red);
        if (threadIdx.x == 0) ws.gate[1] = L.gate_w ? 1.0f / (1.0f + expf(-lg)) : 1.0f;
    }
    bool bad = false;
    XChunks<1> xc;
    load_x<1>(BlockTeam{}, x, d.H, xc);
    float* xq = reinterpret_cast<float*>(lds + ib + 4u * 32u * sizeof(float));
    const int E = x_image<KIND, 1>(BlockTeam{}, xc, x, d.H, S, lds, xq, 0u, red, &bad);
    if (bad && threadIdx.x == 0 && T == 0 && slot == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    const ImageA A{lds, a_lane_offset(lane)};
    const float* SX = reinterpret_cast<const float*>(lds + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    float acc[2] = {0.0f, 0.0f};
    for (uint32_t it = 0; it < n; it += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            if (it + k >= n) break;
            compute_step<KIND, 2>(f[k], s0 + it + k, A, SX, q, acc);
            const uint32_t nx = it + D + k;
            if (nx < n) {
                fetch_one<KIND, 2>(g, T, s0 + nx, lane, f[k], 0);
                fetch_one<KIND, 2>(u, T, s0 + nx, lane, f[k], 1);
            }
        }
    }
    float* part = reinterpret_cast<float*>(lds + ib);  // [wave][gate 16 | up 16]
    const float gs = tile_row_sum(acc[0]), us = tile_row_sum(acc[1]);
    if (lane < 16) {
        part[wave * 32u + lane] = gs;
        part[wave * 32u + 16u + lane] = us;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
        float gv = 0.f, uv = 0.f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            gv += part[w * 32 + threadIdx.x];
            uv += part[w * 32 + 16 + threadIdx.x];
        }
        gv = ldexpf(gv, -E);
        uv = ldexpf(uv, -E);
        const uint32_t row = T * 16u + threadIdx.x;
        if (row < g.rows) ws.act[(size_t)slot * d.Imax + row] = (gv / (1.0f + expf(-gv))) * uv;
    }
}

size_t moe_block_gate_up_lds_bytes(int kind, uint32_t H) {
    return moe_gate_up_lds_bytes(kind, H) + (size_t)std::min<uint32_t>(stage_floats(kind, H), 2048u) * sizeof(float);
}

template <int KIND>
static hipError_t launch_block(const MoeDims& d, const MoeLayerDev& L, const int32_t* route_ids,
                               const float* route_weights, const float* x, float* out, const MoeWs& ws,
                               hipStream_t s) {
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    const uint32_t gu_tiles = n_tiles_for(d.has_shared ? max(d.I, d.SI) : d.I);
    const uint32_t img_stride = (uint32_t)moe_img_bytes(KIND, d.Imax);
    hipLaunchKernelGGL((moe_block_gate_up_kernel<KIND, 4>), dim3(gu_tiles, slots), dim3(256),
                       moe_block_gate_up_lds_bytes(KIND, d.H), s, d, L, ws, route_ids, x);
    hipLaunchKernelGGL((moe_down_kernel<KIND, 4, false>), dim3(n_tiles_for(d.H)), dim3(64u * slots),
                       moe_down_lds_bytes(KIND, d.Imax, slots), s, d, L, out, out, ws, route_ids, route_weights,
                       img_stride);
    return hipGetLastError();
}

hipError_t launch_moe_block(int kind, const MoeDims& d, const MoeLayerDev& L, const int32_t* route_ids,
                            const float* route_weights, const float* x, float* out, const MoeWs& ws, hipStream_t s) {
    if (kind == HK_Q4) return launch_block<HK_Q4>(d, L, route_ids, route_weights, x, out, ws, s);
    if (kind == HK_MIXED) return launch_block<HK_MIXED>(d, L, route_ids, route_weights, x, out, ws, s);
    return hipErrorInvalidValue;
}

template <int KIND>
static hipError_t launch_layer(const MoeDims& d, const MoeLayerDev& L, const float* h_in, float* h_out,
                               const MoeWs& ws, int32_t* ids_out, float* w_out, hipStream_t s) {
    const uint32_t nrb = (d.E + 3u) / 4u;
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    const uint32_t gu_tiles = n_tiles_for(d.has_shared ? max(d.I, d.SI) : d.I);
    const uint32_t img_stride = (uint32_t)moe_img_bytes(KIND, d.Imax);
    hipLaunchKernelGGL(moe_route_kernel<KIND>, dim3(nrb + 1u), dim3(256), moe_route_lds_bytes(KIND, d.H), s, d, L,
                       h_in, ws);
    const dim3 gg(gu_tiles, slots);
    const size_t gl = moe_gate_up_lds_bytes(KIND, d.H);
    if (d.E <= 512)
        hipLaunchKernelGGL((moe_gate_up_kernel<KIND, 4, 8>), gg, dim3(256), gl, s, d, L, ws, ids_out, w_out);
    else if (d.E <= 1024)
        hipLaunchKernelGGL((moe_gate_up_kernel<KIND, 4, 16>), gg, dim3(256), gl, s, d, L, ws, ids_out, w_out);
    else if (d.E <= 2048)
        hipLaunchKernelGGL((moe_gate_up_kernel<KIND, 4, 32>), gg, dim3(256), gl, s, d, L, ws, ids_out, w_out);
    else
        hipLaunchKernelGGL((moe_gate_up_kernel<KIND, 4, 64>), gg, dim3(256), gl, s, d, L, ws, ids_out, w_out);
    // mixed: the down weights follow the headers the gate/up kernel copied
    // (when every step of the down organs is in the first fetch)
    if (KIND == HK_MIXED && n_steps_for(HK_MIXED, d.Imax) <= 4u)
        hipLaunchKernelGGL((moe_down_kernel<KIND, 4, KIND == HK_MIXED>), dim3(n_tiles_for(d.H)), dim3(64u * slots),
                           moe_down_lds_bytes(KIND, d.Imax, slots), s, d, L, h_in, h_out, ws, ws.ids, ws.weights,
                           img_stride);
    else
        hipLaunchKernelGGL((moe_down_kernel<KIND, 4, false>), dim3(n_tiles_for(d.H)), dim3(64u * slots),
                           moe_down_lds_bytes(KIND, d.Imax, slots), s, d, L, h_in, h_out, ws, ws.ids, ws.weights,
                           img_stride);
    return hipGetLastError();
}

hipError_t launch_moe_layer(int kind, const MoeDims& d, const MoeLayerDev& L, const float* h_in, float* h_out,
                            const MoeWs& ws, int32_t* ids_out, float* w_out, hipStream_t s) {
    if (kind == HK_Q4) return launch_layer<HK_Q4>(d, L, h_in, h_out, ws, ids_out, w_out, s);
    if (kind == HK_MIXED) return launch_layer<HK_MIXED>(d, L, h_in, h_out, ws, ids_out, w_out, s);
    return hipErrorInvalidValue;
}

}  // namespace hk
