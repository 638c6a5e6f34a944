// hk_moe.h -- device-side structures of the MoE decode step.
#pragma once

#include "hk_internal.h"
#include "hk_tile.h"

namespace hk {

struct MoeDims {
    uint32_t H;      // hidden
    uint32_t I;      // routed expert intermediate
    uint32_t SI;     // shared expert intermediate (0 = none)
    uint32_t Imax;   // max(I, SI): stride of the activation slots
    uint32_t E;      // routed experts
    uint32_t K;      // top-k
    int32_t has_shared;
    float eps;
    float tie_eps;   // router tie window (route_tie_epsilon); 0 = strict '>'
};

// One layer's device weights; table holds (E+1)*3 tiled organ views:
// [expert*3 + {0: gate, 1: up, 2: down}], expert E = shared expert.  The
// routed experts sit at a uniform stride in the layer's slab (each
// projection placed with the layer's largest layout of it), so routed expert
// e's views are expert 0's with every section pointer advanced by
// e * stride: a kernel loads table[p] (or the shared expert's entry) when it
// starts, in parallel with its other loads, and forms the routed views from
// the route id with no dependent table load.
struct MoeLayerDev {
    const float* norm_w;
    const float* router_w;
    const float* gate_w;   // shared-expert gate, may be null
    const OrganView* table;
    uint64_t stride;
};

// View v (expert 0's, projection p) advanced to routed expert e.
__device__ __forceinline__ OrganView advance_view(OrganView v, uint32_t e, uint64_t stride) {
    const size_t off = (size_t)e * stride;
    v.data += off;
    v.scales = reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(v.scales) + off);
    v.hdr = reinterpret_cast<const uint4*>(reinterpret_cast<const uint8_t*>(v.hdr) + off);
    return v;
}

// Per-model device workspace.
struct MoeWs {
    float* logits;     // [E]
    int32_t* ids;      // [K]
    float* weights;    // [K]
    float* gate;       // [2]: shared-gate logit, shared-gate value
    float* act;        // [(K+1) * Imax]
    float* xn;         // [H] RMSNorm(1+w)(h): the gate/up kernel builds its x image (E = 0) from it
    uint4* dn_hdr;     // [slots][moe_dn_hdr_stride]: the step headers of each slot's down organ (mixed), copied
                       // by the gate/up kernel so the down kernel needs no route before them
    uint32_t* status;  // device error bits
};

// Headers per slot of the down organs (hidden rows, Imax columns).
__host__ __device__ inline uint32_t moe_dn_hdr_stride(uint32_t H, uint32_t Imax) {
    return n_tiles_for(H) * n_steps_for(HK_MIXED, Imax);
}

// Bytes of the gate/up x image and of the down kernel's LDS.
size_t moe_img_bytes(int kind, uint32_t H);
size_t moe_down_lds_bytes(int kind, uint32_t Imax, uint32_t slots);
size_t moe_route_lds_bytes(int kind, uint32_t H);
size_t moe_gate_up_lds_bytes(int kind, uint32_t H);

// The expert block for caller routes (d.K = n_routes, d.has_shared = the
// shared slot included): out += sum_r w_r mlp_r(x) (+ g mlp_shared(x)).
size_t moe_block_gate_up_lds_bytes(int kind, uint32_t H);
hipError_t launch_moe_block(int kind, const MoeDims& d, const MoeLayerDev& L, const int32_t* route_ids,
                            const float* route_weights, const float* x, float* out, const MoeWs& ws, hipStream_t s);

// Every layer of a token in one persistent cooperative launch (hk_moe_stack.hip).
// Hand-off buffers are flag-tagged 64-bit words {value, tag}, one set per
// layer, all carrying the launch's tag.  Blocks: (E + 3) / 4 + 1 route,
// ng = gu_tiles * slots gate/up, n_tiles(H) down.
constexpr uint32_t RDY_REP = 8;  // replicas of each ready word (readers spread over them)

struct StackArgs {
    MoeDims d;
    const MoeLayerDev* layers;  // [n_layers], device
    uint32_t n_layers;
    uint32_t tag;       // this launch's tag (every hand-off word of the launch carries it)
    const float* h_in;
    float* h_out;
    int32_t* ids;       // [n_layers * K] or null
    float* weights;     // [n_layers * K] or null
    uint32_t* status;
    // hand-off words {value bits, tag}, every layer its own (layer l at l * stride)
    uint64_t* h;        // [H]: the layer's input h
    uint64_t* logits;   // [E + 1]: router logits, then the shared-gate logit
    uint64_t* act;      // [slots * Imax]
    uint32_t hs, ls, as;
    // ready words (value unused), RDY_REP replicas per layer (replica r of
    // layer l at (l RDY_REP + r) * stride): one per producer, stored after
    // its outputs; a reader polls these first and then reads the outputs
    // once (the outputs' own tags decide)
    uint64_t* h_rdy;    // [n_tiles(H)]: down tile T wrote its rows of the layer's h
    uint64_t* l_rdy;    // [E/4 + 1]: route block b wrote its logits
    uint64_t* a_rdy;    // [slots * gu_tiles]: gate/up tile T of a slot wrote its activations
    uint32_t hrs, lrs, ars;
    uint32_t* abort;    // the tag of a launch whose wait ran out
    uint32_t ng, gu_tiles;
    uint32_t spin_limit;  // polls a wait makes before the launch gives up (hk_moe_model_set_stall_polls)
};
size_t moe_stack_lds_bytes(int kind, const MoeDims& d);
// Zeroes n 64-bit words on stream s with a kernel (graph-capture safe).
hipError_t launch_zero_words(uint64_t* p, size_t n, hipStream_t s);
// *fits = false (nothing launched) when the grid cannot be resident at once
// or the shape is outside the kernel's limits; the caller then uses the
// per-layer launches.  launch = false only answers *fits.
hipError_t launch_moe_stack(int kind, const StackArgs& a, int cu_count, hipStream_t s, bool* fits, bool launch = true);

// ids_out / w_out (device, top_k each) may be null.
hipError_t launch_moe_layer(int kind, const MoeDims& d, const MoeLayerDev& L, const float* h_in,
                            float* h_out, const MoeWs& ws, int32_t* ids_out, float* w_out, hipStream_t s);

// ------------------------------------------------------------------ batched (noaux_tc) block

constexpr uint32_t MOE_BATCH_MAX_TOKENS = 64;
constexpr uint32_t MOE_BATCH_MAX_EXPERTS = 512;
#ifndef HK_BATCH_ROUTER_COLS
#define HK_BATCH_ROUTER_COLS 512
#endif
constexpr uint32_t MOE_BATCH_ROUTER_COLS = HK_BATCH_ROUTER_COLS;  // router columns per split-K workgroup

struct MoeBatchDims {
    uint32_t T;         // tokens
    uint32_t H, I, SI;  // hidden, routed / shared intermediate (SI 0 = none)
    uint32_t Imax;
    uint32_t E, K;
    uint32_t n_group, topk_group;
    int32_t norm_topk_prob;
    float scaling;
    uint32_t S;         // router split-K partials
};

// A routed (token, slot) pair is p = t*K + r; the shared expert's pair for
// token t is T*K + t.  active[a] = {expert, first member, members}; entry 0 is
// the shared expert (if any), then the routed experts in ascending id.
struct MoeBatchWs {
    uint8_t* ximg;       // [T] x images of x (stride ximg_stride)
    int32_t* ximg_e;     // [T]
    float* part;         // [S x T x E] router partials
    int32_t* ids;        // [T x K] route order
    float* w;            // [T x K]
    int32_t* rank;       // [T x K] each routed pair's position among its token's slots in ascending expert id
    uint4* active;       // [E + 1]
    uint32_t* n_active;  // [1]
    uint32_t* members;   // [T*K + T] pair ids, grouped by active expert
    float* act;          // [pairs x Imax]
    uint8_t* aimg;       // [pairs] x images of the activations (stride aimg_stride)
    int32_t* aimg_e;     // [pairs]
    float* ybuf;         // [pairs x H] weighted expert outputs: token t's routed ones at rows t K + rank
                         // (ascending expert id), the shared expert's at T K + t
    uint32_t ximg_stride, aimg_stride;
    uint32_t* status;
};

size_t moe_batch_img_bytes(uint32_t cols);  // Q4 x image of `cols` columns
hipError_t launch_moe_batch(const MoeBatchDims& d, const MoeLayerDev& L, const float* bias, const uint16_t* x_bf16,
                            float* y, const MoeBatchWs& ws, int32_t* ids_out, float* w_out, hipStream_t s);

}  // namespace hk
