// hk_moe.h -- device-side structures of the MoE decode step.
#pragma once

#include "hk_internal.h"

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
    uint8_t* img;      // x image (E = 0) of RMSNorm(h) for the gate/up organs
    uint32_t* status;  // device error bits
};

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

// ids_out / w_out (device, top_k each) may be null.
hipError_t launch_moe_layer(int kind, const MoeDims& d, const MoeLayerDev& L, const float* h_in,
                            float* h_out, const MoeWs& ws, int32_t* ids_out, float* w_out, hipStream_t s);

// ------------------------------------------------------------------ batched (noaux_tc) block

constexpr uint32_t MOE_BATCH_MAX_TOKENS = 64;
constexpr uint32_t MOE_BATCH_MAX_EXPERTS = 512;
constexpr uint32_t MOE_BATCH_ROUTER_COLS = 256;  // router columns per split-K workgroup

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
    float* x32;          // [T x H]
    uint8_t* ximg;       // [T] x images of x (stride ximg_stride)
    int32_t* ximg_e;     // [T]
    float* part;         // [S x T x E] router partials
    int32_t* ids;        // [T x K] route order
    float* w;            // [T x K]
    int32_t* order;      // [T x K] slots of each token in ascending expert id
    uint4* active;       // [E + 1]
    uint32_t* n_active;  // [1]
    uint32_t* members;   // [T*K + T] pair ids, grouped by active expert
    float* act;          // [pairs x Imax]
    uint8_t* aimg;       // [pairs] x images of the activations (stride aimg_stride)
    int32_t* aimg_e;     // [pairs]
    float* ybuf;         // [pairs x H] weighted expert outputs
    uint32_t ximg_stride, aimg_stride;
    uint32_t* status;
};

size_t moe_batch_img_bytes(uint32_t cols);  // Q4 x image of `cols` columns
hipError_t launch_moe_batch(const MoeBatchDims& d, const MoeLayerDev& L, const float* bias, const uint16_t* x_bf16,
                            float* y, const MoeBatchWs& ws, int32_t* ids_out, float* w_out, hipStream_t s);

}  // namespace hk
