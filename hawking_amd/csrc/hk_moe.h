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

// One layer's device weights; table holds (E+1)*3 organ views:
// [expert*3 + {0: gate, 1: up, 2: down}], expert E = shared expert.
struct MoeLayerDev {
    const float* norm_w;
    const float* router_w;
    const float* gate_w;   // shared-expert gate, may be null
    const CanonView* table;
};

// Per-model device workspace.
struct MoeWs {
    float* xn;        // [H]
    float* logits;    // [E]
    int32_t* ids;     // [K]
    float* weights;   // [K]
    float* gate;      // [2]: shared-gate logit, shared-gate value
    float* act;       // [(K+1) * Imax]
    uint32_t* status; // device error bits
};

hipError_t launch_moe_layer(int kind, const MoeDims& d, const MoeLayerDev& L, const float* h_in,
                            float* h_out, const MoeWs& ws, hipStream_t s);

}  // namespace hk
