// hk_moe.hip -- one MoE decode layer (moe_suffix) at batch 1 on device data.
//
// Four stream-ordered launches, no host round trip; the routed expert ids
// are read from device memory by the expert kernels
// (run_qwen80_routed_expert_table,
//  crates/hawking-core/src/model/qwen80_device_expert_table.rs:1204-1247):
//   1. router:  xn = RMSNorm(1+w)(h) (recomputed per block, block 0 stores it);
//               logits = Wr xn; shared-gate logit = wg . xn
//   2. top-k:   softmax, top-k, renormalise; gate = sigmoid(gate logit)
//   3. gate/up: act[slot] = silu(gate_e xn) * (up_e xn) for the K routed
//               slots and the shared expert (SwiGLU fused)
//   4. down:    out = h + sum_r w_r (down_r act_r)  (route order)
//                       + gate * (down_shared act_shared)
#include "hk_internal.h"
#include "hk_moe.h"
#include "hk_router_dev.h"
#include "hk_rowdot.h"

namespace hk {

__device__ __forceinline__ float block_inv_rms(const float* __restrict__ h, uint32_t H, float eps,
                                               float* red) {
    float ss = 0.f;
    for (uint32_t c = threadIdx.x; c < H; c += blockDim.x) ss += h[c] * h[c];
    ss = block_sum(ss, red);
    return 1.0f / sqrtf(ss / (float)H + eps);
}

__global__ void __launch_bounds__(256) moe_router_kernel(MoeDims d, MoeLayerDev L,
                                                         const float* __restrict__ h, MoeWs ws) {
    extern __shared__ __align__(16) float xn[];
    __shared__ float red[4];
    const float inv = block_inv_rms(h, d.H, d.eps, red);
    for (uint32_t c = threadIdx.x; c < d.H; c += blockDim.x) {
        const float v = h[c] * inv * (1.0f + L.norm_w[c]);
        xn[c] = v;
        if (blockIdx.x == 0) ws.xn[c] = v;
    }
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    CanonView o{};
    o.kind = HK_F32;
    o.cols = d.H;
    if (row < d.E) {
        o.rows = d.E;
        o.dense = L.router_w;
        const float acc = wave_sum(row_dot_partial<HK_F32>(o, row, xn, lane));
        if (lane == 0) ws.logits[row] = acc;
    } else if (row == d.E && L.gate_w) {
        o.rows = 1;
        o.dense = L.gate_w;
        const float acc = wave_sum(row_dot_partial<HK_F32>(o, 0, xn, lane));
        if (lane == 0) ws.gate[0] = acc;
    }
}

__global__ void __launch_bounds__(256) moe_topk_kernel(MoeDims d, int has_gate, MoeWs ws) {
    extern __shared__ float p[];
    __shared__ float redf[4];
    __shared__ ArgBest reda[4];
    softmax_topk_block(ws.logits, d.E, d.K, 0.0f, 1, p, ws.ids, ws.weights, ws.status, redf, reda);
    if (threadIdx.x == 0) ws.gate[1] = has_gate ? 1.0f / (1.0f + expf(-ws.gate[0])) : 1.0f;
}

template <int KIND>
__global__ void __launch_bounds__(256) moe_gate_up_kernel(MoeDims d, MoeLayerDev L, MoeWs ws) {
    extern __shared__ __align__(16) float xn[];
    for (uint32_t c = threadIdx.x; c < d.H; c += blockDim.x) xn[c] = ws.xn[c];
    __syncthreads();
    const uint32_t slot = blockIdx.y;
    const bool shared = slot >= d.K;
    const uint32_t e = shared ? d.E : (uint32_t)ws.ids[slot];
    if (e > d.E || (!shared && e == d.E)) {
        // invalid route (non-finite logits): flag it and touch no expert
        if (threadIdx.x == 0) atomicOr(ws.status, HK_DEVERR_ROUTE);
        return;
    }
    const CanonView& g = L.table[e * 3 + 0];
    const CanonView& u = L.table[e * 3 + 1];
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= g.rows) return;
    const float gv = wave_sum(row_dot_partial<KIND>(g, row, xn, lane));
    const float uv = wave_sum(row_dot_partial<KIND>(u, row, xn, lane));
    if (lane == 0) ws.act[(size_t)slot * d.Imax + row] = (gv / (1.0f + expf(-gv))) * uv;
}

template <int KIND>
__global__ void __launch_bounds__(256) moe_down_kernel(MoeDims d, MoeLayerDev L,
                                                       const float* __restrict__ h_in,
                                                       float* __restrict__ h_out, MoeWs ws) {
    extern __shared__ __align__(16) float act[];
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    for (uint32_t i = threadIdx.x; i < slots * d.Imax; i += blockDim.x) act[i] = ws.act[i];
    __syncthreads();
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= d.H) return;
    float combined = 0.0f;
    for (uint32_t r = 0; r < d.K; ++r) {
        const uint32_t e = (uint32_t)ws.ids[r];
        if (e >= d.E) continue;  // flagged by the gate/up kernel
        const CanonView& dn = L.table[e * 3 + 2];
        const float y = wave_sum(row_dot_partial<KIND>(dn, row, act + (size_t)r * d.Imax, lane));
        combined += y * ws.weights[r];
    }
    if (d.has_shared) {
        const CanonView& dn = L.table[d.E * 3 + 2];
        const float y = wave_sum(row_dot_partial<KIND>(dn, row, act + (size_t)d.K * d.Imax, lane));
        combined += y * ws.gate[1];
    }
    if (lane == 0) h_out[row] = h_in[row] + combined;
}

hipError_t launch_moe_layer(int kind, const MoeDims& d, const MoeLayerDev& L, const float* h_in,
                            float* h_out, const MoeWs& ws, hipStream_t s) {
    const size_t xn_bytes = (size_t)d.H * sizeof(float);
    hipLaunchKernelGGL(moe_router_kernel, dim3((d.E + 1 + 3) / 4), dim3(256), xn_bytes, s, d, L, h_in, ws);
    hipLaunchKernelGGL(moe_topk_kernel, dim3(1), dim3(256), (size_t)d.E * sizeof(float), s, d,
                       L.gate_w != nullptr ? 1 : 0, ws);
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    const dim3 gu((d.Imax + 3) / 4, slots);
    const size_t act_bytes = (size_t)slots * d.Imax * sizeof(float);
    if (kind == HK_Q4) {
        hipLaunchKernelGGL(moe_gate_up_kernel<HK_Q4>, gu, dim3(256), xn_bytes, s, d, L, ws);
        hipLaunchKernelGGL(moe_down_kernel<HK_Q4>, dim3((d.H + 3) / 4), dim3(256), act_bytes, s, d, L,
                           h_in, h_out, ws);
    } else if (kind == HK_MIXED) {
        hipLaunchKernelGGL(moe_gate_up_kernel<HK_MIXED>, gu, dim3(256), xn_bytes, s, d, L, ws);
        hipLaunchKernelGGL(moe_down_kernel<HK_MIXED>, dim3((d.H + 3) / 4), dim3(256), act_bytes, s, d, L,
                           h_in, h_out, ws);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace hk
