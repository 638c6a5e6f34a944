// hk_router.hip -- device routers: softmax top-k (Qwen3-Next) and noaux_tc
// (DeepSeek-V3).  One 256-thread block per token; ids and weights stay in
// device memory.
//
// Top-k selection with tie_eps == 0 is a parallel lexicographic max over
// (value desc, index asc), which returns exactly what the reference's serial
// strict-'>' scan returns, including on exact ties
// (crates/hawking-core/tests/moe_topk_gate_exact_ties_parity.rs).  With
// tie_eps > 0 the reference rule is order dependent (a later score replaces
// the best only when it beats it by more than eps), so that mode runs the
// serial scan in one thread, as the reference does.
#include "hk_internal.h"
#include "hk_router.h"
#include "hk_router_dev.h"

namespace hk {

__global__ void __launch_bounds__(256) softmax_topk_kernel(const float* __restrict__ logits,
                                                           uint32_t n, uint32_t k, float tie_eps,
                                                           int renorm, int32_t* __restrict__ ids,
                                                           float* __restrict__ weights,
                                                           uint32_t* status) {
    extern __shared__ float p[];
    __shared__ float redf[4];
    __shared__ ArgBest reda[4];
    __shared__ int32_t sel_i[HK_TOPK_MAX];
    __shared__ float sel_v[HK_TOPK_MAX];
    const size_t t = blockIdx.x;
    softmax_topk_block(logits + t * n, n, k, tie_eps, renorm, p, ids + t * k, weights + t * k, status,
                       redf, reda, sel_i, sel_v);
}

// noaux_tc (gravity_glm.rs:447-500) for one token.
__global__ void __launch_bounds__(256) noaux_tc_kernel(const float* __restrict__ logits,
                                                       const float* __restrict__ bias, uint32_t n,
                                                       uint32_t n_group, uint32_t topk_group,
                                                       uint32_t k, int norm, float scaling,
                                                       int32_t* __restrict__ ids,
                                                       float* __restrict__ weights) {
    extern __shared__ float smem[];
    float* score = smem;                 // n
    float* corr = smem + n;              // n
    float* gscore = smem + 2 * n;        // n_group
    uint8_t* allowed = reinterpret_cast<uint8_t*>(smem + 2 * n + n_group);  // n_group
    __shared__ ArgBest reda[4];
    __shared__ int32_t sel_i[HK_TOPK_MAX];
    __shared__ float sel_v[HK_TOPK_MAX];
    const size_t t = blockIdx.x;
    const float* lg = logits + t * n;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float s = 1.0f / (1.0f + expf(-lg[i]));
        score[i] = s;
        corr[i] = s + bias[i];
    }
    __syncthreads();
    const uint32_t per = n / n_group;
    for (uint32_t g = threadIdx.x; g < n_group; g += blockDim.x) {
        // topk_desc(slice, min(2, per)) then the f32 sum of those values
        const float* sl = corr + g * per;
        uint32_t b0 = 0;
        for (uint32_t i = 1; i < per; ++i)
            if (sl[i] > sl[b0]) b0 = i;
        float s = -0.0f + sl[b0];
        if (per >= 2) {
            uint32_t b1 = b0 == 0 ? 1 : 0;
            for (uint32_t i = 0; i < per; ++i)
                if (i != b0 && (sl[i] > sl[b1] || (sl[i] == sl[b1] && i < b1))) b1 = i;
            s = s + sl[b1];
        }
        gscore[g] = s;
        allowed[g] = 0;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (uint32_t c = 0; c < topk_group; ++c) {
            int best = -1;
            for (uint32_t g = 0; g < n_group; ++g) {
                if (allowed[g]) continue;
                if (best < 0 || gscore[g] > gscore[best]) best = (int)g;
            }
            allowed[best] = 1;
        }
    }
    __syncthreads();
    // choice = corrected score inside the chosen groups, -inf elsewhere; an
    // expert already taken is marked by a NaN in corr and skipped.
    for (uint32_t r = 0; r < k; ++r) {
        ArgBest a{0.f, -1};
        for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
            const float c = corr[i];
            if (isnan(c)) continue;
            const float v = allowed[i / per] ? c : -INFINITY;
            if (a.i < 0 || better(v, (int)i, a.v, a.i)) {
                a.v = v;
                a.i = (int)i;
            }
        }
        const ArgBest b = block_argmax(a, reda);
        if (threadIdx.x == 0) {
            sel_i[r] = b.i;
            sel_v[r] = score[b.i];
            corr[b.i] = __builtin_nanf("");
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        if (norm) {
            float total = -0.0f;
            for (uint32_t r = 0; r < k; ++r) total += sel_v[r];
            total = total + 1e-20f;
            for (uint32_t r = 0; r < k; ++r) sel_v[r] = sel_v[r] / total;
        }
        for (uint32_t r = 0; r < k; ++r) sel_v[r] = sel_v[r] * scaling;
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < k; r += blockDim.x) {
        ids[t * k + r] = sel_i[r];
        weights[t * k + r] = sel_v[r];
    }
}

hipError_t launch_softmax_topk(const float* logits, uint32_t n_tokens, uint32_t n, uint32_t k,
                               float tie_eps, int renorm, int32_t* ids, float* weights,
                               uint32_t* status, hipStream_t s) {
    hipLaunchKernelGGL(softmax_topk_kernel, dim3(n_tokens), dim3(256), n * sizeof(float), s, logits, n,
                       k, tie_eps, renorm, ids, weights, status);
    return hipGetLastError();
}

hipError_t launch_noaux_tc(const float* logits, const float* bias, uint32_t n_tokens, uint32_t n,
                           uint32_t n_group, uint32_t topk_group, uint32_t k, int norm,
                           float scaling, int32_t* ids, float* weights, hipStream_t s) {
    const size_t shm = (2 * (size_t)n + n_group) * sizeof(float) + n_group + 16;
    hipLaunchKernelGGL(noaux_tc_kernel, dim3(n_tokens), dim3(256), shm, s, logits, bias, n, n_group,
                       topk_group, k, norm, scaling, ids, weights);
    return hipGetLastError();
}

}  // namespace hk
