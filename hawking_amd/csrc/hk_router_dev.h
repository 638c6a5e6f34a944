// hk_router_dev.h -- block-level device helpers for routers (top-k,
// reductions), shared by the router and MoE kernels.
#pragma once

#include "hk_internal.h"
#include "hk_router.h"

namespace hk {

struct ArgBest {
    float v;
    int i;
};

__device__ __forceinline__ bool better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// Block-wide lexicographic argmax over candidates with i >= 0; i = -1 is "none".
__device__ ArgBest block_argmax(ArgBest a, ArgBest* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        const float ov = __shfl_xor(a.v, off, 64);
        const int oi = __shfl_xor(a.i, off, 64);
        if (oi >= 0 && (a.i < 0 || better(ov, oi, a.v, a.i))) {
            a.v = ov;
            a.i = oi;
        }
    }
    if (lane == 0) lds[wave] = a;
    __syncthreads();
    ArgBest b = lds[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); ++w) {
        const ArgBest c = lds[w];
        if (c.i >= 0 && (b.i < 0 || better(c.v, c.i, b.v, b.i))) b = c;
    }
    __syncthreads();
    return b;
}

__device__ float block_sum(float v, float* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_sum(v);
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t += lds[w];
    __syncthreads();
    return t;
}

__device__ float block_max(float v, float* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) lds[wave] = v;
    __syncthreads();
    float t = -INFINITY;
    for (int w = 0; w < (int)(blockDim.x >> 6); ++w) t = fmaxf(t, lds[w]);
    __syncthreads();
    return t;
}

// Softmax top-k over one token's logits, p and taken in LDS.  renorm = 1:
// source_qwen80_topk_router (divide by the sum, renormalise by the selected
// sum); renorm = 0: topk_softmax_batch (multiply by 1/sum, raw probs).
__device__ void softmax_topk_block(const float* __restrict__ logits, uint32_t n, uint32_t k,
                                   float tie_eps, int renorm, float* p, int32_t* ids_out,
                                   float* w_out, uint32_t* status, float* redf, ArgBest* reda) {
    float m = -INFINITY;
    uint32_t bad = 0;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float v = logits[i];
        if (!isfinite(v)) bad = 1;
        m = fmaxf(m, v);
    }
    if (bad && status) atomicOr(status, HK_DEVERR_NONFINITE);
    m = block_max(m, redf);
    float local = 0.f;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
        const float e = expf(logits[i] - m);
        p[i] = e;
        local += e;
    }
    const float sum = block_sum(local, redf);
    const float inv = 1.0f / sum;
    for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) p[i] = renorm ? p[i] / sum : p[i] * inv;
    __syncthreads();
    if (tie_eps > 0.0f) {
        if (threadIdx.x == 0) {
            for (uint32_t r = 0; r < k; ++r) {
                uint32_t bi = 0;
                float bv = -INFINITY;
                for (uint32_t i = 0; i < n; ++i) {
                    const float v = p[i];
                    const bool finite_pair = isfinite(bv) && isfinite(v);
                    const bool tied = finite_pair && fabsf(v - bv) <= tie_eps;
                    if ((v > bv && !tied) || (tied && i < bi)) {
                        bi = i;
                        bv = v;
                    }
                }
                ids_out[r] = (int32_t)bi;
                w_out[r] = bv;
                p[bi] = -INFINITY;
            }
        }
    } else {
        for (uint32_t r = 0; r < k; ++r) {
            ArgBest a{-INFINITY, -1};
            for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
                const float v = p[i];
                if (v != -INFINITY && (a.i < 0 || better(v, (int)i, a.v, a.i))) {
                    a.v = v;
                    a.i = (int)i;
                }
            }
            const ArgBest b = block_argmax(a, reda);
            if (threadIdx.x == 0) {
                ids_out[r] = b.i;
                w_out[r] = b.v;
                if (b.i >= 0) p[b.i] = -INFINITY;
            }
            __syncthreads();
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && renorm) {
        float sel = -0.0f;
        for (uint32_t r = 0; r < k; ++r) sel += w_out[r];
        for (uint32_t r = 0; r < k; ++r) w_out[r] = w_out[r] / sel;
    }
    __syncthreads();
}

}  // namespace hk
