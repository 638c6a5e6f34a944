// hk_head.hip -- the device-side terminal head: final RMSNorm(1+w), the
// lm_head GEMV on the packed engine, and the greedy pick, so the token id is
// produced on the device (terminal_greedy,
// model/qwen80_mixed_hybrid_decode.rs:3754-3790, without its host_sample
// fallback).
#include "hk_internal.h"
#include "hk_router.h"

namespace hk {

// xn = h * (1 / sqrt(mean(h^2) + eps)) * (1 + w), multiplied left to right as
// source_qwen80_residual_rms_norm (model/qwen80_complete_runtime.rs:6778-6797);
// the sum of squares is a block reduction.  A non-finite xn sets the status
// and marks the token -1 (the pick keeps it), else the token slot is 0.
__global__ void __launch_bounds__(1024) head_norm_kernel(const float* __restrict__ h, const float* __restrict__ w,
                                                         uint32_t n, float eps, float* __restrict__ xn,
                                                         int32_t* __restrict__ token, uint64_t* __restrict__ key,
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
    const int any_bad = __syncthreads_or(bad ? 1 : 0);
    if (tid == 0) {
        token[0] = any_bad ? -1 : 0;
        key[0] = 0ull;
        if (any_bad) atomicOr(status, HK_DEVERR_NONFINITE);
    }
}

// Order key of logit i: NaN is 0 (never chosen); -0 counts as +0; a larger
// value, then a lower index, gives a larger key.
__device__ __forceinline__ uint64_t greedy_key(float v, uint32_t i) {
    if (v != v) return 0ull;
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(~i);
}

constexpr uint32_t HEAD_PER_BLOCK = 256u * 16u;  // logits per block of the pick (16 per thread)

// Each block reduces HEAD_PER_BLOCK logits (loads issued together) to its
// largest key and folds it into *key with one atomic max.
__global__ void __launch_bounds__(256) head_argmax_kernel(const float* __restrict__ logits, uint32_t n_valid,
                                                          uint64_t* __restrict__ key) {
    __shared__ uint64_t red[4];
    const uint32_t tid = threadIdx.x, b0 = blockIdx.x * HEAD_PER_BLOCK;
    float v[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const uint32_t i = b0 + tid + 256u * (uint32_t)j;
        v[j] = i < n_valid ? logits[i] : __uint_as_float(0x7FC00000u);  // NaN: never chosen
    }
    uint64_t best = 0;
#pragma unroll
    for (int j = 0; j < 16; ++j) best = max(best, greedy_key(v[j], b0 + tid + 256u * (uint32_t)j));
    for (int off = 32; off; off >>= 1) best = max(best, (uint64_t)__shfl_xor((unsigned long long)best, off, 64));
    if ((tid & 63) == 0) red[tid >> 6] = best;
    __syncthreads();
    if (tid == 0) {
        best = max(max(red[0], red[1]), max(red[2], red[3]));
        if (best) atomicMax(reinterpret_cast<unsigned long long*>(key), (unsigned long long)best);
    }
}

// The lowest index of the largest non-NaN logit among the first n_valid (the
// reference's scan keeps the first maximum), or -1 and the status bit when
// that logit is not finite or there is none; a token the norm marked -1
// stays -1.  The key is left zeroed for the next call.
__global__ void head_pick_kernel(uint64_t* __restrict__ key, int32_t* __restrict__ token, uint32_t* status) {
    if (threadIdx.x == 0) {
        const uint64_t best = key[0];
        key[0] = 0ull;
        key[1] = 0ull;
        const uint32_t ord = (uint32_t)(best >> 32);
        const float v = __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
        const bool ok = best != 0ull && isfinite(v) && token[0] != -1;
        token[0] = ok ? (int32_t)(~(uint32_t)best) : -1;
        if (!ok) atomicOr(status, HK_DEVERR_NONFINITE);
    }
}

hipError_t launch_head_norm(const float* h, const float* w, uint32_t n, float eps, float* xn, int32_t* token,
                            uint64_t* key, uint32_t* status, hipStream_t s) {
    hipLaunchKernelGGL(head_norm_kernel, dim3(1), dim3(1024), 0, s, h, w, n, eps, xn, token, key, status);
    return hipGetLastError();
}

hipError_t launch_head_argmax(const float* logits, uint32_t n_valid, uint64_t* key, int32_t* token, uint32_t* status,
                              hipStream_t s) {
    hipLaunchKernelGGL(head_argmax_kernel, dim3((n_valid + HEAD_PER_BLOCK - 1) / HEAD_PER_BLOCK), dim3(256), 0, s,
                       logits, n_valid, key);
    hipLaunchKernelGGL(head_pick_kernel, dim3(1), dim3(64), 0, s, key, token, status);
    return hipGetLastError();
}

}  // namespace hk
