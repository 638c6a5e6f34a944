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

__device__ __forceinline__ void take_better(ArgBest& a, float ov, int oi) {
    const bool t = (oi >= 0) & ((a.i < 0) | (ov > a.v) | ((ov == a.v) & (oi < a.i)));
    a.v = t ? ov : a.v;
    a.i = t ? oi : a.i;
}

// Wave-wide lexicographic argmax (value desc, index asc) over candidates with
// i >= 0 (i = -1 is "none"), on the DPP network; every lane gets lane 63's
// result.  All 64 lanes must be active.
__device__ __forceinline__ ArgBest wave_argbest(ArgBest a) {
    take_better(a, dpp_f32<DPP_ROW_SHR1, 0xF>(-INFINITY, a.v), dpp_i32<DPP_ROW_SHR1, 0xF>(-1, a.i));
    take_better(a, dpp_f32<DPP_ROW_SHR2, 0xF>(-INFINITY, a.v), dpp_i32<DPP_ROW_SHR2, 0xF>(-1, a.i));
    take_better(a, dpp_f32<DPP_ROW_SHR4, 0xF>(-INFINITY, a.v), dpp_i32<DPP_ROW_SHR4, 0xF>(-1, a.i));
    take_better(a, dpp_f32<DPP_ROW_SHR8, 0xF>(-INFINITY, a.v), dpp_i32<DPP_ROW_SHR8, 0xF>(-1, a.i));
    take_better(a, dpp_f32<DPP_ROW_BCAST15, 0xA>(-INFINITY, a.v), dpp_i32<DPP_ROW_BCAST15, 0xA>(-1, a.i));
    take_better(a, dpp_f32<DPP_ROW_BCAST31, 0xC>(-INFINITY, a.v), dpp_i32<DPP_ROW_BCAST31, 0xC>(-1, a.i));
    return ArgBest{lane63_f32(a.v), __builtin_amdgcn_readlane(a.i, 63)};
}

// Block-wide lexicographic argmax over candidates with i >= 0; i = -1 is "none".
__device__ ArgBest block_argmax(ArgBest a, ArgBest* lds) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    a = wave_argbest(a);
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

// Largest top_k the device routers select (per-token selections are staged
// in LDS and written out once).
constexpr uint32_t HK_TOPK_MAX = 64;

// Softmax top-k over one token's logits, p in LDS, the k selections staged in
// sel_i / sel_v (LDS, HK_TOPK_MAX each) and written to ids_out / w_out at the
// end.  renorm = 1: source_qwen80_topk_router (divide by the sum, renormalise
// by the selected sum); renorm = 0: topk_softmax_batch (multiply by 1/sum,
// raw probs).
__device__ void softmax_topk_block(const float* __restrict__ logits, uint32_t n, uint32_t k,
                                   float tie_eps, int renorm, float* p, int32_t* ids_out,
                                   float* w_out, uint32_t* status, float* redf, ArgBest* reda,
                                   int32_t* sel_i, float* sel_v) {
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
                sel_i[r] = (int32_t)bi;
                sel_v[r] = bv;
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
                sel_i[r] = b.i;
                sel_v[r] = b.v;
                if (b.i >= 0) p[b.i] = -INFINITY;
            }
            __syncthreads();
        }
    }
    __syncthreads();
    if (threadIdx.x == 0 && renorm) {
        float sel = -0.0f;
        for (uint32_t r = 0; r < k; ++r) sel += sel_v[r];
        for (uint32_t r = 0; r < k; ++r) sel_v[r] = sel_v[r] / sel;
    }
    __syncthreads();
    for (uint32_t r = threadIdx.x; r < k; r += blockDim.x) {
        ids_out[r] = sel_i[r];
        w_out[r] = sel_v[r];
    }
}

// Selection key of a softmax probability p >= 0 at index i: high word =
// bits(p) + 1 (non-negative floats order like their bit patterns), low word =
// ~i (the lower index wins a tie), so the (value desc, index asc) order is
// the unsigned order of the keys; 0 = taken / absent.
__device__ __forceinline__ uint64_t prob_key(float p, uint32_t i) {
    return ((uint64_t)(__builtin_bit_cast(uint32_t, p) + 1u) << 32) | (uint64_t)(~i);
}

__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
    const int lo = dpp_i32<CTRL, ROW_MASK>(0, (int)(uint32_t)v);
    const int hi = dpp_i32<CTRL, ROW_MASK>(0, (int)(uint32_t)(v >> 32));
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Wave-wide max of 64-bit keys on the DPP network; every lane gets it.
__device__ __forceinline__ uint64_t wave_max_key(uint64_t k) {
    k = umax64(k, dpp_u64<DPP_ROW_SHR1, 0xF>(k));
    k = umax64(k, dpp_u64<DPP_ROW_SHR2, 0xF>(k));
    k = umax64(k, dpp_u64<DPP_ROW_SHR4, 0xF>(k));
    k = umax64(k, dpp_u64<DPP_ROW_SHR8, 0xF>(k));
    k = umax64(k, dpp_u64<DPP_ROW_BCAST15, 0xA>(k));
    k = umax64(k, dpp_u64<DPP_ROW_BCAST31, 0xC>(k));
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)k, 63);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(k >> 32), 63);
    return ((uint64_t)hi << 32) | lo;
}

__device__ __forceinline__ uint32_t wave_incl_sum_u32(uint32_t v) {
    v += (uint32_t)dpp_i32<DPP_ROW_SHR1, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR2, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR4, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR8, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_BCAST15, 0xA>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_BCAST31, 0xC>(0, (int)v);
    return v;
}

// Wave-wide minimum of unsigned words on the DPP network; every lane gets it.
__device__ __forceinline__ uint32_t wave_min_u32(uint32_t v) {
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_SHR1, 0xF>(-1, (int)v));
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_SHR2, 0xF>(-1, (int)v));
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_SHR4, 0xF>(-1, (int)v));
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_SHR8, 0xF>(-1, (int)v));
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_BCAST15, 0xA>(-1, (int)v));
    v = min(v, (uint32_t)dpp_i32<DPP_ROW_BCAST31, 0xC>(-1, (int)v));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// The tie-window selection of source_qwen80_topk_router
// (model/qwen80_complete_runtime.rs:5988-6000 with route_tie_epsilon,
// moe.rs:8-14) for one wave: lane l holds q[l + 64 j] (the normalised
// probabilities, -inf past n).  The reference scans left to right and a later
// q replaces the best only when it is above it and not within eps of it (a
// later index never has the lower index, so its "tied and lower index" branch
// cannot fire); the result is the last of a chain of replacements, which the
// wave follows one link per reduction: the next link is the lowest index past
// the current best that would replace it.  Returns, in lane r < k, the r-th
// selection (id -1, weight 0 if nothing is selectable).  q is consumed.
template <int NPL>
__device__ __forceinline__ ArgBest tie_eps_select_wave(float (&q)[NPL], uint32_t n, uint32_t k, float eps, int lane) {
    ArgBest mine{0.0f, -1};
    for (uint32_t r = 0; r < k; ++r) {
        float bv = -INFINITY;
        uint32_t bi = 0;
        bool any = false;
        for (;;) {
            uint32_t cand = 0xFFFFFFFFu;
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const uint32_t i = (uint32_t)lane + 64u * (uint32_t)j;
                const float v = q[j];
                const bool tied = isfinite(bv) && isfinite(v) && fabsf(v - bv) <= eps;
                if (i < n && (!any || i > bi) && v > bv && !tied) cand = min(cand, i);
            }
            cand = wave_min_u32(cand);
            if (cand == 0xFFFFFFFFu) break;
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < NPL; ++j) v = (cand >> 6) == (uint32_t)j ? q[j] : v;
            bv = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)(cand & 63u)));
            bi = cand;
            any = true;
        }
        if ((uint32_t)lane == r) {
            mine.i = any ? (int)bi : -1;
            mine.v = any ? bv : 0.0f;
        }
        if (any && (bi & 63u) == (uint32_t)lane) {
#pragma unroll
            for (int j = 0; j < NPL; ++j) q[j] = (bi >> 6) == (uint32_t)j ? -INFINITY : q[j];
        }
    }
    return mine;
}

// LDS a wave's top-k selection works in (HK_TOPK_MAX candidates and slots).
struct TopkLds {
    uint64_t cand[64];
    int32_t sel_i[HK_TOPK_MAX];
    float sel_v[HK_TOPK_MAX];
};

// The tie_eps == 0 selection of softmax_topk_block for one wave (all 64 lanes,
// n <= 64 * NPL, k <= 64); same result as the block form for finite logits.
// Lane l holds p[l + 64 j].  The order is (q desc, index asc) with
// q = p / sum (renorm = 1) or p * (1/sum), on 64-bit keys: high word
// bits(q) + 1, low word ~index.
//   1. tau = the k-th largest lane-best p, to 16 bits (a bitwise ballot
//      count), is a lower bound of the k-th largest p; every p >= tau
//      (1 - 2^-20) is a candidate -- the relaxation keeps any element whose
//      rounded quotient could tie a selected one.
//   2. The candidates (usually k..2k) are compacted into LDS; each forms its
//      quotient and key, and its rank is the number of larger keys; ranks < k
//      are the selection, in order.
// With more than 64 candidates (flat distributions) it falls back to k
// rounds of a wave-wide key max.  Returns, in lane r < k, the r-th selection
// (id, weight); ids_out / w_out (if not null) get all k.
//
// tie_eps > 0 selects with the reference's tie window instead
// (tie_eps_select_wave); renormalisation and outputs are the same.
template <int NPL>
__device__ __forceinline__ ArgBest softmax_topk_wave(const float* __restrict__ logits, uint32_t n, uint32_t k, int renorm,
                                     int32_t* ids_out, float* w_out, uint32_t* status, TopkLds* t,
                                     int lane = (int)(threadIdx.x & 63), float tie_eps = 0.0f) {
    float p[NPL];
    float m = -INFINITY;
    uint32_t bad = 0;
    // unconditional loads (index clamped, value dropped past n): a load under
    // a per-lane condition would wait for the one before it
#pragma unroll
    for (int j = 0; j < NPL; ++j) p[j] = logits[min((uint32_t)lane + 64u * j, n - 1u)];
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        const uint32_t i = (uint32_t)lane + 64u * j;
        p[j] = i < n ? p[j] : -INFINITY;
        if (i < n && !isfinite(p[j])) bad = 1;
        m = fmaxf(m, p[j]);
    }
    if (bad && status) atomicOr(status, HK_DEVERR_NONFINITE);
    m = wave_max(m);
    float local = 0.f;
    uint32_t bv = 0;
#pragma unroll
    for (int j = 0; j < NPL; ++j) {
        p[j] = (uint32_t)lane + 64u * j < n ? expf(p[j] - m) : 0.0f;
        local += p[j];
        bv = max(bv, __builtin_bit_cast(uint32_t, p[j]));
    }
    const float sum = wave_sum(local);
    const float inv = 1.0f / sum;
    ArgBest mine{0.0f, -1};
    if (tie_eps > 0.0f) {
#pragma unroll
        for (int j = 0; j < NPL; ++j)
            p[j] = (uint32_t)lane + 64u * j < n ? (renorm ? p[j] / sum : p[j] * inv) : -INFINITY;
        mine = tie_eps_select_wave<NPL>(p, n, k, tie_eps, lane);
    } else {
        const uint32_t kk = min(k, 64u);
        uint32_t tau = 0;
#pragma unroll
        for (int b = 30; b >= 15; --b) {
            const uint32_t c = tau | (1u << b);
            if ((uint32_t)__popcll(__ballot(bv >= c)) >= kk) tau = c;
        }
        const float tf = __builtin_bit_cast(float, tau) * (1.0f - 0x1p-20f);
        uint32_t cnt = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) cnt += ((uint32_t)lane + 64u * j < n && p[j] >= tf) ? 1u : 0u;
        const uint32_t incl = wave_incl_sum_u32(cnt);
        const uint32_t C = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
        if (C <= 64u) {
            // slots no candidate fills (fewer than k candidates: a NaN logit never
            // passes p >= tf) stay id -1, weight 0; the status bit is already set
            if ((uint32_t)lane < k) {
                t->sel_i[lane] = -1;
                t->sel_v[lane] = 0.0f;
            }
            uint32_t o = incl - cnt;
#pragma unroll
            for (int j = 0; j < NPL; ++j)
                if ((uint32_t)lane + 64u * j < n && p[j] >= tf)
                    t->cand[o++] = ((uint64_t)__builtin_bit_cast(uint32_t, p[j]) << 32) | (uint64_t)((uint32_t)lane + 64u * j);
            __builtin_amdgcn_wave_barrier();
            uint64_t me = 0;
            if ((uint32_t)lane < C) {
                const uint64_t c = t->cand[lane];
                const float pv = __builtin_bit_cast(float, (uint32_t)(c >> 32));
                const float q = renorm ? pv / sum : pv * inv;
                me = ((uint64_t)(__builtin_bit_cast(uint32_t, q) + 1u) << 32) | (uint64_t)(~(uint32_t)c);
            }
            __builtin_amdgcn_wave_barrier();
            if ((uint32_t)lane < C) t->cand[lane] = me;
            __builtin_amdgcn_wave_barrier();
            uint32_t rank = 0;
            for (uint32_t u = 0; u < C; ++u) rank += t->cand[u] > me ? 1u : 0u;
            if ((uint32_t)lane < C && rank < k) {
                t->sel_i[rank] = (int32_t)~(uint32_t)me;
                t->sel_v[rank] = __builtin_bit_cast(float, (uint32_t)(me >> 32) - 1u);
            }
            __builtin_amdgcn_wave_barrier();
            if ((uint32_t)lane < k) {
                mine.i = t->sel_i[lane];
                mine.v = t->sel_v[lane];
            }
        } else {
            uint64_t key[NPL];
            uint64_t best = 0;
#pragma unroll
            for (int j = 0; j < NPL; ++j) {
                const uint32_t i = (uint32_t)lane + 64u * j;
                key[j] = i < n ? prob_key(renorm ? p[j] / sum : p[j] * inv, i) : 0ull;
                best = umax64(best, key[j]);
            }
            for (uint32_t r = 0; r < k; ++r) {
                const uint64_t w = wave_max_key(best);
                const uint32_t wi = ~(uint32_t)w;
                if ((uint32_t)lane == r) {
                    mine.i = w ? (int)wi : -1;
                    mine.v = __builtin_bit_cast(float, (uint32_t)(w >> 32) - 1u);
                }
                if (w && (wi & 63u) == (uint32_t)lane) {
                    best = 0;
#pragma unroll
                    for (int j = 0; j < NPL; ++j) {
                        key[j] = key[j] == w ? 0ull : key[j];
                        best = umax64(best, key[j]);
                    }
                }
            }
        }
    }
    if (renorm) {
        float sel = -0.0f;
        for (uint32_t r = 0; r < k; ++r)
            sel += __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mine.v), (int)r));
        mine.v = mine.i >= 0 ? mine.v / sel : 0.0f;
    }
    if ((uint32_t)lane < k) {
        if (ids_out) ids_out[lane] = mine.i;
        if (w_out) w_out[lane] = mine.v;
    }
    return mine;
}

}  // namespace hk
