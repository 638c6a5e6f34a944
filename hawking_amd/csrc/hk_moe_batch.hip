// hk_moe_batch.hip -- the noaux_tc MoE block for a batch of tokens
// (routed_moe, crates/hawking-core/src/gravity_glm.rs:550-600, with
// batched_mlp :515-548): every active expert's weights are streamed from HBM
// once for all of the tokens routed to it (a grouped expert GEMM on the int8
// matrix-core engine of hk_mfma.h: every weight fetch serves all the member
// tokens whose x images are in LDS).
//
//   1. xprep:    the fixed-point x image of each token (from its bf16 x)
//   2. router:   logits partials, split-K over 512-column slices (f32 matrix
//                cores, weights and bf16 x straight from global memory);
//                steps 1 and 2 share one launch
//   3. route:    one block per token: the noaux_tc route (gravity_glm.rs:447-500)
//                with ranks by counting in LDS
//   4. group:    one block: the (token, slot) pairs grouped by expert (shared
//                expert first, then ascending id) and each token's slots in
//                ascending expert id
//   5. gate/up:  per (active expert, 8 row tiles): the member tokens' x images
//                in LDS, each wave runs two gate+up tile pairs over all columns
//                and applies SwiGLU
//   6. act image: the x image of every (token, expert) activation row
//   7. down:     per (active expert, 8 row tiles): w * (down . act) per member
//   8. combine:  y_t = sum over t's experts in ascending id, then + shared
#include "hk_internal.h"
#include "hk_mfma.h"
#include "hk_moe.h"
#include "hk_router_dev.h"

namespace hk {

// router tiling: RT_WAVES waves of RT_WCOLS columns per split
constexpr uint32_t RT_WAVES = 4, RT_WCOLS = 128, RT_SLICE = RT_WAVES * RT_WCOLS;
static_assert(RT_SLICE == MOE_BATCH_ROUTER_COLS, "split width");

size_t moe_batch_img_bytes(uint32_t cols) { return x_lds_bytes<HK_Q4>(n_steps_for(HK_Q4, cols)); }

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// Orders LDS writes before later LDS reads of other lanes of the same wave
// (a wave's LDS instructions execute in order; this keeps the compiler from
// reordering them).
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Inclusive prefix sum over the 64 lanes on the DPP network.
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
    v += (uint32_t)dpp_i32<DPP_ROW_SHR1, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR2, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR4, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_SHR8, 0xF>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_BCAST15, 0xA>(0, (int)v);
    v += (uint32_t)dpp_i32<DPP_ROW_BCAST31, 0xC>(0, (int)v);
    return v;
}

// Selection key of any non-NaN float v at index i: the unsigned order of the
// keys is (value desc, index asc); 0 = taken.
__device__ __forceinline__ uint64_t order_key(float v, uint32_t i) {
    const uint32_t b = __builtin_bit_cast(uint32_t, v);
    const uint32_t o = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)o << 32) | (uint64_t)(~i);
}

__device__ __forceinline__ uint32_t pair_token(const MoeBatchDims& d, uint32_t p) {
    return p < d.T * d.K ? p / d.K : p - d.T * d.K;
}

// ------------------------------------------------------------------ 1. x prep

// Floats of LDS x staging for `cols` columns (rounded up to whole Q4 steps).
static uint32_t q4_stage_floats(uint32_t cols) { return n_steps_for(HK_Q4, cols) * tile_step_cols(HK_Q4); }

// Image parts of 512 columns (4 Q4 steps): a token's image is built by
// ceil(cols / 512) blocks, each computing E from all of x.
constexpr uint32_t XPART_COLS = 512, XPART_STEPS = XPART_COLS / 128u;

// Steps [tb, tb + ns) of the Q4 x image of xs (LDS, >=
// q4_stage_floats(cols) floats, those columns quantized in place) into img
// (global), by the whole block.
__device__ int x_image_in_place(float* xs, uint32_t cols, uint8_t* img, float* red, bool* bad, uint32_t tb,
                                uint32_t ns = XPART_STEPS) {
    const uint32_t S = n_steps_for(HK_Q4, cols);
    XChunks<1> xc;
    load_x<1>(BlockTeam{}, xs, cols, xc);
    return x_image<HK_Q4, 1>(BlockTeam{}, xc, xs, cols, S, img, xs + tb * 128u, 8u * blockDim.x, red, bad, tb, tb + ns);
}

// Token t's image part `part`; xs: LDS of q4_stage_floats(H) floats.
__device__ __forceinline__ void xprep_block(const MoeBatchDims& d, const uint16_t* __restrict__ xb, const MoeBatchWs& ws,
                                            uint32_t t, uint32_t part, float* xs) {
    __shared__ float red[4];
    {
        // 8 bf16 per thread and piece, 4 pieces in flight (hidden <= 8192)
        const uint4* src = reinterpret_cast<const uint4*>(xb + (size_t)t * d.H);
        const uint32_t n8 = d.H / 8u;
        uint4 v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t k = threadIdx.x + (uint32_t)i * blockDim.x;
            if (k < n8) v[i] = ldg(src + k);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t k = threadIdx.x + (uint32_t)i * blockDim.x;
            if (k < n8) {
                const uint32_t w[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
                float f[8];
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    f[2 * q] = bf16_to_f32((uint16_t)(w[q] & 0xFFFFu));
                    f[2 * q + 1] = bf16_to_f32((uint16_t)(w[q] >> 16));
                }
                float4* o = reinterpret_cast<float4*>(xs + 8u * k);
                o[0] = make_float4(f[0], f[1], f[2], f[3]);
                o[1] = make_float4(f[4], f[5], f[6], f[7]);
            }
        }
    }
    __syncthreads();
    bool bad = false;
    const int E = x_image_in_place(xs, d.H, ws.ximg + (size_t)t * ws.ximg_stride, red, &bad, part * XPART_STEPS);
    if (threadIdx.x == 0) {
        if (part == 0) ws.ximg_e[t] = E;
        if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
}

// ------------------------------------------------------------------ 2. router (split-K, f32 matrix cores)

// part[s][t][e] = sum over the columns [RT_SLICE s, RT_SLICE (s + 1)) of
// W[e][k] x[t][k], x read as bf16 (exact in f32).  A workgroup owns 16 router
// rows and one slice; each of its RT_WAVES waves takes RT_WCOLS columns of it
// and the waves' sums meet in LDS (in wave order).  A wave loads its weights
// (16 rows) and its tokens' x (16 per token tile) straight into registers and
// multiplies on v_mfma_f32_16x16x4_f32: in 32-column group g, lane l supplies
// row / token l % 16 at columns 32 g + 8 (l / 16) + i, i < 8, the same map for
// both operands (MFMA i of the group takes column offset i of every lane).
__device__ __forceinline__ void router_block(const MoeBatchDims& d, const float* __restrict__ W,
                                             const uint16_t* __restrict__ xb, const MoeBatchWs& ws, uint32_t bx, uint32_t s) {
    constexpr uint32_t G = RT_WCOLS / 32u;
    __shared__ float red[RT_WAVES][2][16][17];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6, li = (uint32_t)lane & 15u, lg = (uint32_t)lane >> 4;
    const uint32_t r0 = bx * 16u;
    const uint32_t c0 = s * RT_SLICE + wave * RT_WCOLS;
    const bool on = c0 < d.H;  // hidden % 128 == 0: a wave's columns are all in or all out
    const uint32_t row = r0 + li;
    float4 wv[G][2];
#pragma unroll
    for (uint32_t g = 0; g < G; ++g) {
        const float* src = W + (size_t)row * d.H + c0 + 32u * g + 8u * lg;
        const bool ok = on && row < d.E;
        wv[g][0] = ok ? ldg(reinterpret_cast<const float4*>(src)) : make_float4(0.f, 0.f, 0.f, 0.f);
        wv[g][1] = ok ? ldg(reinterpret_cast<const float4*>(src + 4)) : make_float4(0.f, 0.f, 0.f, 0.f);
    }
    for (uint32_t tb = 0; tb < d.T; tb += 32u) {
        uint4 xv[2][G];
#pragma unroll
        for (uint32_t tt = 0; tt < 2; ++tt) {
            const uint32_t t = tb + 16u * tt + li;
#pragma unroll
            for (uint32_t g = 0; g < G; ++g)
                xv[tt][g] = (on && t < d.T)
                                ? ldg(reinterpret_cast<const uint4*>(xb + (size_t)t * d.H + c0 + 32u * g + 8u * lg))
                                : make_uint4(0u, 0u, 0u, 0u);
        }
        hk_f32x4 acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (uint32_t g = 0; g < G; ++g) {
            const float wk[8] = {wv[g][0].x, wv[g][0].y, wv[g][0].z, wv[g][0].w,
                                 wv[g][1].x, wv[g][1].y, wv[g][1].z, wv[g][1].w};
#pragma unroll
            for (uint32_t tt = 0; tt < 2; ++tt) {
                const uint32_t xw[4] = {xv[tt][g].x, xv[tt][g].y, xv[tt][g].z, xv[tt][g].w};
#pragma unroll
                for (uint32_t i = 0; i < 8; ++i) {
                    const float xf = __builtin_bit_cast(float, (i & 1u) ? (xw[i >> 1] & 0xFFFF0000u) : (xw[i >> 1] << 16));
                    acc[tt] = __builtin_amdgcn_mfma_f32_16x16x4f32(wk[i], xf, acc[tt], 0, 0, 0);
                }
            }
        }
        // lane l, register j holds row 4 (l / 16) + j, token l % 16 of its tile
        __syncthreads();
#pragma unroll
        for (uint32_t tt = 0; tt < 2; ++tt)
#pragma unroll
            for (uint32_t j = 0; j < 4; ++j) red[wave][tt][4u * lg + j][li] = acc[tt][j];
        __syncthreads();
        for (uint32_t o = threadIdx.x; o < 2u * 16u * 16u; o += blockDim.x) {
            const uint32_t tt = o >> 8, m = (o >> 4) & 15u, n = o & 15u;
            float v = red[0][tt][m][n];
#pragma unroll
            for (uint32_t w = 1; w < RT_WAVES; ++w) v += red[w][tt][m][n];
            const uint32_t e = r0 + m, t = tb + 16u * tt + n;
            if (e < d.E && t < d.T) ws.part[((size_t)s * d.T + t) * d.E + e] = v;
        }
    }
}

// Steps 1 and 2 in one launch (they are independent): blocks [0, nr) are
// router blocks (row tile b % rt, split b / rt), the rest x image blocks
// (token i % T, part i / T).
__global__ void __launch_bounds__(64 * RT_WAVES) moe_batch_prep_kernel(MoeBatchDims d, const uint16_t* __restrict__ xb,
                                                                      const float* __restrict__ W, MoeBatchWs ws) {
    extern __shared__ __align__(16) float xs[];  // [H rounded up to whole steps]
    const uint32_t rt = (d.E + 15u) / 16u, nr = rt * d.S, b = blockIdx.x;
    if (b < nr) {
        router_block(d, W, xb, ws, b % rt, b / rt);
    } else {
        const uint32_t i = b - nr;
        xprep_block(d, xb, ws, i % d.T, i / d.T, xs);
    }
}

// ------------------------------------------------------------------ 3. route (one block per token)

__device__ __forceinline__ float key_value(uint64_t k) {
    const uint32_t o = (uint32_t)(k >> 32);
    return __builtin_bit_cast(float, (o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
}

// Experts i in [lo, hi) whose key is above k.
__device__ __forceinline__ uint32_t keys_above(const uint64_t* keys, uint32_t lo, uint32_t hi, uint64_t k) {
    uint32_t n = 0;
#pragma unroll 8
    for (uint32_t i = lo; i < hi; ++i) n += keys[i] > k ? 1u : 0u;
    return n;
}

constexpr uint32_t MOE_ROUTER_MAX_SPLITS = (8192 + MOE_BATCH_ROUTER_COLS - 1) / MOE_BATCH_ROUTER_COLS;

// The block sums each expert's split-K partials (in split order, every load
// of a thread in flight at once) and ranks by counting: an expert's rank is
// the number of keys above its own (keys are distinct: value desc, index asc),
// so every selection below is the order-exact top-n.  The final top k counts
// among candidates only: experts ranked below k inside their 64-expert range
// (any expert above a top-k expert is itself top-k, so its rank inside its
// range is below k too, and a candidate's rank among candidates is its rank
// among all experts whenever either is below k).
__global__ void __launch_bounds__(256) moe_batch_route_kernel(MoeBatchDims d, const float* __restrict__ bias,
                                                              MoeBatchWs ws, int32_t* ids_out, float* w_out) {
    __shared__ uint64_t key[MOE_BATCH_MAX_EXPERTS];
    __shared__ float sc[MOE_BATCH_MAX_EXPERTS];
    __shared__ float top2[64][2];
    __shared__ uint64_t gkey[64];
    __shared__ uint32_t chosen[64];
    __shared__ uint64_t ckey[MOE_BATCH_MAX_EXPERTS];
    __shared__ uint16_t cand[MOE_BATCH_MAX_EXPERTS];
    __shared__ uint32_t ncand;
    __shared__ int32_t sel_i[16];
    __shared__ float sel_w[16];
    const uint32_t t = blockIdx.x, E = d.E, K = d.K, per = d.E / d.n_group, tid = threadIdx.x;
    uint32_t bad = 0;
    if (tid == 0) ncand = 0;
    for (uint32_t e = tid; e < E; e += blockDim.x) {
        float pv[MOE_ROUTER_MAX_SPLITS];
#pragma unroll
        for (uint32_t s = 0; s < MOE_ROUTER_MAX_SPLITS; ++s)
            pv[s] = s < d.S ? ws.part[((size_t)s * d.T + t) * E + e] : 0.0f;
        float l = 0.f;
#pragma unroll
        for (uint32_t s = 0; s < MOE_ROUTER_MAX_SPLITS; ++s)
            if (s < d.S) l += pv[s];
        if (!isfinite(l)) bad = 1;
        const float v = 1.0f / (1.0f + expf(-l));
        sc[e] = v;
        key[e] = order_key(v + bias[e], e);
    }
    if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    __syncthreads();
    if (d.topk_group < d.n_group) {
        // group strength = sum of its best two corrected scores, in topk_desc order
        for (uint32_t e = tid; e < E; e += blockDim.x) {
            const uint32_t g = e / per, rk = keys_above(key, g * per, g * per + per, key[e]);
            if (rk < 2) top2[g][rk] = key_value(key[e]);
        }
        __syncthreads();
        if (tid < d.n_group) {
            float gs = -0.0f + top2[tid][0];
            if (per >= 2) gs = gs + top2[tid][1];
            gkey[tid] = order_key(gs, tid);
        }
        __syncthreads();
        if (tid < d.n_group) chosen[tid] = keys_above(gkey, 0, d.n_group, gkey[tid]) < d.topk_group ? 1u : 0u;
        __syncthreads();
        // only experts inside a chosen group compete (the others at -inf)
        for (uint32_t e = tid; e < E; e += blockDim.x)
            if (!chosen[e / per]) key[e] = order_key(-INFINITY, e);
        __syncthreads();
    }
    for (uint32_t e = tid; e < E; e += blockDim.x) {
        const uint32_t lo = e & ~63u;
        if (keys_above(key, lo, min(lo + 64u, E), key[e]) < K) {
            const uint32_t c = atomicAdd(&ncand, 1u);
            cand[c] = (uint16_t)e;
            ckey[c] = key[e];
        }
    }
    __syncthreads();
    const uint32_t nc = ncand;
    for (uint32_t c = tid; c < nc; c += blockDim.x) {
        const uint32_t rk = keys_above(ckey, 0, nc, ckey[c]);
        if (rk < K) {
            sel_i[rk] = (int32_t)cand[c];
            sel_w[rk] = sc[cand[c]];  // weights are the uncorrected scores
        }
    }
    __syncthreads();
    if (tid == 0) {
        float total = -0.0f;
        for (uint32_t r = 0; r < K; ++r) total += sel_w[r];
        total = total + 1e-20f;
        for (uint32_t r = 0; r < K; ++r) {
            float v = sel_w[r];
            if (d.norm_topk_prob) v = v / total;
            sel_w[r] = v * d.scaling;
        }
    }
    __syncthreads();
    if (tid < K) {
        const uint32_t p = t * K + tid;
        ws.ids[p] = sel_i[tid];
        ws.w[p] = sel_w[tid];
        if (ids_out) ids_out[p] = sel_i[tid];
        if (w_out) w_out[p] = sel_w[tid];
    }
}

// ------------------------------------------------------------------ 4. group

__global__ void __launch_bounds__(1024) moe_batch_group_kernel(MoeBatchDims d, MoeBatchWs ws) {
    constexpr int NPL = MOE_BATCH_MAX_EXPERTS / 64;
    __shared__ int32_t sids[MOE_BATCH_MAX_TOKENS * 16];
    __shared__ uint32_t cnt[MOE_BATCH_MAX_EXPERTS], fill[MOE_BATCH_MAX_EXPERTS], start[MOE_BATCH_MAX_EXPERTS];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6, E = d.E, K = d.K, np = d.T * d.K, has_shared = d.SI ? 1u : 0u;
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    for (uint32_t p = threadIdx.x; p < np; p += blockDim.x) sids[p] = ws.ids[p];
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < np; p += blockDim.x) atomicAdd(&cnt[(uint32_t)sids[p]], 1u);
    __syncthreads();
    if (wave == 0) {
        // lane l owns experts 8l .. 8l+7: member offsets and active indexes by prefix sums
        uint32_t c[NPL], lc = 0, lf = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const uint32_t e = (uint32_t)lane * NPL + j;
            c[j] = e < E ? cnt[e] : 0u;
            lc += c[j];
            lf += c[j] ? 1u : 0u;
        }
        const uint32_t ic = wave_incl_scan(lc), iff = wave_incl_scan(lf);
        uint32_t m = has_shared * d.T + ic - lc, a = has_shared + iff - lf;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const uint32_t e = (uint32_t)lane * NPL + j;
            if (c[j]) {
                start[e] = m;
                ws.active[a] = make_uint4(e, m, c[j], 0u);
                m += c[j];
                ++a;
            }
        }
        if (lane == 63) {
            *ws.n_active = a;
            if (has_shared) ws.active[0] = make_uint4(E, 0u, d.T, 0u);
        }
    }
    __syncthreads();
    for (uint32_t p = threadIdx.x; p < np; p += blockDim.x) {
        const uint32_t e = (uint32_t)sids[p];
        ws.members[start[e] + atomicAdd(&fill[e], 1u)] = p;  // member order does not change any result
    }
    if (has_shared)
        for (uint32_t t = threadIdx.x; t < d.T; t += blockDim.x) ws.members[t] = np + t;
    // each routed pair's position among its token's slots in ascending
    // expert id (ids of a token are distinct): the down kernel stores the
    // pair's output there, so the combine reads a token's outputs in order
    for (uint32_t p = threadIdx.x; p < np; p += blockDim.x) {
        const uint32_t t = p / K;
        uint32_t rank = 0;
        for (uint32_t j = 0; j < K; ++j) rank += sids[t * K + j] < sids[p] ? 1u : 0u;
        ws.rank[p] = (int32_t)rank;
    }
}

// ------------------------------------------------------------------ grouped tile worker

#ifndef HK_BATCH_NT
#define HK_BATCH_NT 1
#endif
// Where the weight pipelines' fetches past an item's last step go (they stay
// unconditional): a re-read of the last step under the non-temporal hint
// would come from HBM again; this buffer stays in the caches.  Nothing
// fetched from it is consumed.
__device__ __align__(256) uint8_t g_batch_refetch_dummy[2048];

// Step t of weight tiles r < R (tile r of organ r's data/scales, the lane's
// 16 data bytes at base_d[r] + 1024 t) into fr; past: the same loads from the
// refetch buffer.  The data loads carry the non-temporal hint (HK_BATCH_NT).
template <int R>
__device__ __forceinline__ void tiles_fetch(const uint8_t* const* base_d, const uint16_t* const* base_s, uint32_t t,
                                            Frag<HK_Q4, R>& fr, bool past = false) {
    const uint32_t lane = threadIdx.x & 63u;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const uint4* pd = past ? reinterpret_cast<const uint4*>(g_batch_refetch_dummy + 16u * lane)
                               : reinterpret_cast<const uint4*>(base_d[r] + (size_t)t * 1024u);
        const uint16_t* ps = past ? reinterpret_cast<const uint16_t*>(g_batch_refetch_dummy + 1024u) + lane
                                  : base_s[r] + (size_t)t * 64u;
        fr.v[r] = HK_BATCH_NT ? ldg_nt(pd) : ldg(pd);
        fr.s[r] = ldg(ps);
    }
}

// The pipeline's first D steps (past the end they re-read the last): issued
// before the member tokens' images are staged, so the staging's latency and
// the weights' overlap.
template <int R, int D>
__device__ __forceinline__ void tiles_fetch_first(const uint8_t* const* base_d, const uint16_t* const* base_s,
                                                  uint32_t S, Frag<HK_Q4, R> (&f)[D]) {
#pragma unroll
    for (int k = 0; k < D; ++k) tiles_fetch<R>(base_d, base_s, min((uint32_t)k, S - 1u), f[k], (uint32_t)k >= S);
}

// acc[j][r] += this lane's partial dot of weight tile r (tile Tr[r] of organ
// r's data/scales, S column steps) with member token j's x image in LDS
// (img + j*img_bytes), over all S steps with a D-deep weight pipeline whose
// first D steps are already in f (tiles_fetch_first).
template <int R, int TB, int D>
__device__ __forceinline__ void tiles_x_tokens(const uint8_t* const* base_d, const uint16_t* const* base_s, uint32_t S,
                                               const uint8_t* img, uint32_t img_bytes, uint32_t nm, uint32_t aoff,
                                               int q, float (*acc)[R], Frag<HK_Q4, R> (&f)[D]) {
    auto fetch = [&](uint32_t t, Frag<HK_Q4, R>& fr, bool past) { tiles_fetch<R>(base_d, base_s, t, fr, past); };
    const float* SX0 = reinterpret_cast<const float*>(img + (size_t)S * 2u * A_TILE_STRIDE);
    auto consume = [&](const Frag<HK_Q4, R>& fr, uint32_t t) {
        v4i alo[TB], ahi[TB];
        float2 sx[TB];  // the unit's {f_u, 8 f_u sum X}
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            if ((uint32_t)j < nm) {
                const uint8_t* ij = img + (size_t)j * img_bytes;
                alo[j] = lds_a(ij, 2u * t, aoff);
                ahi[j] = lds_a(ij, 2u * t + 1u, aoff);
                sx[j] = reinterpret_cast<const float2*>(reinterpret_cast<const uint8_t*>(SX0) + (size_t)j * img_bytes)[4u * t + (uint32_t)q];
            }
        }
        const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const v4i lo = {(int)(fr.v[r].x & m), (int)(fr.v[r].y & m), (int)(fr.v[r].z & m), (int)(fr.v[r].w & m)};
            const v4i hi = {(int)((fr.v[r].x >> 4) & m), (int)((fr.v[r].y >> 4) & m), (int)((fr.v[r].z >> 4) & m),
                            (int)((fr.v[r].w >> 4) & m)};
            const float sc = f16_bits_to_f32(fr.s[r]);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if ((uint32_t)j < nm) {
                    v4i c = mfma_i8(alo[j], lo, v4i{0, 0, 0, 0});
                    c = mfma_i8(ahi[j], hi, c);
                    acc[j][r] += sc * (combine_limbs(c) * sx[j].x - sx[j].y);
                }
            }
        }
    };
    // branch-free pipeline (refetches past the end re-read the last step), so
    // each consume waits only for its own slot's loads
    const uint32_t last = S - 1u;
    uint32_t it = 0;
    for (; it + D <= S; it += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            consume(f[k], it + (uint32_t)k);
            fetch(min(it + D + (uint32_t)k, last), f[k], it + D + (uint32_t)k > last);
        }
    }
#pragma unroll
    for (int k = 0; k < D; ++k) {
        if (it + (uint32_t)k >= S) break;
        consume(f[k], it + (uint32_t)k);
    }
}

// Copies the x images of nm <= TB member tokens (rows idx[] of src) into LDS
// (all threads of the block): per pass every thread loads PT pieces of each
// image before its first store (the image index is a compile-time loop
// variable, so no per-piece table lookup).
template <int TB, int PT>
__device__ __forceinline__ void stage_images(uint8_t* lds, const uint8_t* src, uint32_t stride, const uint32_t* idx,
                                             uint32_t nm, uint32_t img_bytes) {
    const uint32_t n16 = img_bytes / 16u, nt = blockDim.x;
    for (uint32_t b = 0; b < n16; b += PT * nt) {
        uint4 v[TB][PT];
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            const uint4* sj = reinterpret_cast<const uint4*>(src + (size_t)idx[j] * stride);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const uint32_t k = b + threadIdx.x + (uint32_t)i * nt;
                if ((uint32_t)j < nm && k < n16) v[j][i] = ldg(sj + k);
            }
        }
#pragma unroll
        for (int j = 0; j < TB; ++j) {
            uint4* dj = reinterpret_cast<uint4*>(lds + (size_t)j * img_bytes);
#pragma unroll
            for (int i = 0; i < PT; ++i) {
                const uint32_t k = b + threadIdx.x + (uint32_t)i * nt;
                if ((uint32_t)j < nm && k < n16) dj[k] = v[j][i];
            }
        }
    }
}

// Work items of a grouped kernel: (active expert a, tile group tg, member
// groups [m_lo, m_hi) of TB tokens).  The shared expert (active entry 0) has
// every token as a member, so each of its member groups is an item of its
// own, listed first; a routed expert's item covers all of its members
// (rarely more than one group).  Workgroup b runs on XCD b % 8 (dispatch is
// round robin over the XCDs), so the shared expert's items are placed to put
// every member group of a tile group on one XCD, in consecutive waves of the
// dispatch: its weights are read from HBM once per tile group and the other
// member groups find them in that XCD's L2.  Slots past the last tile group
// (tile groups rounded up to a multiple of 8) are empty items.
constexpr uint32_t MOE_BATCH_XCDS = 8;
__host__ __device__ inline uint32_t moe_batch_items(uint32_t gpe, uint32_t ngs, uint32_t n_routed) {
    return (gpe + MOE_BATCH_XCDS - 1u) / MOE_BATCH_XCDS * MOE_BATCH_XCDS * ngs + n_routed * gpe;
}
struct ItemMap {
    uint32_t gpe, ngs, nsh, n_items;
    __device__ ItemMap(const MoeBatchDims& d, uint32_t gpe_, uint32_t n_active, uint32_t TB) : gpe(gpe_) {
        ngs = d.SI ? (d.T + TB - 1) / TB : 0u;
        nsh = moe_batch_items(gpe, ngs, 0u);
        n_items = moe_batch_items(gpe, ngs, n_active - (ngs ? 1u : 0u));
    }
    __device__ void at(uint32_t item, uint32_t* a, uint32_t* tg, uint32_t* m_lo, uint32_t* m_hi) const {
        if (item < nsh) {
            const uint32_t x = item % MOE_BATCH_XCDS, s = item / MOE_BATCH_XCDS;
            *a = 0;
            *tg = x + MOE_BATCH_XCDS * (s / ngs);  // >= gpe: an empty slot
            *m_lo = s % ngs;
            *m_hi = *m_lo + 1u;
            return;
        }
        const uint32_t i = item - nsh;
        *a = (ngs ? 1u : 0u) + i / gpe;
        *tg = i % gpe;
        *m_lo = 0;
        *m_hi = 0xFFFFFFFFu;
    }
};

// ------------------------------------------------------------------ 5. gate/up (grouped)

// An item covers TPI row tiles; a workgroup of TPI / TPW waves, each wave
// runs TPW row tiles (gate and up of each) for the item's member tokens.
template <int TB, int D, int TPW, int TPI>
__global__ void __launch_bounds__(64 * TPI / TPW)
moe_batch_gate_up_kernel(MoeBatchDims d, const OrganView* __restrict__ table, MoeBatchWs ws) {
    extern __shared__ __align__(16) uint8_t lds[];  // TB x images of H columns
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t aoff = a_lane_offset(lane);
    const uint32_t tiles = n_tiles_for(max(d.I, d.SI)), gpe = (tiles + TPI - 1) / TPI;
    const uint32_t S = n_steps_for(HK_Q4, d.H);
    const uint32_t img_bytes = (uint32_t)x_lds_bytes<HK_Q4>(S);
    const ItemMap im(d, gpe, __builtin_amdgcn_readfirstlane(*ws.n_active), TB);
    for (uint32_t item = blockIdx.x; item < im.n_items; item += gridDim.x) {
        uint32_t a, tg, mg_lo, mg_hi;
        im.at(item, &a, &tg, &mg_lo, &mg_hi);
        const uint4 ent = ws.active[a];
        const OrganView g = table[ent.x * 3u + 0u], u = table[ent.x * 3u + 1u];
        if (tg * TPI >= g.n_tiles) continue;
        // this wave's tiles (past the end they alias the first)
        const uint32_t Tb = tg * TPI + TPW * wave;
        bool vw[TPW];
        const uint8_t* bd[2 * TPW];
        const uint16_t* bs[2 * TPW];
#pragma unroll
        for (int h = 0; h < TPW; ++h) {
            vw[h] = Tb + h < g.n_tiles;
            const size_t Tc = vw[h] ? Tb + h : Tb;
            bd[2 * h] = g.data + Tc * S * 1024u + 16u * lane;
            bd[2 * h + 1] = u.data + Tc * S * 1024u + 16u * lane;
            bs[2 * h] = g.scales + Tc * S * 64u + lane;
            bs[2 * h + 1] = u.scales + Tc * S * 64u + lane;
        }
        const uint32_t m_end = mg_hi == 0xFFFFFFFFu ? ent.z : min(ent.z, mg_hi * (uint32_t)TB);
        for (uint32_t m0 = mg_lo * TB; m0 < m_end; m0 += TB) {
            const uint32_t nm = min((uint32_t)TB, ent.z - m0);
            uint32_t pair[TB], tok[TB];
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                pair[j] = ws.members[ent.y + m0 + min((uint32_t)j, nm - 1u)];
                tok[j] = pair_token(d, pair[j]);
            }
            Frag<HK_Q4, 2 * TPW> f[D];
            if (vw[0]) tiles_fetch_first<2 * TPW, D>(bd, bs, S, f);
            __syncthreads();
            stage_images<TB, 4>(lds, ws.ximg, ws.ximg_stride, tok, nm, img_bytes);
            __syncthreads();
            if (!vw[0]) continue;
            float acc[TB][2 * TPW] = {};
            tiles_x_tokens<2 * TPW, TB, D>(bd, bs, S, lds, img_bytes, nm, aoff, q, acc, f);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if ((uint32_t)j >= nm) break;
                const int E = ws.ximg_e[tok[j]];
#pragma unroll
                for (int h = 0; h < TPW; ++h) {
                    const float gs = ldexpf(tile_row_sum(acc[j][2 * h]), -E), us = ldexpf(tile_row_sum(acc[j][2 * h + 1]), -E);
                    const uint32_t row = (Tb + h) * 16u + (uint32_t)(lane & 15);
                    if (lane < 16 && vw[h] && row < g.rows)
                        ws.act[(size_t)pair[j] * d.Imax + row] = (gs / (1.0f + expf(-gs))) * us;
                }
            }
        }
    }
}

// ------------------------------------------------------------------ 6. activation images

__global__ void __launch_bounds__(256) moe_batch_act_image_kernel(MoeBatchDims d, MoeBatchWs ws) {
    extern __shared__ __align__(16) float xs[];  // [Imax rounded up to whole steps]
    __shared__ float red[4];
    const uint32_t p = blockIdx.x;
    const uint32_t cols = p < d.T * d.K ? d.I : d.SI;
    copy16_to_lds<4>(reinterpret_cast<uint4*>(xs), reinterpret_cast<const uint4*>(ws.act + (size_t)p * d.Imax), cols / 4u,
                     threadIdx.x, blockDim.x);
    __syncthreads();
    bool bad = false;
    const uint32_t ns = (n_steps_for(HK_Q4, d.Imax) + gridDim.y - 1u) / gridDim.y;  // steps per part
    const int E = x_image_in_place(xs, cols, ws.aimg + (size_t)p * ws.aimg_stride, red, &bad, blockIdx.y * ns, ns);
    if (threadIdx.x == 0) {
        if (blockIdx.y == 0) ws.aimg_e[p] = E;
        if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
}

// ------------------------------------------------------------------ 7. down (grouped)

template <int TB, int D, int TPW, int TPI>
__global__ void __launch_bounds__(64 * TPI / TPW)
moe_batch_down_kernel(MoeBatchDims d, const OrganView* __restrict__ table, MoeBatchWs ws) {
    extern __shared__ __align__(16) uint8_t lds[];  // TB activation images
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t aoff = a_lane_offset(lane);
    const uint32_t tiles = n_tiles_for(d.H), gpe = (tiles + TPI - 1) / TPI;
    const ItemMap im(d, gpe, __builtin_amdgcn_readfirstlane(*ws.n_active), TB);
    const uint32_t np = d.T * d.K;
    for (uint32_t item = blockIdx.x; item < im.n_items; item += gridDim.x) {
        uint32_t a, tg, mg_lo, mg_hi;
        im.at(item, &a, &tg, &mg_lo, &mg_hi);
        const uint4 ent = ws.active[a];
        const OrganView o = table[ent.x * 3u + 2u];
        const uint32_t S = o.steps, img_bytes = (uint32_t)x_lds_bytes<HK_Q4>(S);
        const uint32_t Tb = tg * TPI + TPW * wave;
        bool vw[TPW];
        const uint8_t* bd[TPW];
        const uint16_t* bs[TPW];
#pragma unroll
        for (int h = 0; h < TPW; ++h) {
            vw[h] = Tb + h < o.n_tiles;
            const size_t Tc = vw[h] ? Tb + h : Tb;
            bd[h] = o.data + Tc * S * 1024u + 16u * lane;
            bs[h] = o.scales + Tc * S * 64u + lane;
        }
        const uint32_t m_end = mg_hi == 0xFFFFFFFFu ? ent.z : min(ent.z, mg_hi * (uint32_t)TB);
        for (uint32_t m0 = mg_lo * TB; m0 < m_end; m0 += TB) {
            const uint32_t nm = min((uint32_t)TB, ent.z - m0);
            uint32_t pair[TB];
#pragma unroll
            for (int j = 0; j < TB; ++j) pair[j] = ws.members[ent.y + m0 + min((uint32_t)j, nm - 1u)];
            Frag<HK_Q4, TPW> f[D];
            if (vw[0]) tiles_fetch_first<TPW, D>(bd, bs, S, f);
            __syncthreads();
            stage_images<TB, 2>(lds, ws.aimg, ws.aimg_stride, pair, nm, img_bytes);
            __syncthreads();
            if (!vw[0]) continue;
            float acc[TB][TPW] = {};
            tiles_x_tokens<TPW, TB, D>(bd, bs, S, lds, img_bytes, nm, aoff, q, acc, f);
#pragma unroll
            for (int j = 0; j < TB; ++j) {
                if ((uint32_t)j >= nm) break;
                const int E = ws.aimg_e[pair[j]];
                const bool routed = pair[j] < np;
                const float w = routed ? ws.w[pair[j]] : 1.0f;
                // a routed pair's output goes to its token's row of its rank in expert order
                const uint32_t dst = routed ? pair[j] - pair[j] % d.K + (uint32_t)ws.rank[pair[j]] : pair[j];
#pragma unroll
                for (int h = 0; h < TPW; ++h) {
                    const float y = ldexpf(tile_row_sum(acc[j][h]), -E);
                    const uint32_t row = (Tb + h) * 16u + (uint32_t)(lane & 15);
                    if (lane < 16 && vw[h] && row < d.H) ws.ybuf[(size_t)dst * d.H + row] = y * w;
                }
            }
        }
    }
}

// ------------------------------------------------------------------ 8. combine

__global__ void __launch_bounds__(256) moe_batch_combine_kernel(MoeBatchDims d, MoeBatchWs ws, float* __restrict__ y) {
    const uint32_t t = blockIdx.x, row = blockIdx.y * blockDim.x + threadIdx.x;
    if (row >= d.H) return;
    // routed = 0; routed += o * w over the experts in ascending id; routed += shared
    // (every load in flight at once: top_k <= 16)
    float v[17];
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j)
        v[j] = j < d.K ? ws.ybuf[(size_t)(t * d.K + j) * d.H + row] : 0.0f;  // in expert order (the down kernel's rows)
    v[16] = d.SI ? ws.ybuf[(size_t)(d.T * d.K + t) * d.H + row] : 0.0f;
    float acc = 0.0f;
#pragma unroll
    for (uint32_t j = 0; j < 16; ++j)
        if (j < d.K) acc += v[j];
    if (d.SI) acc += v[16];
    y[(size_t)t * d.H + row] = acc;
}

// LDS a grouped workgroup may fill with staged token images: the device's
// per-block maximum, at most 128 KiB (gfx950: 160 KiB per CU; for config 5,
// four 31 KB x images per gate/up group, one workgroup per CU, beat two
// images and two workgroups: 775 vs 816 us per step, as fewer member groups
// re-stream an expert's weights).
static uint32_t image_lds_budget() {
    int dev = 0, v = 65536;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMaxSharedMemoryPerBlock, dev) != hipSuccess)
        v = 65536;
    return min((uint32_t)v, 131072u);
}

// Token images per member group that fit the budget.
static uint32_t tokens_per_group(uint32_t img_bytes, uint32_t cap, uint32_t budget) {
    return min(cap, budget / img_bytes);
}

hipError_t launch_moe_batch(const MoeBatchDims& d, const MoeLayerDev& L, const float* bias, const uint16_t* x_bf16,
                            float* y, const MoeBatchWs& ws, int32_t* ids_out, float* w_out, hipStream_t s) {
    const uint32_t pairs = d.T * d.K + (d.SI ? d.T : 0u);
    // from sweeps of config 5: gate/up 8-tile items, one tile per wave, 6 steps
    // in flight (5: same, 8: +0.7 %; 4-tile items with two tokens a group and
    // two workgroups a CU: +5.8 %, with four tokens: +20 %; 8-tile items with
    // two tokens: +6.6 %); down 8-tile items, two tiles per wave, 3 steps in
    // flight (4: +0.2 %, 6: +3 % with 201 VGPRs)
#ifndef HK_BATCH_GU_D  // (build-time overrides for launch-shape sweeps)
#define HK_BATCH_GU_D 6
#define HK_BATCH_DN_D 3
#endif
#ifndef HK_BATCH_GU_TPI
#define HK_BATCH_GU_TPI 8
#define HK_BATCH_GU_TBMAX 4
#endif
    constexpr int GU_TPI = HK_BATCH_GU_TPI, GU_TPW = 1, GU_D = HK_BATCH_GU_D, DN_TPI = 8, DN_TPW = 2, DN_D = HK_BATCH_DN_D;
    const uint32_t gpe_gu = (n_tiles_for(max(d.I, d.SI)) + GU_TPI - 1) / GU_TPI;
    const uint32_t gpe_dn = (n_tiles_for(d.H) + DN_TPI - 1) / DN_TPI;
    const uint32_t ximg = (uint32_t)moe_batch_img_bytes(d.H), aimg = (uint32_t)moe_batch_img_bytes(d.Imax);
    const uint32_t budget = image_lds_budget();
    // 4 tokens per down group too: 8 (the activation images are small) took
    // 237 VGPRs and ran the down kernel 22 % slower
    const uint32_t tb_gu = tokens_per_group(ximg, HK_BATCH_GU_TBMAX, budget), tb_dn = tokens_per_group(aimg, 4u, budget);
    if (tb_gu == 0 || tb_dn == 0) return hipErrorInvalidValue;
    // the kernels' item counts (an upper bound: every active expert routed)
    const uint32_t tbg = tb_gu >= 4 ? 4u : tb_gu >= 2 ? 2u : 1u;
    const uint32_t tbd = tb_dn >= 4 ? 4u : tb_dn >= 2 ? 2u : 1u;
    const uint32_t n_routed = min(d.E, d.T * d.K);
    const uint32_t gu_items = moe_batch_items(gpe_gu, d.SI ? (d.T + tbg - 1) / tbg : 0u, n_routed);
    const uint32_t dn_items = moe_batch_items(gpe_dn, d.SI ? (d.T + tbd - 1) / tbd : 0u, n_routed);
    const uint32_t n_prep = (d.E + 15u) / 16u * d.S + d.T * ((d.H + XPART_COLS - 1) / XPART_COLS);
    hipLaunchKernelGGL(moe_batch_prep_kernel, dim3(n_prep), dim3(64 * RT_WAVES), (size_t)q4_stage_floats(d.H) * sizeof(float),
                       s, d, x_bf16, L.router_w, ws);
    hipLaunchKernelGGL(moe_batch_route_kernel, dim3(d.T), dim3(256), 0, s, d, bias, ws, ids_out, w_out);
    hipLaunchKernelGGL(moe_batch_group_kernel, dim3(1), dim3(1024), 0, s, d, ws);
    // one workgroup per item (the item count is an upper bound; the device
    // count decides): the dispatcher then balances ~1 MB items across the CUs
    // better than a persistent grid (measured: 862 vs 910 us per step)
    const dim3 ggu(gu_items), gdn(dn_items);
    // one tile per wave, 8 waves sharing the staged images
    const dim3 bgu(64 * GU_TPI / GU_TPW), bdn(64 * DN_TPI / DN_TPW);
    if (tb_gu >= 4)
        hipLaunchKernelGGL((moe_batch_gate_up_kernel<4, GU_D, GU_TPW, GU_TPI>), ggu, bgu, (size_t)4 * ximg, s, d, L.table, ws);
    else if (tb_gu >= 2)
        hipLaunchKernelGGL((moe_batch_gate_up_kernel<2, GU_D, GU_TPW, GU_TPI>), ggu, bgu, (size_t)2 * ximg, s, d, L.table, ws);
    else
        hipLaunchKernelGGL((moe_batch_gate_up_kernel<1, GU_D, GU_TPW, GU_TPI>), ggu, bgu, (size_t)ximg, s, d, L.table, ws);
#ifndef HK_BATCH_AIMG_COLS
#define HK_BATCH_AIMG_COLS 2048  // activation image columns per block (512: +0.4 us; build-time override)
#endif
    hipLaunchKernelGGL(moe_batch_act_image_kernel, dim3(pairs, (d.Imax + HK_BATCH_AIMG_COLS - 1) / HK_BATCH_AIMG_COLS), dim3(256),
                       (size_t)q4_stage_floats(d.Imax) * sizeof(float), s, d, ws);
    if (tb_dn >= 4)
        hipLaunchKernelGGL((moe_batch_down_kernel<4, DN_D, DN_TPW, DN_TPI>), gdn, bdn, (size_t)4 * aimg, s, d, L.table, ws);
    else if (tb_dn >= 2)
        hipLaunchKernelGGL((moe_batch_down_kernel<2, DN_D, DN_TPW, DN_TPI>), gdn, bdn, (size_t)2 * aimg, s, d, L.table, ws);
    else
        hipLaunchKernelGGL((moe_batch_down_kernel<1, DN_D, DN_TPW, DN_TPI>), gdn, bdn, (size_t)aimg, s, d, L.table, ws);
    hipLaunchKernelGGL(moe_batch_combine_kernel, dim3(d.T, (d.H + 255u) / 256u), dim3(256), 0, s, d, ws, y);
    return hipGetLastError();
}

}  // namespace hk
