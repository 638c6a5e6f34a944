// hk_moe_batch.hip -- the noaux_tc MoE block for a batch of tokens
// (routed_moe, crates/hawking-core/src/gravity_glm.rs:550-600, with
// batched_mlp :515-548): every active expert's weights are streamed from HBM
// once for all of the tokens routed to it (a grouped expert GEMM on the int8
// matrix-core engine of hk_mfma.h, up to MOE_TB tokens per weight fetch).
//
//   1. xprep:    x (bf16) -> f32 rows and the fixed-point x image of each token
//   2. router:   logits partials, split-K over 1024-column slices (f32)
//   3. route:    one block: per token (one wave each) the noaux_tc route
//                (gravity_glm.rs:447-500) on the DPP network, then the tokens
//                grouped by expert (shared expert first, then ascending id)
//   4. gate/up:  per (active expert, 16-row tile): SwiGLU activations of every
//                member token; 4 waves split the columns
//   5. act image: the x image of every (token, expert) activation row
//   6. down:     per (active expert, 16-row tile): w * (down . act) per member
//   7. combine:  y_t = sum over t's experts in ascending id, then + shared
#include "hk_internal.h"
#include "hk_mfma.h"
#include "hk_moe.h"
#include "hk_router_dev.h"

namespace hk {

constexpr int MOE_TB = 4;  // member tokens per weight fetch

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

__global__ void __launch_bounds__(256) moe_batch_xprep_kernel(MoeBatchDims d, const uint16_t* __restrict__ xb,
                                                              MoeBatchWs ws) {
    extern __shared__ __align__(16) float xs[];  // [H]
    __shared__ float red[4];
    const uint32_t t = blockIdx.x;
    for (uint32_t c = threadIdx.x; c < d.H; c += blockDim.x) {
        const float v = bf16_to_f32(xb[(size_t)t * d.H + c]);
        xs[c] = v;
        ws.x32[(size_t)t * d.H + c] = v;
    }
    __syncthreads();
    bool bad = false;
    const int E = prepare_x<HK_Q4>(BlockTeam{}, xs, d.H, n_steps_for(HK_Q4, d.H), ws.ximg + (size_t)t * ws.ximg_stride,
                                   red, &bad);
    if (threadIdx.x == 0) {
        ws.ximg_e[t] = E;
        if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
}

// ------------------------------------------------------------------ 2. router (split-K)

// part[s][t][e] = sum over columns [1024 s, 1024 (s+1)) of W[e][k] x[t][k];
// thread (row r = tid / 32, token tt = tid % 32), x staged in LDS as [k][t].
__global__ void __launch_bounds__(256) moe_batch_router_kernel(MoeBatchDims d, const float* __restrict__ W,
                                                               MoeBatchWs ws) {
    __shared__ float xs[256 * 33];
    const uint32_t tt = threadIdx.x & 31u;
    const uint32_t r = blockIdx.x * 8u + (threadIdx.x >> 5), s = blockIdx.y;
    const uint32_t k0 = s * MOE_BATCH_ROUTER_COLS, k1 = min(k0 + MOE_BATCH_ROUTER_COLS, d.H);
    const bool row_ok = r < d.E;
    const float* wr = W + (size_t)(row_ok ? r : 0u) * d.H;
    for (uint32_t tb = 0; tb < d.T; tb += 32u) {
        float acc = 0.f;
        for (uint32_t kc = k0; kc < k1; kc += 256u) {
            const uint32_t kn = min(256u, k1 - kc);
            __syncthreads();
            for (uint32_t idx = threadIdx.x; idx < 32u * 256u; idx += blockDim.x) {
                const uint32_t t = idx >> 8, k = idx & 255u;
                xs[k * 33u + t] = (tb + t < d.T && k < kn) ? ws.x32[(size_t)(tb + t) * d.H + kc + k] : 0.f;
            }
            __syncthreads();
            if (row_ok) {
                for (uint32_t k = 0; k < kn; k += 4u) {
                    const float4 w4 = *reinterpret_cast<const float4*>(wr + kc + k);
                    acc += w4.x * xs[k * 33u + tt] + w4.y * xs[(k + 1u) * 33u + tt] + w4.z * xs[(k + 2u) * 33u + tt] +
                           w4.w * xs[(k + 3u) * 33u + tt];
                }
            }
        }
        if (row_ok && tb + tt < d.T) ws.part[((size_t)s * d.T + tb + tt) * d.E + r] = acc;
    }
}

// ------------------------------------------------------------------ 3. route + group

__global__ void __launch_bounds__(1024) moe_batch_route_kernel(MoeBatchDims d, const float* __restrict__ bias,
                                                               MoeBatchWs ws, int32_t* ids_out, float* w_out) {
    constexpr int NPL = MOE_BATCH_MAX_EXPERTS / 64;
    constexpr uint32_t MAXP = MOE_BATCH_MAX_TOKENS * 16;
    __shared__ float corr[16][MOE_BATCH_MAX_EXPERTS];
    __shared__ int32_t sids[MAXP];
    __shared__ float sw[MAXP];
    __shared__ uint32_t cnt[MOE_BATCH_MAX_EXPERTS], fill[MOE_BATCH_MAX_EXPERTS], start[MOE_BATCH_MAX_EXPERTS];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
    const uint32_t E = d.E, K = d.K, per = d.E / d.n_group;
    for (uint32_t e = threadIdx.x; e < E; e += blockDim.x) {
        cnt[e] = 0;
        fill[e] = 0;
    }
    // ---- noaux_tc per token, one wave per token
    for (uint32_t t = wave; t < d.T; t += 16u) {
        float sc[NPL], cv[NPL];
        uint32_t bad = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const uint32_t i = (uint32_t)lane + 64u * j;
            sc[j] = 0.f;
            cv[j] = -INFINITY;
            if (i < E) {
                float l = 0.f;
                for (uint32_t s = 0; s < d.S; ++s) l += ws.part[((size_t)s * d.T + t) * E + i];
                if (!isfinite(l)) bad = 1;
                sc[j] = 1.0f / (1.0f + expf(-l));
                cv[j] = sc[j] + bias[i];
                corr[wave][i] = cv[j];
            }
        }
        if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
        wave_lds_sync();
        // group strength = sum of its best two corrected scores (topk_desc order)
        uint64_t gkey = 0;
        if ((uint32_t)lane < d.n_group) {
            const float* sl = corr[wave] + (size_t)lane * per;
            uint32_t b0 = 0;
            for (uint32_t i = 1; i < per; ++i)
                if (sl[i] > sl[b0]) b0 = i;
            float gs = -0.0f + sl[b0];
            if (per >= 2) {
                uint32_t b1 = b0 == 0 ? 1u : 0u;
                for (uint32_t i = 0; i < per; ++i)
                    if (i != b0 && (sl[i] > sl[b1] || (sl[i] == sl[b1] && i < b1))) b1 = i;
                gs = gs + sl[b1];
            }
            gkey = order_key(gs, (uint32_t)lane);
        }
        uint64_t chosen = 0;
        for (uint32_t c = 0; c < d.topk_group; ++c) {
            const uint64_t w = wave_max_key(gkey);
            const uint32_t g = ~(uint32_t)w;
            chosen |= 1ull << g;
            if ((uint32_t)lane == g) gkey = 0;
        }
        // only experts inside a chosen group compete (others at -inf)
        uint64_t key[NPL];
        uint64_t best = 0;
#pragma unroll
        for (int j = 0; j < NPL; ++j) {
            const uint32_t i = (uint32_t)lane + 64u * j;
            key[j] = i < E ? order_key(((chosen >> (i / per)) & 1ull) ? cv[j] : -INFINITY, i) : 0ull;
            best = key[j] > best ? key[j] : best;
        }
        for (uint32_t r = 0; r < K; ++r) {
            const uint64_t w = wave_max_key(best);
            const uint32_t id = ~(uint32_t)w;
            if ((id & 63u) == (uint32_t)lane) {
                float s_id = 0.f;
                best = 0;
#pragma unroll
                for (int j = 0; j < NPL; ++j) {
                    if ((uint32_t)j == (id >> 6)) {
                        s_id = sc[j];
                        key[j] = 0;
                    }
                    best = key[j] > best ? key[j] : best;
                }
                sids[t * K + r] = (int32_t)id;
                sw[t * K + r] = s_id;  // weights are the uncorrected scores
            }
        }
        wave_lds_sync();
        if (lane == 0) {
            float total = -0.0f;
            for (uint32_t r = 0; r < K; ++r) total += sw[t * K + r];
            total = total + 1e-20f;
            for (uint32_t r = 0; r < K; ++r) {
                float v = sw[t * K + r];
                if (d.norm_topk_prob) v = v / total;
                sw[t * K + r] = v * d.scaling;
            }
        }
        wave_lds_sync();
        if ((uint32_t)lane < K) {
            const uint32_t p = t * K + (uint32_t)lane;
            ws.ids[p] = sids[p];
            ws.w[p] = sw[p];
            if (ids_out) ids_out[p] = sids[p];
            if (w_out) w_out[p] = sw[p];
        }
    }
    __syncthreads();
    // ---- group the (token, slot) pairs by expert
    const uint32_t np = d.T * K, has_shared = d.SI ? 1u : 0u;
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
    // each token's slots in ascending expert id (the combine order)
    for (uint32_t t = threadIdx.x; t < d.T; t += blockDim.x) {
        int32_t o[16];
        for (uint32_t r = 0; r < K; ++r) {
            uint32_t j = r;
            while (j > 0 && sids[t * K + (uint32_t)o[j - 1]] > sids[t * K + r]) {
                o[j] = o[j - 1];
                --j;
            }
            o[j] = (int32_t)r;
        }
        for (uint32_t r = 0; r < K; ++r) ws.order[t * K + r] = o[r];
    }
}

// ------------------------------------------------------------------ 4. gate/up (grouped)

// One fetched step of the gate and up tiles plus the A operands and column
// sums of up to MOE_TB member tokens.
struct GuStep {
    Frag<HK_Q4, 2> f;
    v4i alo[MOE_TB], ahi[MOE_TB];
    float sx[MOE_TB];
};

__device__ __forceinline__ void gu_fetch(const OrganView& g, const OrganView& u, uint32_t T, uint32_t t, int lane,
                                         uint32_t aoff, int q, const uint8_t* const* img, uint32_t steps_x, uint32_t nm,
                                         GuStep& st) {
    fetch_one<HK_Q4, 2>(g, T, t, lane, st.f, 0);
    fetch_one<HK_Q4, 2>(u, T, t, lane, st.f, 1);
#pragma unroll
    for (int j = 0; j < MOE_TB; ++j) {
        if ((uint32_t)j < nm) {
            const uint8_t* ib = img[j] + (size_t)t * 2u * A_TILE_STRIDE + aoff;
            st.alo[j] = *reinterpret_cast<const v4i*>(ib);
            st.ahi[j] = *reinterpret_cast<const v4i*>(ib + A_TILE_STRIDE);
            st.sx[j] = reinterpret_cast<const float*>(img[j] + (size_t)steps_x * 2u * A_TILE_STRIDE)[4u * t + (uint32_t)q];
        }
    }
}

template <int R>
__device__ __forceinline__ void q4_tokens(const Frag<HK_Q4, R>& f, const v4i* alo, const v4i* ahi, const float* sx,
                                          uint32_t nm, float (*acc)[R]) {
    const uint32_t m = 0x0F0F0F0Fu;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const v4i lo = {(int)(f.v[r].x & m), (int)(f.v[r].y & m), (int)(f.v[r].z & m), (int)(f.v[r].w & m)};
        const v4i hi = {(int)((f.v[r].x >> 4) & m), (int)((f.v[r].y >> 4) & m), (int)((f.v[r].z >> 4) & m),
                        (int)((f.v[r].w >> 4) & m)};
#pragma unroll
        for (int j = 0; j < MOE_TB; ++j) {
            if ((uint32_t)j < nm) {
                v4i c = mfma_i8(alo[j], lo, v4i{0, 0, 0, 0});
                c = mfma_i8(ahi[j], hi, c);
                acc[j][r] += f.s[r] * (combine_limbs(c) - 8.0f * sx[j]);
            }
        }
    }
}

template <int D>
__global__ void __launch_bounds__(256) moe_batch_gate_up_kernel(MoeBatchDims d, const OrganView* __restrict__ table,
                                                                MoeBatchWs ws) {
    __shared__ float part[4][MOE_TB][2][16];
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t aoff = a_lane_offset(lane);
    const uint32_t tiles = n_tiles_for(max(d.I, d.SI));
    const uint32_t steps_x = n_steps_for(HK_Q4, d.H);
    const uint32_t n_items = __builtin_amdgcn_readfirstlane(*ws.n_active) * tiles;
    for (uint32_t item = blockIdx.x; item < n_items; item += gridDim.x) {
        const uint32_t a = item / tiles, T = item % tiles;
        const uint4 ent = ws.active[a];
        const OrganView g = table[ent.x * 3u + 0u];
        if (T >= g.n_tiles) continue;
        const OrganView u = table[ent.x * 3u + 1u];
        const uint32_t S = g.steps, per = (S + 3u) / 4u;
        const uint32_t s0 = min(wave * per, S), ns = min(s0 + per, S) - s0;
        for (uint32_t m0 = 0; m0 < ent.z; m0 += MOE_TB) {
            const uint32_t nm = min((uint32_t)MOE_TB, ent.z - m0);
            uint32_t pair[MOE_TB];
            const uint8_t* img[MOE_TB];
#pragma unroll
            for (int j = 0; j < MOE_TB; ++j) {
                pair[j] = ws.members[ent.y + m0 + min((uint32_t)j, nm - 1u)];
                img[j] = ws.ximg + (size_t)pair_token(d, pair[j]) * ws.ximg_stride;
            }
            GuStep st[D];
#pragma unroll
            for (int k = 0; k < D; ++k)
                if ((uint32_t)k < ns) gu_fetch(g, u, T, s0 + k, lane, aoff, q, img, steps_x, nm, st[k]);
            float acc[MOE_TB][2] = {};
            for (uint32_t it = 0; it < ns; it += D) {
#pragma unroll
                for (int k = 0; k < D; ++k) {
                    if (it + k >= ns) break;
                    q4_tokens<2>(st[k].f, st[k].alo, st[k].ahi, st[k].sx, nm, acc);
                    const uint32_t nx = it + D + k;
                    if (nx < ns) gu_fetch(g, u, T, s0 + nx, lane, aoff, q, img, steps_x, nm, st[k]);
                }
            }
#pragma unroll
            for (int j = 0; j < MOE_TB; ++j) {
                const float gs = tile_row_sum(acc[j][0]), us = tile_row_sum(acc[j][1]);
                if (lane < 16) {
                    part[wave][j][0][lane] = gs;
                    part[wave][j][1][lane] = us;
                }
            }
            __syncthreads();
            if (threadIdx.x < 16u * nm) {
                const uint32_t j = threadIdx.x >> 4, row = threadIdx.x & 15u;
                float gv = 0.f, uv = 0.f;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    gv += part[w][j][0][row];
                    uv += part[w][j][1][row];
                }
                const int E = ws.ximg_e[pair_token(d, pair[j])];
                gv = ldexpf(gv, -E);
                uv = ldexpf(uv, -E);
                const uint32_t orow = T * 16u + row;
                if (orow < g.rows) ws.act[(size_t)pair[j] * d.Imax + orow] = (gv / (1.0f + expf(-gv))) * uv;
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------ 5. activation images

__global__ void __launch_bounds__(256) moe_batch_act_image_kernel(MoeBatchDims d, MoeBatchWs ws) {
    extern __shared__ __align__(16) float xs[];  // [Imax]
    __shared__ float red[4];
    const uint32_t p = blockIdx.x;
    const uint32_t cols = p < d.T * d.K ? d.I : d.SI;
    const float4* a4 = reinterpret_cast<const float4*>(ws.act + (size_t)p * d.Imax);
    for (uint32_t j = threadIdx.x; j < cols / 4u; j += blockDim.x) reinterpret_cast<float4*>(xs)[j] = a4[j];
    __syncthreads();
    bool bad = false;
    const int E = prepare_x<HK_Q4>(BlockTeam{}, xs, cols, n_steps_for(HK_Q4, cols), ws.aimg + (size_t)p * ws.aimg_stride,
                                   red, &bad);
    if (threadIdx.x == 0) {
        ws.aimg_e[p] = E;
        if (bad) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
}

// ------------------------------------------------------------------ 6. down (grouped)

struct DnStep {
    Frag<HK_Q4, 1> f;
    v4i alo[MOE_TB], ahi[MOE_TB];
    float sx[MOE_TB];
};

__device__ __forceinline__ void dn_fetch(const OrganView& o, uint32_t T, uint32_t t, int lane, uint32_t aoff, int q,
                                         const uint8_t* const* img, uint32_t steps_x, uint32_t nm, DnStep& st) {
    fetch_one<HK_Q4, 1>(o, T, t, lane, st.f, 0);
#pragma unroll
    for (int j = 0; j < MOE_TB; ++j) {
        if ((uint32_t)j < nm) {
            const uint8_t* ib = img[j] + (size_t)t * 2u * A_TILE_STRIDE + aoff;
            st.alo[j] = *reinterpret_cast<const v4i*>(ib);
            st.ahi[j] = *reinterpret_cast<const v4i*>(ib + A_TILE_STRIDE);
            st.sx[j] = reinterpret_cast<const float*>(img[j] + (size_t)steps_x * 2u * A_TILE_STRIDE)[4u * t + (uint32_t)q];
        }
    }
}

template <int D>
__global__ void __launch_bounds__(256) moe_batch_down_kernel(MoeBatchDims d, const OrganView* __restrict__ table,
                                                             MoeBatchWs ws) {
    __shared__ float part[4][MOE_TB][16];
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t aoff = a_lane_offset(lane);
    const uint32_t tiles = n_tiles_for(d.H);
    const uint32_t n_items = __builtin_amdgcn_readfirstlane(*ws.n_active) * tiles;
    const uint32_t np = d.T * d.K;
    for (uint32_t item = blockIdx.x; item < n_items; item += gridDim.x) {
        const uint32_t a = item / tiles, T = item % tiles;
        const uint4 ent = ws.active[a];
        const OrganView o = table[ent.x * 3u + 2u];
        const uint32_t S = o.steps, per = (S + 3u) / 4u;
        const uint32_t s0 = min(wave * per, S), ns = min(s0 + per, S) - s0;
        const uint32_t steps_x = S;  // the activation image has the down organ's column steps
        for (uint32_t m0 = 0; m0 < ent.z; m0 += MOE_TB) {
            const uint32_t nm = min((uint32_t)MOE_TB, ent.z - m0);
            uint32_t pair[MOE_TB];
            const uint8_t* img[MOE_TB];
#pragma unroll
            for (int j = 0; j < MOE_TB; ++j) {
                pair[j] = ws.members[ent.y + m0 + min((uint32_t)j, nm - 1u)];
                img[j] = ws.aimg + (size_t)pair[j] * ws.aimg_stride;
            }
            DnStep st[D];
#pragma unroll
            for (int k = 0; k < D; ++k)
                if ((uint32_t)k < ns) dn_fetch(o, T, s0 + k, lane, aoff, q, img, steps_x, nm, st[k]);
            float acc[MOE_TB][1] = {};
            for (uint32_t it = 0; it < ns; it += D) {
#pragma unroll
                for (int k = 0; k < D; ++k) {
                    if (it + k >= ns) break;
                    q4_tokens<1>(st[k].f, st[k].alo, st[k].ahi, st[k].sx, nm, acc);
                    const uint32_t nx = it + D + k;
                    if (nx < ns) dn_fetch(o, T, s0 + nx, lane, aoff, q, img, steps_x, nm, st[k]);
                }
            }
#pragma unroll
            for (int j = 0; j < MOE_TB; ++j) {
                const float ys = tile_row_sum(acc[j][0]);
                if (lane < 16) part[wave][j][lane] = ys;
            }
            __syncthreads();
            if (threadIdx.x < 16u * nm) {
                const uint32_t j = threadIdx.x >> 4, row = threadIdx.x & 15u;
                const float y = ldexpf(part[0][j][row] + part[1][j][row] + part[2][j][row] + part[3][j][row],
                                       -ws.aimg_e[pair[j]]);
                const float w = pair[j] < np ? ws.w[pair[j]] : 1.0f;
                const uint32_t orow = T * 16u + row;
                if (orow < d.H) ws.ybuf[(size_t)pair[j] * d.H + orow] = y * w;
            }
            __syncthreads();
        }
    }
}

// ------------------------------------------------------------------ 7. combine

__global__ void __launch_bounds__(256) moe_batch_combine_kernel(MoeBatchDims d, MoeBatchWs ws, float* __restrict__ y) {
    const uint32_t t = blockIdx.x, row = blockIdx.y * blockDim.x + threadIdx.x;
    if (row >= d.H) return;
    // routed = 0; routed += o * w over the experts in ascending id; routed += shared
    float acc = 0.0f;
    for (uint32_t j = 0; j < d.K; ++j) acc += ws.ybuf[(size_t)(t * d.K + (uint32_t)ws.order[t * d.K + j]) * d.H + row];
    if (d.SI) acc += ws.ybuf[(size_t)(d.T * d.K + t) * d.H + row];
    y[(size_t)t * d.H + row] = acc;
}

hipError_t launch_moe_batch(const MoeBatchDims& d, const MoeLayerDev& L, const float* bias, const uint16_t* x_bf16,
                            float* y, const MoeBatchWs& ws, int32_t* ids_out, float* w_out, hipStream_t s) {
    const uint32_t pairs = d.T * d.K + (d.SI ? d.T : 0u);
    const uint32_t max_active = min(d.E, d.T * d.K) + (d.SI ? 1u : 0u);
    const uint32_t gu_items = max_active * n_tiles_for(max(d.I, d.SI)), dn_items = max_active * n_tiles_for(d.H);
    hipLaunchKernelGGL(moe_batch_xprep_kernel, dim3(d.T), dim3(256), (size_t)d.H * sizeof(float), s, d, x_bf16, ws);
    hipLaunchKernelGGL(moe_batch_router_kernel, dim3((d.E + 7u) / 8u, d.S), dim3(256), 0, s, d, L.router_w, ws);
    hipLaunchKernelGGL(moe_batch_route_kernel, dim3(1), dim3(1024), 0, s, d, bias, ws, ids_out, w_out);
    hipLaunchKernelGGL(moe_batch_gate_up_kernel<2>, dim3(min(gu_items, 1024u)), dim3(256), 0, s, d, L.table, ws);
    hipLaunchKernelGGL(moe_batch_act_image_kernel, dim3(pairs), dim3(256), (size_t)d.Imax * sizeof(float), s, d, ws);
    hipLaunchKernelGGL(moe_batch_down_kernel<2>, dim3(min(dn_items, 1024u)), dim3(256), 0, s, d, L.table, ws);
    hipLaunchKernelGGL(moe_batch_combine_kernel, dim3(d.T, (d.H + 255u) / 256u), dim3(256), 0, s, d, ws, y);
    return hipGetLastError();
}

}  // namespace hk
