// hk_moe_stack.hip -- every MoE decode layer of one token in a single
// persistent cooperative launch (configs 3-4).
//
// The per-layer path (hk_moe.hip) needs three launches per layer because a
// layer has three points where every workgroup needs every other's output:
// the router logits, the activations, and the next h.  On gfx950 each launch
// boundary costs ~1.4 us, and the kernel behind it pays its argument and
// first loads again; a device-scope fence inside a kernel lowers to an L2
// writeback (microseconds), and a counter every block increments serializes
// on one address.  Here every workgroup stays resident for the whole token
// (cooperative launch: the grid is admitted only if it fits at once) and the
// three hand-offs go through flag-tagged words instead:
//
//   word = {value bits (low 32), tag (high 32)}, written with one 64-bit
//   system-scope atomic store and polled with system-scope atomic loads.
//
// Each word carries its own validity, so no fence, counter or barrier orders
// different words, and a reader waits only for the words it uses.  Every
// layer has its own words (nothing is overwritten within a launch) and every
// word of a launch carries the launch's tag (the host advances it per call,
// so a word left by an earlier call never matches).
//
// Cost is in the polls and the fan-out, not the hand-off itself (a word
// crosses between XCDs in ~0.5 us).  ~500 waves polling the same lines, or
// all reading h with loads that bypass the caches, queue on a few memory
// channels and starve the producers.  So each producer, right behind its
// output stores, stores one ready word into RDY_REP replicas (the readers
// spread over them); a reader polls only the ready words of its producers
// with one wave, then reads the outputs with ordinary loads, so the L2 of
// each XCD serves the fan-out (a word read before it arrived shows an older
// tag: the read then falls back to polling the words past the caches).  Roles by block:
//   route   (E/4 + 1 blocks): prefetch the layer's router rows, wait for h,
//           RMSNorm(1+w), one logit per wave (the last block: the shared-gate
//           logit) -- moe_route_kernel's arithmetic.
//   gate/up (one per 16-row tile and slot): wait for h, RMSNorm and the x
//           image of xn in LDS, wait for the logits and rank them (routed
//           slots), then moe_gate_up_kernel's compute; SwiGLU rows out as
//           tagged words.
//   down    (one per 16-row tile of h): wait for the logits, rank them, issue
//           every slot's weights, then per slot wait for its activations,
//           build its image and run it; combine in slot order, h += combined
//           as tagged words (the rows this block owns stay in registers).
// Every output is bit-identical to the per-layer path's.  Every wait is
// bounded: one that runs out sets the launch's abort word and a status bit,
// and every wait then returns at once, so the launch always ends (its output
// is then undefined and the status says so).
#include "hk_internal.h"
#include "hk_mfma.h"
#include "hk_moe.h"
#include "hk_router_dev.h"

namespace hk {

namespace {

constexpr int ROW_PRE = 8;                 // router row float4 per lane held in registers (2048 columns)
// gate/up steps in flight (a mixed step of both organs is 24 registers, a Q4 step 10)
template <int KIND>
constexpr int gu_depth() { return KIND == HK_MIXED ? 2 : 4; }
// down steps in flight per slot (a wave holds every one of its slots' steps
// across the activation waits; a mixed step is 12 registers, a Q4 step 5)
template <int KIND>
constexpr int dn_depth() { return KIND == HK_MIXED ? 1 : 3; }
constexpr int DN_SPW = 3;  // slots per down wave: top_k + shared <= 12

// Stores and polls at system scope: they write through and read past the L2
// of the XCD (each XCD's L2 is not coherent with the others').
__device__ __forceinline__ void ll_put(uint64_t* p, float v, uint32_t tag) {
    __hip_atomic_store(p, ((uint64_t)tag << 32) | (uint64_t)__float_as_uint(v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_SYSTEM);
}
__device__ __forceinline__ uint64_t ll_get(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
}
// An ordinary 64-bit load (single-copy atomic), which the caches may serve.
__device__ __forceinline__ uint64_t ll_get_cached(const uint64_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Ready word i of a ready array, into every replica (lanes 0..RDY_REP-1 of
// the calling wave store), right behind the wave's output stores.  Not
// waiting for those stores to complete first saves their acknowledgement
// (~0.5 us) on every hand-off; a reader that sees the ready word before an
// output word reads an older tag there and polls that word.
__device__ __forceinline__ void put_ready(uint64_t* rdy, uint32_t rstride, uint32_t i, uint32_t lane, uint32_t tag) {
    if (lane < RDY_REP) ll_put(rdy + (size_t)lane * rstride + i, 0.0f, tag);
}

enum : uint32_t { WAIT_OK = 0, WAIT_ABORT = 1 };

// Waits until the N words p[idx[j]] this lane names carry `tag` and returns
// their values; every lane of the wave takes part (wave-uniform result).
// WAIT_ABORT: the launch gave up.
template <int N>
__device__ uint32_t ll_wait(const uint64_t* p, const uint32_t (&idx)[N], uint32_t tag, float (&out)[N],
                            const StackArgs& a) {
    uint32_t* abort = a.abort;
    for (uint32_t spin = 0;; ++spin) {
        uint64_t w[N];
#pragma unroll
        for (int j = 0; j < N; ++j) w[j] = ll_get(p + idx[j]);
        const uint32_t ab = __hip_atomic_load(abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        bool ok = true;
#pragma unroll
        for (int j = 0; j < N; ++j) ok = ok && (uint32_t)(w[j] >> 32) == tag;
        if (__all(ok)) {
#pragma unroll
            for (int j = 0; j < N; ++j) out[j] = __uint_as_float((uint32_t)w[j]);
            return WAIT_OK;
        }
        if ((int32_t)(ab - a.tag) >= 0) return WAIT_ABORT;  // any wait of this launch gave up
        if (spin >= a.spin_limit) {
            __hip_atomic_store(abort, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (__lane_id() == 0) atomicOr(a.status, HK_DEVERR_STALL);
            return WAIT_ABORT;
        }
        __builtin_amdgcn_s_sleep(1);
    }
}

// A chunk of 8 consecutive tagged words at bp, read like ll_read in two
// parts so that several chunks can be in flight: chunk_issue (ordinary
// loads), then chunk_finish (tag check; the bounded poll past the caches if
// any word is not there yet).
__device__ __forceinline__ void chunk_issue(const uint64_t* bp, uint64_t (&w)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) w[e] = ll_get_cached(bp + e);
}
__device__ uint32_t chunk_finish(const uint64_t* bp, uint64_t (&w)[8], uint32_t tag, float4 (&out)[2],
                                 const StackArgs& a) {
    for (uint32_t spin = 0;; ++spin) {
        bool ok = true;
#pragma unroll
        for (int e = 0; e < 8; ++e) ok = ok && (uint32_t)(w[e] >> 32) == tag;
        if (__all(ok)) {
            out[0] = make_float4(__uint_as_float((uint32_t)w[0]), __uint_as_float((uint32_t)w[1]),
                                 __uint_as_float((uint32_t)w[2]), __uint_as_float((uint32_t)w[3]));
            out[1] = make_float4(__uint_as_float((uint32_t)w[4]), __uint_as_float((uint32_t)w[5]),
                                 __uint_as_float((uint32_t)w[6]), __uint_as_float((uint32_t)w[7]));
            return WAIT_OK;
        }
        const uint32_t ab = __hip_atomic_load(a.abort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        if ((int32_t)(ab - a.tag) >= 0) return WAIT_ABORT;
        if (spin >= a.spin_limit) {
            __hip_atomic_store(a.abort, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
            if (__lane_id() == 0) atomicOr(a.status, HK_DEVERR_STALL);
            return WAIT_ABORT;
        }
        __builtin_amdgcn_s_sleep(1);
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = ll_get(bp + e);
    }
}

// threadIdx.x made opaque once per layer: everything derived from it is
// recomputed per layer instead of hoisted out of the layer loop and held in
// registers for the whole token (which spills).
__device__ __forceinline__ uint32_t fresh_tid() {
    uint32_t t = threadIdx.x;
    asm volatile("" : "+v"(t));
    return t;
}

__device__ __forceinline__ float dot4s(const float4& a, const float4& b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// Waits (one wave) until the n <= 64 NR ready words rdy[] carry `tag`; the
// block's replica is picked by its index.
template <int NR>
__device__ uint32_t wait_ready(const uint64_t* rdy, uint32_t rstride, uint32_t n, uint32_t lane, uint32_t tag,
                               const StackArgs& a) {
    uint32_t idx[NR];
    float v[NR];
    const uint32_t r0 = (blockIdx.x % RDY_REP) * rstride;
#pragma unroll
    for (int j = 0; j < NR; ++j) idx[j] = r0 + min(lane + 64u * (uint32_t)j, n - 1u);
    return ll_wait<NR>(rdy, idx, tag, v, a);
}

// The words p[idx[j]] once their producers' ready words were seen: ordinary
// loads, falling back to the bounded poll if any word is not there yet.
template <int N>
__device__ uint32_t ll_read(const uint64_t* p, const uint32_t (&idx)[N], uint32_t tag, float (&out)[N],
                            const StackArgs& a) {
    uint64_t w[N];
#pragma unroll
    for (int j = 0; j < N; ++j) w[j] = ll_get_cached(p + idx[j]);
    bool ok = true;
#pragma unroll
    for (int j = 0; j < N; ++j) ok = ok && (uint32_t)(w[j] >> 32) == tag;
    if (__all(ok)) {
#pragma unroll
        for (int j = 0; j < N; ++j) out[j] = __uint_as_float((uint32_t)w[j]);
        return WAIT_OK;
    }
    return ll_wait<N>(p, idx, tag, out, a);
}

// h of the current layer from its tagged words: thread t holds float4 j =
// t + 256 k (k < HP), values past H dropped; returns the wait state.  Every
// thread of the block calls it: wave 0 polls the down tiles' ready words
// while the other waves sit at the barrier, then every thread reads its words
// once (a poll of all of h by every wave of ~500 blocks is tens of MB per
// round of uncached reads, enough to starve the producers).
template <int HP>
__device__ uint32_t wait_h(const StackArgs& a, uint32_t l, uint32_t tid, float4 (&hv)[HP]) {
    const uint32_t n4 = a.d.H / 4u, tag = a.tag;
    if (tid < 64u)
        (void)wait_ready<2>(a.h_rdy + (size_t)l * RDY_REP * a.hrs, a.hrs, (a.d.H + 15u) / 16u, tid, tag, a);
    __syncthreads();
    uint32_t idx[4 * HP];
    float v[4 * HP];
#pragma unroll
    for (int k = 0; k < HP; ++k) {
        const uint32_t j = min(tid + 256u * (uint32_t)k, n4 - 1u);
#pragma unroll
        for (int e = 0; e < 4; ++e) idx[4 * k + e] = 4u * j + (uint32_t)e;
    }
    const uint32_t st = ll_read<4 * HP>(a.h + (size_t)l * a.hs, idx, tag, v, a);
#pragma unroll
    for (int k = 0; k < HP; ++k) hv[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
    return st;
}

// xn = RMSNorm(1+w)(h) into LDS (the route kernel's order of operations).
template <int HP>
__device__ void rmsnorm_to_lds(const StackArgs& a, uint32_t tid, const float4 (&hv)[HP], const float4 (&gv)[HP],
                               float* xn, float* red) {
    const uint32_t n4 = a.d.H / 4u;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < HP; ++k) ss += tid + 256u * k < n4 ? dot4s(hv[k], hv[k]) : 0.0f;
    const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)a.d.H + a.d.eps);
    float4* x4 = reinterpret_cast<float4*>(xn);
#pragma unroll
    for (int k = 0; k < HP; ++k) {
        const uint32_t j = tid + 256u * k;
        if (j < n4)
            x4[j] = make_float4(hv[k].x * inv * (1.0f + gv[k].x), hv[k].y * inv * (1.0f + gv[k].y),
                                hv[k].z * inv * (1.0f + gv[k].z), hv[k].w * inv * (1.0f + gv[k].w));
    }
    __syncthreads();
}

template <int HP>
__device__ void load_norm(const StackArgs& a, uint32_t tid, const MoeLayerDev& L, float4 (&gv)[HP]) {
    const uint32_t n4 = a.d.H / 4u;
    const float4* g4 = reinterpret_cast<const float4*>(L.norm_w);
#pragma unroll
    for (int k = 0; k < HP; ++k) gv[k] = ldg(g4 + min(tid + 256u * (uint32_t)k, n4 - 1u));
}

// Wave 0: the logits (and the shared-gate logit) of the layer into LDS.
template <int NPL>
__device__ uint32_t wait_logits(const StackArgs& a, uint32_t l, uint32_t tid, float* lg, bool with_gate) {
    const uint32_t lane = tid & 63u, E = a.d.E, tag = a.tag;
    (void)wait_ready<3>(a.l_rdy + (size_t)l * RDY_REP * a.lrs, a.lrs, (E + 3u) / 4u + 1u, lane, tag, a);
    uint32_t idx[NPL + 1];
    float v[NPL + 1];
#pragma unroll
    for (int j = 0; j < NPL; ++j) idx[j] = min(lane + 64u * (uint32_t)j, E - 1u);
    idx[NPL] = with_gate ? E : E - 1u;
    const uint32_t st = ll_read<NPL + 1>(a.logits + (size_t)l * a.ls, idx, tag, v, a);
#pragma unroll
    for (int j = 0; j < NPL; ++j)
        if (lane + 64u * j < E) lg[lane + 64u * j] = v[j];
    if (lane == 0) lg[E] = v[NPL];
    return st;
}

// ------------------------------------------------------------------ route role

template <int KIND, int HP>
__device__ void route_role(const StackArgs& a, uint32_t b, uint8_t* lds) {
    float* xn = reinterpret_cast<float*>(lds);
    __shared__ float red[4];
    const uint32_t wave = threadIdx.x >> 6, nrb = (a.d.E + 3u) / 4u, n4 = a.d.H / 4u;
    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const MoeLayerDev L = a.layers[l];
        const uint32_t tid = fresh_tid(), lane = tid & 63u;
        // this wave's row: a router row, or the shared-expert gate (last block, wave 0)
        const float* wrow = nullptr;
        uint32_t out = 0xFFFFFFFFu;
        if (b < nrb) {
            const uint32_t row = b * 4u + wave;
            if (row < a.d.E) {
                wrow = L.router_w + (size_t)row * a.d.H;
                out = row;
            }
        } else if (wave == 0 && L.gate_w) {
            wrow = L.gate_w;
            out = a.d.E;
        }
        // the weights first: they wait for nothing
        float4 gv[HP];
        load_norm<HP>(a, tid, L, gv);
        const float4* w4 = reinterpret_cast<const float4*>(wrow ? wrow : L.router_w);
        float4 wv[ROW_PRE];
#pragma unroll
        for (int k = 0; k < ROW_PRE; ++k) wv[k] = ldg(w4 + min(lane + 64u * (uint32_t)k, n4 - 1u));
        float4 hv[HP];
        const uint32_t st = wait_h<HP>(a, l, tid, hv);
        rmsnorm_to_lds<HP>(a, tid, hv, gv, xn, red);
        if (wrow) {
            const float4* x4 = reinterpret_cast<const float4*>(xn);
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < ROW_PRE; ++k) {
                const uint32_t j = lane + 64u * k;
                if (j < n4) acc += dot4s(wv[k], x4[j]);
            }
            for (uint32_t j = lane + 64u * ROW_PRE; j < n4; j += 64u) acc += dot4s(w4[j], x4[j]);
            acc = wave_sum(acc);
            if (lane == 0 && st == WAIT_OK) ll_put(a.logits + (size_t)l * a.ls + out, acc, a.tag);
        }
        __syncthreads();  // xn is rewritten next layer
        if (wave == 0 && st == WAIT_OK) put_ready(a.l_rdy + (size_t)l * RDY_REP * a.lrs, a.lrs, b, lane, a.tag);
    }
}

// ------------------------------------------------------------------ gate/up role

template <int KIND, int NPL, int HP>
__device__ void gate_up_role(const StackArgs& a, uint32_t gi, uint8_t* lds) {
    const MoeDims& d = a.d;
    const uint32_t T = gi % a.gu_tiles, slot = gi / a.gu_tiles;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const bool routed = slot < d.K;
    const uint32_t S = n_steps_for(KIND, d.H), ib = (uint32_t)x_lds_bytes<KIND>(S);
    const uint32_t nch = S * tile_step_cols(KIND) / 8u;
    uint8_t* img = lds;
    float* part = reinterpret_cast<float*>(lds + ib);                       // [4 waves][32]
    float* xn = part + 128;                                                  // [H, whole steps]
    float* lg = xn + S * tile_step_cols(KIND);                              // [E + 1]
    __shared__ TopkLds tk;
    __shared__ float red[4];
    __shared__ int32_t sel_id;
    __shared__ uint32_t state;
    const uint32_t per = (S + 3u) / 4u;
    const uint32_t s0 = min(wave * per, S), nst = min(s0 + per, S) - s0;
    if (threadIdx.x == 0) state = WAIT_OK;
    __syncthreads();
    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const MoeLayerDev L = a.layers[l];
        const uint32_t tid = fresh_tid(), lane = tid & 63u, q = lane >> 4;
        const uint32_t base = routed ? 0u : d.E * 3u;
        const OrganView g0 = L.table[base], u0 = L.table[base + 1u];
        float4 gv[HP];
        load_norm<HP>(a, tid, L, gv);
        float4 hv[HP];
        const uint32_t sth = wait_h<HP>(a, l, tid, hv);
        if (sth != WAIT_OK && lane == 0) atomicMax(&state, sth);
        rmsnorm_to_lds<HP>(a, tid, hv, gv, xn, red);
        // the x image of xn (E = 0), 512 columns per wave
        for (uint32_t cb = wave * 64u; cb < nch; cb += 256u) {
            bool bad = false;
            const uint32_t ce = min(cb + 64u, nch);
            const bool flag = T == 0 && slot == 0;
            image_wave<KIND>(lane, xn, d.H, img + (size_t)(cb * 8u / tile_step_cols(KIND)) * Kcfg<KIND>::P * A_TILE_STRIDE,
                             reinterpret_cast<float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE) +
                                 (size_t)(cb * 8u / Kcfg<KIND>::SXG) * Kcfg<KIND>::SXW,
                             cb, ce, &bad);
            if (flag && sth == WAIT_OK && __ballot(bad) != 0 && lane == 0) atomicOr(a.status, HK_DEVERR_NONFINITE);
        }
        if (routed && wave == 0) {
            const uint32_t stl = wait_logits<NPL>(a, l, tid, lg, false);
            if (stl != WAIT_OK && lane == 0) atomicMax(&state, stl);
            const ArgBest mine = softmax_topk_wave<NPL>(lg, d.E, d.K, 1, nullptr, nullptr, nullptr, &tk, (int)lane,
                                                        d.tie_eps);
            if (lane == slot) sel_id = mine.i;
        }
        __syncthreads();
        // ids from LDS made wave-uniform, so the organ views stay in scalar registers
        const int32_t id = routed ? __builtin_amdgcn_readfirstlane(sel_id) : (int32_t)d.E;
        const bool ok = state == WAIT_OK && (!routed || (id >= 0 && (uint32_t)id < d.E));
        if (state == WAIT_OK && !ok && T == 0 && threadIdx.x == 0) atomicOr(a.status, HK_DEVERR_ROUTE);
        const OrganView g = routed ? advance_view(g0, ok ? (uint32_t)id : 0u, L.stride) : g0;
        const OrganView u = routed ? advance_view(u0, ok ? (uint32_t)id : 0u, L.stride) : u0;
        const bool active = ok && T < g.n_tiles;
        float acc[2] = {0.0f, 0.0f};
        if (active) {
            constexpr int GU_D = gu_depth<KIND>();
            Frag<KIND, 2> f[GU_D];
#pragma unroll
            for (int k = 0; k < GU_D; ++k)
                if ((uint32_t)k < nst) {
                    fetch_one<KIND, 2>(g, T, s0 + k, lane, f[k], 0);
                    fetch_one<KIND, 2>(u, T, s0 + k, lane, f[k], 1);
                }
            const ImageA A{img, a_lane_offset((int)lane)};
            const float* SX = reinterpret_cast<const float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
            for (uint32_t it = 0; it < nst; it += GU_D) {
#pragma unroll
                for (int k = 0; k < GU_D; ++k) {
                    if (it + k >= nst) break;
                    compute_step<KIND, 2>(f[k], s0 + it + k, A, SX, (int)q, acc);
                    const uint32_t nx = it + GU_D + k;
                    if (nx < nst) {
                        fetch_one<KIND, 2>(g, T, s0 + nx, lane, f[k], 0);
                        fetch_one<KIND, 2>(u, T, s0 + nx, lane, f[k], 1);
                    }
                }
            }
        }
        const float gs = tile_row_sum(acc[0]), us = tile_row_sum(acc[1]);
        if (lane < 16) {
            part[wave * 32u + lane] = gs;
            part[wave * 32u + 16u + lane] = us;
        }
        __syncthreads();
        if (active && threadIdx.x < 16) {
            float gvv = 0.f, uvv = 0.f;
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                gvv += part[w * 32 + threadIdx.x];
                uvv += part[w * 32 + 16 + threadIdx.x];
            }
            // the image has E = 0: no rescale
            const uint32_t row = T * 16u + threadIdx.x;
            if (row < g.rows)
                ll_put(a.act + (size_t)l * a.as + (size_t)slot * d.Imax + row, (gvv / (1.0f + expf(-gvv))) * uvv, a.tag);
            put_ready(a.a_rdy + (size_t)l * RDY_REP * a.ars, a.ars, slot * a.gu_tiles + T, threadIdx.x, a.tag);
        }
        if (threadIdx.x == 0) state = WAIT_OK;  // read by every thread before the barrier above
        __syncthreads();  // LDS is rewritten next layer
    }
}

// ------------------------------------------------------------------ down role

template <int KIND, int NPL>
__device__ void down_role(const StackArgs& a, uint32_t T, uint8_t* lds) {
    const MoeDims& d = a.d;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    const uint32_t smax = n_steps_for(KIND, d.Imax);
    const uint32_t img_stride = (uint32_t)x_lds_bytes<KIND>(smax);
    uint8_t* img = lds + (size_t)wave * DN_SPW * img_stride;                   // [DN_SPW] per wave
    float* part = reinterpret_cast<float*>(lds + 4u * DN_SPW * img_stride);   // [slots][16]
    float* lg = part + 16u * slots;                                            // [E + 1]
    __shared__ TopkLds tk;
    __shared__ int32_t sel_i[HK_TOPK_MAX];
    __shared__ float sel_w[HK_TOPK_MAX];
    __shared__ float gate_v;
    __shared__ uint32_t state;
    const uint32_t row = T * 16u + threadIdx.x;
    for (int j = 0; j < DN_SPW; ++j) image_zero_blocks<KIND>(threadIdx.x & 63u, img + (size_t)j * img_stride, smax);
    // the rows of h this block owns live in registers across the layers
    float hreg = threadIdx.x < 16u && row < d.H ? a.h_in[row] : 0.0f;
    if (threadIdx.x < 16u) {
        if (row < d.H) ll_put(a.h + row, hreg, a.tag);
        put_ready(a.h_rdy, a.hrs, T, threadIdx.x, a.tag);
    }
    for (uint32_t l = 0; l < a.n_layers; ++l) {
        const MoeLayerDev L = a.layers[l];
        const uint32_t tid = fresh_tid(), lane = tid & 63u, q = lane >> 4;
        if (threadIdx.x == 0) state = WAIT_OK;
        __syncthreads();
        if (wave == 0) {
            const uint32_t stl = wait_logits<NPL>(a, l, tid, lg, L.gate_w != nullptr);
            if (stl != WAIT_OK && lane == 0) atomicMax(&state, stl);
            const ArgBest mine = softmax_topk_wave<NPL>(lg, d.E, d.K, 1, nullptr, nullptr,
                                                        T == 0 && stl == WAIT_OK ? a.status : nullptr, &tk, (int)lane,
                                                        d.tie_eps);
            if (lane < d.K) {
                sel_i[lane] = mine.i;
                sel_w[lane] = mine.v;
                if (T == 0 && a.ids) a.ids[(size_t)l * d.K + lane] = mine.i;
                if (T == 0 && a.weights) a.weights[(size_t)l * d.K + lane] = mine.v;
            }
            if (lane == 0) gate_v = L.gate_w ? 1.0f / (1.0f + expf(-lg[d.E])) : 1.0f;
        }
        __syncthreads();
        const bool live = state == WAIT_OK;
        // this wave's slots: wave, wave + 4, ...; every slot's first steps issued before any wait
        constexpr int DN_D = dn_depth<KIND>();
        Frag<KIND, 1> f[DN_SPW][DN_D];
        OrganView o[DN_SPW];
        bool act[DN_SPW];
        uint32_t S[DN_SPW];
#pragma unroll
        for (int j = 0; j < DN_SPW; ++j) {
            const uint32_t s = wave + 4u * (uint32_t)j;
            const bool has = s < slots;
            const bool rt = s < d.K;
            const OrganView o0 = L.table[rt ? 2u : d.E * 3u + 2u];
            const int32_t id = rt ? __builtin_amdgcn_readfirstlane(sel_i[has ? s : 0u]) : (int32_t)d.E;
            const bool ok = live && has && (!rt || (id >= 0 && (uint32_t)id < d.E));
            o[j] = rt ? advance_view(o0, ok ? (uint32_t)id : 0u, L.stride) : o0;
            act[j] = ok && T < o[j].n_tiles;
            S[j] = act[j] ? o[j].steps : 0u;
#pragma unroll
            for (int k = 0; k < DN_D; ++k)
                if ((uint32_t)k < S[j]) fetch_one<KIND, 1>(o[j], T, (uint32_t)k, lane, f[j][k], 0);
        }
        // the wave's slots together: one poll of their producers' ready words,
        // then their activations in rounds of 512 columns (8 per lane per
        // slot), each slot's chunk imaged straight from registers
        uint32_t acols[DN_SPW];
        int jf = -1;  // the first active slot (stands in for inactive ones' indices)
#pragma unroll
        for (int j = DN_SPW - 1; j >= 0; --j) {
            const uint32_t s = wave + 4u * (uint32_t)j;
            acols[j] = act[j] ? (s < d.K ? d.I : d.SI) : 0u;
            if (act[j]) jf = j;
        }
        bool bad = false;
        if (jf >= 0) {
            uint32_t ridx[2 * DN_SPW];
            float rv[2 * DN_SPW];
            const uint32_t r0 = (blockIdx.x % RDY_REP) * a.ars;
#pragma unroll
            for (int j = 0; j < DN_SPW; ++j) {
                const int sj = act[j] ? j : jf;
                const uint32_t s = wave + 4u * (uint32_t)sj, ntl = (acols[sj] + 15u) / 16u;
#pragma unroll
                for (int k = 0; k < 2; ++k) ridx[2 * j + k] = r0 + s * a.gu_tiles + min(lane + 64u * (uint32_t)k, ntl - 1u);
            }
            const uint32_t str = ll_wait<2 * DN_SPW>(a.a_rdy + (size_t)l * RDY_REP * a.ars, ridx, a.tag, rv, a);
            if (str != WAIT_OK && lane == 0) atomicMax(&state, str);
            uint32_t maxc = 0;
#pragma unroll
            for (int j = 0; j < DN_SPW; ++j) maxc = max(maxc, acols[j]);
            for (uint32_t c0 = 0; c0 < maxc; c0 += 512u) {
                // slot j + 1's chunk is in flight while slot j's is imaged
                const uint64_t* bp[DN_SPW];
#pragma unroll
                for (int j = 0; j < DN_SPW; ++j) {
                    // whole chunks (acols is a multiple of 8)
                    const int sj = act[j] ? j : jf;
                    bp[j] = a.act + (size_t)l * a.as + (wave + 4u * (uint32_t)sj) * d.Imax +
                            min(c0 + 8u * lane, acols[sj] - 8u);
                }
                uint64_t w[2][8];
                chunk_issue(bp[0], w[0]);
#pragma unroll
                for (int j = 0; j < DN_SPW; ++j) {
                    if (j + 1 < DN_SPW) chunk_issue(bp[j + 1], w[(j + 1) & 1]);
                    float4 cv[2];
                    const uint32_t sta = chunk_finish(bp[j], w[j & 1], a.tag, cv, a);
                    if (sta != WAIT_OK && lane == 0) atomicMax(&state, sta);
                    const uint32_t ch = c0 / 8u + lane;
                    if (!act[j] || ch >= S[j] * tile_step_cols(KIND) / 8u) continue;
                    if (c0 + 8u * lane >= acols[j]) cv[0] = cv[1] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    uint8_t* im = img + (size_t)j * img_stride;
                    bad |= image_chunk<KIND>(ch, cv, im,
                                             reinterpret_cast<float*>(im + (size_t)S[j] * Kcfg<KIND>::P * A_TILE_STRIDE),
                                             0u, 0u);
                }
            }
        }
        if (__ballot(bad) != 0 && lane == 0) atomicOr(a.status, HK_DEVERR_NONFINITE);
#pragma unroll
        for (int j = 0; j < DN_SPW; ++j) {
            const uint32_t s = wave + 4u * (uint32_t)j;
            if (s >= slots) break;
            float y = 0.0f;
            if (act[j]) {
                const uint8_t* im = img + (size_t)j * img_stride;
                const ImageA A{im, a_lane_offset((int)lane)};
                const float* SX = reinterpret_cast<const float*>(im + (size_t)S[j] * Kcfg<KIND>::P * A_TILE_STRIDE);
                float acc[1] = {0.0f};
                for (uint32_t it = 0; it < S[j]; it += DN_D) {
#pragma unroll
                    for (int k = 0; k < DN_D; ++k) {
                        if (it + k >= S[j]) break;
                        compute_step<KIND, 1>(f[j][k], it + k, A, SX, (int)q, acc);
                        const uint32_t nx = it + DN_D + k;
                        if (nx < S[j]) fetch_one<KIND, 1>(o[j], T, nx, lane, f[j][k], 0);
                    }
                }
                y = tile_row_sum(acc[0]) * (s < d.K ? sel_w[s] : gate_v);
            }
            if (lane < 16) part[s * 16u + lane] = act[j] ? y : 0.0f;
        }
        __syncthreads();
        if (threadIdx.x < 16u) {
            // combined += out_r * w_r in route order, then += gate * shared; h += combined
            float comb = 0.0f;
            for (uint32_t r = 0; r < slots; ++r) comb += part[r * 16u + threadIdx.x];
            hreg = hreg + comb;
            if (row < d.H) {
                if (l + 1u < a.n_layers)
                    ll_put(a.h + (size_t)(l + 1u) * a.hs + row, hreg, a.tag);
                else
                    a.h_out[row] = hreg;
            }
            if (l + 1u < a.n_layers)
                put_ready(a.h_rdy + (size_t)(l + 1u) * RDY_REP * a.hrs, a.hrs, T, threadIdx.x, a.tag);
        }
    }
}

template <int KIND, int NPL, int HP>
__global__ void __launch_bounds__(256, 3) moe_stack_kernel(StackArgs a) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t b = blockIdx.x;
    const uint32_t nr = (a.d.E + 3u) / 4u + 1u;
    if (b < nr)
        route_role<KIND, HP>(a, b, lds);
    else if (b < nr + a.ng)
        gate_up_role<KIND, NPL, HP>(a, b - nr, lds);
    else
        down_role<KIND, NPL>(a, b - nr - a.ng, lds);
}

template <int KIND>
size_t stack_lds(const MoeDims& d) {
    const uint32_t S = n_steps_for(KIND, d.H), hcols = S * tile_step_cols(KIND);
    const size_t gu = x_lds_bytes<KIND>(S) + 128 * 4 + (size_t)hcols * 4 + ((size_t)d.E + 1) * 4;
    const uint32_t slots = d.K + (d.has_shared ? 1u : 0u);
    const size_t img_stride = x_lds_bytes<KIND>(n_steps_for(KIND, d.Imax));
    const size_t dn = 4 * DN_SPW * img_stride + (size_t)slots * 16 * 4 + ((size_t)d.E + 1) * 4;
    const size_t rt = (size_t)hcols * 4;
    return std::max(gu, std::max(dn, rt));
}

template <int KIND, int NPL, int HP>
hipError_t launch_stack_t(const StackArgs& a, int cu_count, hipStream_t s, bool* fits, bool launch) {
    const size_t lds = stack_lds<KIND>(a.d);
    const uint32_t blocks = (a.d.E + 3u) / 4u + 1u + a.ng + n_tiles_for(a.d.H);
    int per_cu = 0;
    hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, moe_stack_kernel<KIND, NPL, HP>, 256, lds);
    if (e != hipSuccess) return e;
    *fits = (size_t)per_cu * (size_t)cu_count >= blocks;
    if (!*fits || !launch) return hipSuccess;
    StackArgs arg = a;
    void* args[] = {&arg};
    return hipLaunchCooperativeKernel(reinterpret_cast<const void*>(moe_stack_kernel<KIND, NPL, HP>), dim3(blocks),
                                      dim3(256), args, (unsigned)lds, s);
}

template <int KIND>
hipError_t launch_stack_k(const StackArgs& a, int cu_count, hipStream_t s, bool* fits, bool launch) {
    return launch_stack_t<KIND, 8, 2>(a, cu_count, s, fits, launch);
}

}  // namespace

// Zero n 64-bit words with a kernel (not a memset node: a caller may capture
// the decode in a graph, and memset nodes have replayed wrongly here).
__global__ void zero_words_kernel(uint64_t* __restrict__ p, size_t n) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0ull;
}

hipError_t launch_zero_words(uint64_t* p, size_t n, hipStream_t s) {
    const size_t blocks = std::min<size_t>((n + 255) / 256, 2048);
    if (blocks) hipLaunchKernelGGL(zero_words_kernel, dim3((uint32_t)blocks), dim3(256), 0, s, p, n);
    return hipGetLastError();
}

size_t moe_stack_lds_bytes(int kind, const MoeDims& d) {
    return kind == HK_Q4 ? stack_lds<HK_Q4>(d) : stack_lds<HK_MIXED>(d);
}

hipError_t launch_moe_stack(int kind, const StackArgs& a, int cu_count, hipStream_t s, bool* fits, bool launch) {
    *fits = false;
    // the shapes whose kernel fits three blocks per CU without spilling:
    // E <= 512 (8 logits per lane), H <= 2048 (2 float4 of h per thread),
    // Imax <= 2048 (128 gate/up tiles: 2 ready words per lane)
    if (a.d.E > 512 || a.d.H > 2048 || a.d.Imax > 2048 || a.d.K + (a.d.has_shared ? 1u : 0u) > 4u * DN_SPW)
        return hipSuccess;
    if (kind == HK_Q4) return launch_stack_k<HK_Q4>(a, cu_count, s, fits, launch);
    if (kind == HK_MIXED) return launch_stack_k<HK_MIXED>(a, cu_count, s, fits, launch);
    return hipSuccess;
}

}  // namespace hk
