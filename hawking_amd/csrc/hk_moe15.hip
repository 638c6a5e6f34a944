// hk_moe15.hip -- one MoE decode layer of the reference's mixed-1p5-v1
// artifact (moe_suffix of model/qwen80_mixed_hybrid_decode.rs:3636-3752 with
// routed_wave, 2192-2386): routed experts with an HGRAVB01 gate, an HGRAVR02
// up (binary base + Rice residual) and an HGRAVS01 down (y = L (R act));
// router, shared-expert gate and shared expert as HGRAVU01 q8 organs.
//
// Four stream-ordered launches per layer on the int8 matrix-core engine
// (hk_mfma.h), no host round trip; the route never leaves the device:
//   1. route:    every block recomputes xn = RMSNorm(1+w)(h) in LDS.  Router
//                tiles (16 logits each), the shared-expert gate row, and the
//                shared expert's gate and up tiles (one organ per block)
//                each build a q8 x image of xn of their own; the last blocks
//                build the binary x image of xn for the routed gate/up
//                (512 columns each) and publish xn.
//   2. gate/up:  one workgroup per (16-row tile, slot): wave 0 ranks the
//                logits (softmax / top-k / renormalise) to find the slot's
//                expert while the others load the binary image and the
//                tile's row of record starts per expert; both binary bases
//                share each image fetch; the epilogue adds the up's Rice
//                residual in index order (rice_rows_from, its records
//                fetched with the weights) and applies SwiGLU.  Tile 0 of
//                each slot publishes the slot's two down factors.
//   3. down R:   mid_r = R_r act_r (3-bit factor) per (slot, 16-row tile),
//                and the shared expert's q8 down per 16-row tile (its x
//                image formed from silu(gate) * up).
//   4. down L:   one workgroup per 16-row output tile, one wave per slot
//                (y_r = L_r mid_r, an x image per wave); the block combines
//                out = h + (sum_r w_r y_r in slot order + sigmoid(g) y_s).
#include <algorithm>
#include <cmath>
#include <memory>
#include <vector>

#include "hk_internal.h"
#include "hk_mfma.h"
#include "hk_rice.h"
#include "hk_router.h"
#include "hk_router_dev.h"

namespace hk {

constexpr uint32_t M15_MAX_K = 16;  // one wave per slot in the down-L block
constexpr int M15_D = 4;            // steps in flight per wave

struct M15Dims {
    uint32_t H, I, SI, E, K, rank;
    float eps;
    float tie_eps;  // router tie window (route_tie_epsilon); 0 = strict '>'
};

// What differs between one routed expert's gate/up and another's (32 bytes):
// every other field of their views is the same (one shape per layer), and
// within an organ the scales and the residual records sit at offsets from
// the data and the row pointers that are the same for every expert
// (checked at create), so the gate/up kernel copies the whole table into
// LDS while its top-k runs and forms the slot's views with no dependent
// global load.
struct M15Expert {
    const uint8_t* gate;    // gate data
    const uint8_t* up;      // up data
    const uint32_t* rptr;   // up residual row pointers
    float rscale;           // up residual scale
    uint32_t pad;
};
static_assert(sizeof(M15Expert) == 32, "an expert record is two 16-byte pieces");

// The layer's constants: single organs by value, per-expert tables in device memory.
struct M15Dev {
    const float* norm_w;
    OrganView router, sgate, sg, su, sdown;  // sgate.n_tiles = 0: no shared expert
    const OrganView* gate;                   // [E] binary gate
    const OrganView* up;                     // [E] binary base of the HGRAVR02 up
    const ResView* res;                      // [E] its residual
    const OrganView* dr;                     // [E] down right factor (rank x I)
    const OrganView* dl;                     // [E] down left factor (H x rank)
    const M15Expert* ex;                     // [E] compact gate/up records
    // [n_tiles(I) + 1][tstride]: entry (T, e) is expert e's up residual
    // row_ptr[min(16 T, I)], so rows T and T + 1 give every expert's record
    // range of tile T (tstride = E rounded up to a multiple of 4)
    const uint32_t* tstart;
    uint32_t tstride;
    uint32_t g_soff, u_soff, rec_off;        // scales - data (gate, up), recs - row_ptr (bytes)
};

struct M15Ws {
    float* logits;   // [E]
    float* gate;     // [2]: shared-gate logit, sigmoid
    float* xn;       // [H]
    uint8_t* img;    // binary x image of xn
    int32_t* img_e;  // [1]
    float* act;      // [K * I]
    float* act_s;    // [2 SI]: the shared expert's gate, then up projection (SwiGLU formed by their reader)
    float* mid;      // [K * rank]
    float* ys;       // [H] shared expert output (ungated)
    int32_t* ids;    // [K]
    float* w;        // [K]
    OrganView* sel;  // [2K]: right, left factor of each slot
    uint32_t* status;
};

__device__ __forceinline__ float dot4(const float4& a, const float4& b) {
    return a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
}

// xn = h * (1 / sqrt(mean(h^2) + eps)) * (1 + w) (source_qwen80_residual_rms_norm,
// model/qwen80_complete_runtime.rs:6778-6797) held in registers: thread t has chunks t + 256 k
// (8 columns each, k < M15_NC; hidden <= 8 * 256 * M15_NC).  h and w are
// loaded once, unconditionally (index clamped, value dropped past H), so
// every load is in flight before the block's one reduction.  Every thread
// of the 256-thread block calls this (xn_load, then xn_finish; a block
// with weights to fetch issues them between the two, after h and w: vector
// loads retire in issue order, so the norm then waits for h and w only).
constexpr int M15_NC = 4;
struct XnRegs {
    float4 v[M15_NC][2];
};
struct XnW {
    float4 v[M15_NC][2];
};
__device__ __forceinline__ void xn_load(const float* __restrict__ h, const float* __restrict__ w, uint32_t H,
                                        XnRegs& x, XnW& wv) {
    const uint32_t nch = H / 8u;
    const float4* h4 = reinterpret_cast<const float4*>(h);
    const float4* w4 = reinterpret_cast<const float4*>(w);
#pragma unroll
    for (int k = 0; k < M15_NC; ++k) {
        const uint32_t ch = min(threadIdx.x + 256u * (uint32_t)k, nch - 1u);
        x.v[k][0] = ldg(h4 + 2u * ch);
        x.v[k][1] = ldg(h4 + 2u * ch + 1u);
        wv.v[k][0] = ldg(w4 + 2u * ch);
        wv.v[k][1] = ldg(w4 + 2u * ch + 1u);
    }
}
__device__ __forceinline__ void xn_finish(uint32_t H, float eps, float* red, XnRegs& x, const XnW& wv) {
    const uint32_t nch = H / 8u;
    float ss = 0.0f;
#pragma unroll
    for (int k = 0; k < M15_NC; ++k)
        if (threadIdx.x + 256u * (uint32_t)k < nch) ss += dot4(x.v[k][0], x.v[k][0]) + dot4(x.v[k][1], x.v[k][1]);
    const float inv = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < M15_NC; ++k)
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const float4 v = x.v[k][j], g = wv.v[k][j];
            x.v[k][j] = make_float4(v.x * inv * (1.0f + g.x), v.y * inv * (1.0f + g.y), v.z * inv * (1.0f + g.z),
                                    v.w * inv * (1.0f + g.w));
        }
}
__device__ __forceinline__ void block_xn(const float* __restrict__ h, const float* __restrict__ w, uint32_t H,
                                         float eps, float* red, XnRegs& x) {
    XnW wv;
    xn_load(h, w, H, x, wv);
    xn_finish(H, eps, red, x, wv);
}

// The first D steps of [s0, s0 + n) of tile T of organs o[0..R-1].
template <int KIND, int R, int D = M15_D>
__device__ __forceinline__ void fetch_first(const OrganView (&o)[R], uint32_t T, uint32_t s0, uint32_t n, int lane,
                                            Frag<KIND, R> (&f)[D]) {
#pragma unroll
    for (int k = 0; k < D; ++k)
        if ((uint32_t)k < n)
#pragma unroll
            for (int r = 0; r < R; ++r) fetch_one<KIND, R>(o[r], T, s0 + (uint32_t)k, lane, f[k], r);
}

// Steps [s0, s0 + n) against the x image img (S steps), the first D
// already fetched into f; acc[r] in units of 2^-E.
template <int KIND, int R, int D = M15_D>
__device__ __forceinline__ void run_steps(const OrganView (&o)[R], uint32_t T, uint32_t s0, uint32_t n,
                                          const uint8_t* img, uint32_t S, int lane, Frag<KIND, R> (&f)[D],
                                          float* acc) {
    const ImageA A{img, a_lane_offset(lane)};
    const float* SX = reinterpret_cast<const float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    const int q = lane >> 4;
    for (uint32_t it = 0; it < n; it += D) {
#pragma unroll
        for (int k = 0; k < D; ++k) {
            if (it + (uint32_t)k >= n) break;
            compute_step<KIND, R>(f[k], s0 + it + (uint32_t)k, A, SX, q, acc);
            const uint32_t nx = it + D + (uint32_t)k;
            if (nx < n)
#pragma unroll
                for (int r = 0; r < R; ++r) fetch_one<KIND, R>(o[r], T, s0 + nx, lane, f[k], r);
        }
    }
}

// The block's 4 waves each hold partial row sums of R organs for tile rows
// lane % 16; returns, in thread t < 16, the totals of row t (sum over the
// waves, times 2^-E) in v[0..R-1].  part: 4 * R * 16 floats of LDS.
template <int R>
__device__ __forceinline__ void block_rows(const float* acc, float* part, int E, float* v) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = threadIdx.x >> 6;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float s = tile_row_sum(acc[r]);
        if (lane < 16) part[(wave * R + (uint32_t)r) * 16u + (uint32_t)lane] = s;
    }
    __syncthreads();
    if (threadIdx.x < 16) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float t = 0.0f;
            for (uint32_t w = 0; w < 4; ++w) t += part[(w * R + (uint32_t)r) * 16u + threadIdx.x];
            v[r] = ldexpf(t, -E);
        }
    }
}

// This wave's share [s0, s0 + n) of S steps split over the block's 4 waves.
__device__ __forceinline__ void wave_share(uint32_t S, uint32_t wave, uint32_t& s0, uint32_t& n) {
    const uint32_t per = (S + 3u) / 4u;
    s0 = min(wave * per, S);
    n = min(s0 + per, S) - s0;
}

// q8 rows of tile T of o[0..R-1] (cols H) against xn, in a block of its own:
// the weights' first D steps per wave (a wave's whole share at H = 2048;
// every route block runs one organ: router, shared gate, or one of the
// shared expert's gate and up projections) are in flight while xn is formed
// in registers (h and w issued before the weights) and each thread scatters
// its chunks of the q8 x image (E = 0: one exponent per 16-column unit, no
// block-wide maximum) into LDS.
template <int R, int D = 8 / R>
__device__ __forceinline__ void q8_tile(const M15Dims& d, const M15Dev& L, const float* h, const OrganView (&o)[R],
                                        uint32_t T, uint8_t* lds, float* red, float* part, uint32_t* status,
                                        float* v) {
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t S = n_steps_for(HK_Q8, d.H), nch = d.H / 8u;
    uint32_t s0, n;
    wave_share(S, wave, s0, n);
    XnRegs x;
    XnW wv;
    xn_load(h, L.norm_w, d.H, x, wv);
    Frag<HK_Q8, R> f[D];
    fetch_first<HK_Q8, R, D>(o, T, s0, n, lane, f);
    uint8_t* img = lds;
    float* sx = reinterpret_cast<float*>(img + (size_t)S * Kcfg<HK_Q8>::P * A_TILE_STRIDE);
    if (threadIdx.x < 64u) image_zero_blocks<HK_Q8>(threadIdx.x, img, S);
    xn_finish(d.H, d.eps, red, x, wv);
    bool bad = false;
#pragma unroll
    for (int k = 0; k < M15_NC; ++k) {
        const uint32_t ch = threadIdx.x + 256u * (uint32_t)k;
        if (ch < nch) bad |= image_chunk<HK_Q8>(ch, x.v[k], img, sx, 0u, 0u);
    }
    if (bad) atomicOr(status, HK_DEVERR_NONFINITE);
    __syncthreads();
    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    run_steps<HK_Q8, R, D>(o, T, s0, n, img, S, lane, f, acc);
    block_rows<R>(acc, part, 0, v);
}

__global__ void __launch_bounds__(256) m15_route_kernel(M15Dims d, M15Dev L, const float* __restrict__ h, M15Ws ws) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[8];
    __shared__ float part[4 * 2 * 16];
    // every descriptor field a role reads, in one round trip before the role branch
    arg_here(d.H);
    arg_here(d.E);
    arg_here(d.SI);
    arg_here(d.eps);
    arg_here(ws.logits);
    arg_here(ws.gate);
    arg_here(ws.act_s);
    arg_here(ws.xn);
    arg_here(ws.img);
    arg_here(ws.img_e);
    arg_here(ws.status);
    view_here(L.router);
    view_here(L.sgate);
    view_here(L.sg);
    view_here(L.su);
    arg_here(L.norm_w);
    arg_here(h);
    const uint32_t nR = L.router.n_tiles, nG = L.sgate.n_tiles, nS = nG ? L.sg.n_tiles : 0u;
    const uint32_t b = blockIdx.x;
    float v[2] = {0.0f, 0.0f};
    if (b < nR) {
        const OrganView o[1] = {L.router};
        q8_tile<1>(d, L, h, o, b, lds, red, part, ws.status, v);
        const uint32_t row = b * 16u + threadIdx.x;
        if (threadIdx.x < 16 && row < d.E) ws.logits[row] = v[0];
    } else if (b < nR + nG) {
        const OrganView o[1] = {L.sgate};
        q8_tile<1>(d, L, h, o, 0, lds, red, part, ws.status, v);
        if (threadIdx.x == 0) {
            // moe_suffix's shared-expert gate: sigmoid, finite and in [0, 1]
            const float g = 1.0f / (1.0f + expf(-v[0]));
            ws.gate[0] = v[0];
            ws.gate[1] = g;
            if (!(isfinite(g) && g >= 0.0f && g <= 1.0f)) atomicOr(ws.status, HK_DEVERR_NONFINITE);
        }
    } else if (b < nR + nG + 2u * nS) {
        // a 16-row tile of the shared expert's gate (the first nS blocks) or
        // up projection (the next nS), each block one organ's share
        const uint32_t k = b - nR - nG, which = k >= nS ? 1u : 0u, T = k - which * nS;
        const OrganView o[1] = {which ? L.su : L.sg};
        q8_tile<1>(d, L, h, o, T, lds, red, part, ws.status, v);
        const uint32_t row = T * 16u + threadIdx.x;
        if (threadIdx.x < 16 && row < d.SI) ws.act_s[which * d.SI + row] = v[0];
    } else {
        // the binary x image of xn (E = 0), one 512-column step per block,
        // scattered by the wave whose threads hold that step's 64 chunks;
        // the first block publishes xn
        const uint32_t tb = b - nR - nG - 2u * nS, S = n_steps_for(HK_BIN, d.H), nch = d.H / 8u;
        XnRegs x;
        block_xn(h, L.norm_w, d.H, d.eps, red, x);
        if (tb == 0) {
#pragma unroll
            for (int k = 0; k < M15_NC; ++k) {
                const uint32_t ch = threadIdx.x + 256u * (uint32_t)k;
                if (ch < nch) {
                    reinterpret_cast<float4*>(ws.xn)[2u * ch] = x.v[k][0];
                    reinterpret_cast<float4*>(ws.xn)[2u * ch + 1u] = x.v[k][1];
                }
            }
            if (threadIdx.x == 0) ws.img_e[0] = 0;
        }
        uint8_t* tiles = ws.img + (size_t)tb * Kcfg<HK_BIN>::P * A_TILE_STRIDE;
        float* sx = reinterpret_cast<float*>(ws.img + (size_t)S * Kcfg<HK_BIN>::P * A_TILE_STRIDE) +
                    (size_t)tb * (512u / Kcfg<HK_BIN>::SXG) * Kcfg<HK_BIN>::SXW;
        if ((threadIdx.x >> 6) == (tb & 3u)) {
            const uint32_t lane = threadIdx.x & 63u;
            image_zero_blocks<HK_BIN>(lane, tiles, 1u);
            bool bad = false;
#pragma unroll
            for (int k = 0; k < M15_NC; ++k)
                if ((uint32_t)k == (tb >> 2)) bad = image_chunk<HK_BIN>(64u * tb + lane, x.v[k], tiles, sx, 64u * tb, 8u * tb);
            if (__ballot(bad) != 0 && lane == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);
        }
    }
}

// Gate/up of one (16-row tile, slot).
template <int NPL>
__global__ void __launch_bounds__(256) m15_gate_up_kernel(M15Dims d, M15Dev L, M15Ws ws, int32_t* ids_out,
                                                          float* w_out) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ int32_t sel_id;
    __shared__ TopkLds tk;
    __shared__ float part[4 * 2 * 16];
    const uint32_t slot = blockIdx.y, T = blockIdx.x;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t S = n_steps_for(HK_BIN, d.H), ib = (uint32_t)x_lds_bytes<HK_BIN>(S);
    const uint32_t ib16 = (ib + 15u) & ~15u;
    // expert 0's views: every field but the pointers is every expert's
    const OrganView g0 = L.gate[0], u0 = L.up[0];
    const ResView r0v = L.res[0];
    M15Expert* ext = reinterpret_cast<M15Expert*>(lds + ib16 + (size_t)d.H * 4u + (size_t)RICE_BATCH * 4u);
    uint32_t* tsl = reinterpret_cast<uint32_t*>(ext + d.E);  // rows T and T + 1 of the tile-start table
    if (wave == 0) {
        const bool pub = T == 0 && slot == 0;
        const ArgBest mine = softmax_topk_wave<NPL>(ws.logits, d.E, d.K, 1, pub ? ws.ids : nullptr,
                                                    pub ? ws.w : nullptr, pub ? ws.status : nullptr, &tk,
                                                    lane, d.tie_eps);
        if (pub && (uint32_t)lane < d.K) {
            if (ids_out) ids_out[lane] = mine.i;
            if (w_out) w_out[lane] = mine.v;
        }
        if ((uint32_t)lane == slot) sel_id = mine.i;
    } else {
        // the binary image, xn (for the residual), the expert records and the
        // tile's two rows of record starts into LDS (at most two 16-byte
        // pieces per thread: tstride <= 512 <= 4 (blockDim.x - 64), as
        // n_experts <= 512 is checked at create)
        const uint32_t tt = threadIdx.x - 64u, nt = blockDim.x - 64u, nts = L.tstride / 2u;
        const uint4* tsrc = reinterpret_cast<const uint4*>(L.tstart + (size_t)T * L.tstride);
        uint4 tv[2];
#pragma unroll
        for (uint32_t i = 0; i < 2u; ++i) tv[i] = ldg(tsrc + min(tt + nt * i, nts - 1u));
        copy16x3_to_lds<12>(reinterpret_cast<uint4*>(lds), reinterpret_cast<const uint4*>(ws.img), ib / 16u,
                            reinterpret_cast<uint4*>(lds + ib16), reinterpret_cast<const uint4*>(ws.xn), d.H / 4u,
                            reinterpret_cast<uint4*>(ext), reinterpret_cast<const uint4*>(L.ex), 2u * d.E, tt, nt);
#pragma unroll
        for (uint32_t i = 0; i < 2u; ++i)
            if (tt + nt * i < nts) reinterpret_cast<uint4*>(tsl)[tt + nt * i] = tv[i];
    }
    __syncthreads();
    const int32_t id = sel_id;
    // an invalid route selects no organ (all-zero down views: n_tiles = 0)
    const bool ok = id >= 0 && (uint32_t)id < d.E;
    if (T == 0 && threadIdx.x < 2u * (sizeof(OrganView) / 8u)) {
        // word copies (a struct assignment here goes through scratch memory)
        static_assert(sizeof(OrganView) % 8 == 0, "OrganView is copied in 8-byte words");
        const uint32_t wpv = sizeof(OrganView) / 8u, which = threadIdx.x / wpv, word = threadIdx.x % wpv;
        const OrganView* tab = which == 0 ? L.dr : L.dl;
        const uint64_t* from = reinterpret_cast<const uint64_t*>(tab + (ok ? (uint32_t)id : 0u));
        reinterpret_cast<uint64_t*>(ws.sel + slot * 2u + which)[word] = ok ? from[word] : 0ull;
        if (!ok && threadIdx.x == 0) atomicOr(ws.status, HK_DEVERR_ROUTE);
    }
    if (!ok) return;
    if (T >= g0.n_tiles) return;
    const M15Expert ex = ext[id];
    OrganView o[2] = {g0, u0};
    o[0].data = ex.gate;
    o[0].scales = reinterpret_cast<const uint16_t*>(ex.gate + L.g_soff);
    o[1].data = ex.up;
    o[1].scales = reinterpret_cast<const uint16_t*>(ex.up + L.u_soff);
    uint32_t s0, n;
    wave_share(S, wave, s0, n);
    // the rows' residual pointers, the weights, then the first records: the
    // tile's record range comes from LDS, so no global load precedes them
    ResView rv = r0v;
    rv.row_ptr = ex.rptr;
    rv.recs = reinterpret_cast<const uint16_t*>(reinterpret_cast<const uint8_t*>(ex.rptr) + L.rec_off);
    rv.scale = ex.rscale;
    const uint32_t r0 = T * 16u, r1 = min(r0 + 16u, d.I);
    RiceTile rt;
    rice_ranges_known(rv, r0, r1, tsl[id], tsl[L.tstride + (uint32_t)id], rt);
    Frag<HK_BIN, 2> f[M15_D];
    fetch_first<HK_BIN, 2>(o, T, s0, n, lane, f);
    rice_first_records(rv, rt);
    const int E = ws.img_e[0];
    // the residual's first batch of products as soon as its records land
    // (xn has been in LDS since the barrier above, and the records were
    // issued right after this wave's weights, so the steps below find their
    // data there); block_rows' barrier then publishes them to the row sums
    float* xs = reinterpret_cast<float*>(lds + ib16);
    float* vals = xs + d.H;
    const uint32_t b0 = rt.e0 & ~7u;
    rice_products(rv, rt, b0, xs, vals);
    float acc[2] = {0.0f, 0.0f};
    run_steps<HK_BIN, 2>(o, T, s0, n, lds, S, lane, f, acc);
    float v[2] = {0.0f, 0.0f};
    block_rows<2>(acc, part, E, v);
    // the up's residual after its base, each row's outliers in index order
    // (the first batch here, any further batch of a long tile after it)
    float racc[2] = {threadIdx.x < 16 ? v[1] : 0.0f, 0.0f};
    rice_load_batch(rv, b0 + RICE_BATCH, rt.e1, rt.rv);
    rice_row_sums(rt, b0, vals, racc);
    rice_batches_from(rv, rt, b0 + RICE_BATCH, racc, xs, vals);
    const uint32_t row = r0 + threadIdx.x;
    if (threadIdx.x < 16 && row < d.I) ws.act[(size_t)slot * d.I + row] = (v[0] / (1.0f + expf(-v[0]))) * racc[0];
}

// The x image (E = 0) of x (cols columns, S steps) in LDS, scattered by the
// block's threads one 8-column chunk each (chunks past cols are zero); the
// block synchronises before returning.  Returns this thread's non-finite flag.
template <int KIND>
__device__ __forceinline__ bool scatter_image(const float* __restrict__ x, uint32_t cols, uint32_t S, uint8_t* img) {
    if (threadIdx.x < 64u) image_zero_blocks<KIND>(threadIdx.x, img, S);
    float* sx = reinterpret_cast<float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    const uint32_t nch = S * (uint32_t)Kcfg<KIND>::STEP_COLS / 8u;
    bool bad = false;
    // a unit's chunks are consecutive threads, active together (nch is whole units)
    for (uint32_t ch = threadIdx.x; ch < nch; ch += blockDim.x) {
        float4 v[2];
        load_chunk(x, 8u * ch, cols, v);
        bad |= image_chunk<KIND>(ch, v, img, sx, 0u, 0u);
    }
    __syncthreads();
    return bad;
}

// scatter_image of silu(g) * u (the shared expert's SwiGLU, formed from its
// two projections with the routed epilogue's expression).
template <int KIND>
__device__ __forceinline__ bool scatter_image_swiglu(const float* __restrict__ g, const float* __restrict__ u,
                                                     uint32_t cols, uint32_t S, uint8_t* img) {
    if (threadIdx.x < 64u) image_zero_blocks<KIND>(threadIdx.x, img, S);
    float* sx = reinterpret_cast<float*>(img + (size_t)S * Kcfg<KIND>::P * A_TILE_STRIDE);
    const uint32_t nch = S * (uint32_t)Kcfg<KIND>::STEP_COLS / 8u;
    bool bad = false;
    for (uint32_t ch = threadIdx.x; ch < nch; ch += blockDim.x) {
        float4 a[2], v[2];
        load_chunk(g, 8u * ch, cols, a);
        load_chunk(u, 8u * ch, cols, v);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            v[j] = make_float4((a[j].x / (1.0f + expf(-a[j].x))) * v[j].x, (a[j].y / (1.0f + expf(-a[j].y))) * v[j].y,
                               (a[j].z / (1.0f + expf(-a[j].z))) * v[j].z, (a[j].w / (1.0f + expf(-a[j].w))) * v[j].w);
        bad |= image_chunk<KIND>(ch, v, img, sx, 0u, 0u);
    }
    __syncthreads();
    return bad;
}

// Down right factors (mid_r = R_r act_r) and the shared expert's down.
__global__ void __launch_bounds__(256) m15_down_r_kernel(M15Dims d, M15Dev L, M15Ws ws) {
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float part[4 * 16];
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t nTr = n_tiles_for(d.rank), nR = d.K * nTr;
    bool bad = false;
    float v[1] = {0.0f};
    if (blockIdx.x < nR) {
        const uint32_t slot = blockIdx.x / nTr, T = blockIdx.x % nTr;
        const OrganView o[1] = {ws.sel[slot * 2u]};
        if (T >= o[0].n_tiles) return;
        const uint32_t S = o[0].steps;
        uint32_t s0, n;
        wave_share(S, wave, s0, n);
        Frag<HK_U3, 1> f[M15_D];
        fetch_first<HK_U3, 1>(o, T, s0, n, lane, f);
        bad = scatter_image<HK_U3>(ws.act + (size_t)slot * d.I, d.I, S, lds);
        float acc[1] = {0.0f};
        run_steps<HK_U3, 1>(o, T, s0, n, lds, S, lane, f, acc);
        block_rows<1>(acc, part, 0, v);
        const uint32_t row = T * 16u + threadIdx.x;
        if (threadIdx.x < 16 && row < d.rank) ws.mid[(size_t)slot * d.rank + row] = v[0];
    } else {
        const uint32_t T = blockIdx.x - nR;
        const OrganView o[1] = {L.sdown};
        const uint32_t S = o[0].steps;
        uint32_t s0, n;
        wave_share(S, wave, s0, n);
        Frag<HK_Q8, 1> f[M15_D];
        fetch_first<HK_Q8, 1>(o, T, s0, n, lane, f);
        bad = scatter_image_swiglu<HK_Q8>(ws.act_s, ws.act_s + d.SI, d.SI, S, lds);
        float acc[1] = {0.0f};
        run_steps<HK_Q8, 1>(o, T, s0, n, lds, S, lane, f, acc);
        block_rows<1>(acc, part, 0, v);
        const uint32_t row = T * 16u + threadIdx.x;
        if (threadIdx.x < 16 && row < d.H) ws.ys[row] = v[0];
    }
    if (bad && threadIdx.x == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);
}

// Down left factors and the combine; one wave per slot.
__global__ void __launch_bounds__(1024) m15_down_l_kernel(M15Dims d, const float* __restrict__ h,
                                                          float* __restrict__ out, M15Ws ws, uint32_t img_stride) {
    extern __shared__ __align__(16) uint8_t lds[];
    const uint32_t T = blockIdx.x, slots = d.K;
    const uint32_t slot = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    const OrganView o[1] = {ws.sel[slot * 2u + 1u]};
    // the combine's inputs (the slot's weight, and in the first 16 threads
    // the tile's residual rows, the shared expert's output and its gate)
    // are loaded now, unconditionally, in flight with everything else
    const uint32_t crow = min(T * 16u + (threadIdx.x & 15u), d.H - 1u);
    const float wslot = ws.w[slot], hres = h[crow], ysh = d.SI ? ws.ys[crow] : 0.0f, gsh = ws.gate[1];
    const bool active = T < o[0].n_tiles;
    const uint32_t S = active ? o[0].steps : 0u;
    Frag<HK_U3, 1> f[M15_D];
    fetch_first<HK_U3, 1>(o, T, 0u, S, lane, f);
    uint8_t* img = lds + (size_t)slot * img_stride;
    float* part = reinterpret_cast<float*>(lds + (size_t)slots * img_stride);
    if (active) {
        // the wave's x image of mid_r (E = 0), one 8-column chunk per lane and round
        const float* x = ws.mid + (size_t)slot * d.rank;
        image_zero_blocks<HK_U3>((uint32_t)lane, img, S);
        float* sx = reinterpret_cast<float*>(img + (size_t)S * Kcfg<HK_U3>::P * A_TILE_STRIDE);
        bool bad = false;
        for (uint32_t ch = (uint32_t)lane; ch < S * 16u; ch += 64u) {
            float4 v[2];
            load_chunk(x, 8u * ch, d.rank, v);
            bad |= image_chunk<HK_U3>(ch, v, img, sx, 0u, 0u);
        }
        if (__ballot(bad) != 0 && lane == 0) atomicOr(ws.status, HK_DEVERR_NONFINITE);
    }
    float acc[1] = {0.0f};
    run_steps<HK_U3, 1>(o, T, 0u, S, img, S, lane, f, acc);
    const float y = tile_row_sum(acc[0]);
    if (lane < 16) part[slot * 16u + (uint32_t)lane] = active ? y * wslot : 0.0f;
    __syncthreads();
    if (threadIdx.x < 16) {
        // combined = sum_r out_r * w_r in route order, += gate * shared; out = h + combined
        const uint32_t row = T * 16u + threadIdx.x;
        float comb = 0.0f;
        for (uint32_t r = 0; r < slots; ++r) comb += part[r * 16u + threadIdx.x];
        if (row < d.H) {
            if (d.SI) comb += ysh * gsh;
            const float v = hres + comb;
            out[row] = v;
            if (!isfinite(v)) atomicOr(ws.status, HK_DEVERR_NONFINITE);
        }
    }
}

// The tile-start table: ts[T * stride + e] = expert e's up residual
// row_ptr[min(16 T, I)] for T = 0..nt (zero for the padding entries e >= E).
__global__ void m15_tile_starts_kernel(const M15Expert* __restrict__ ex, uint32_t E, uint32_t I, uint32_t nt,
                                       uint32_t stride, uint32_t* __restrict__ ts) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    if (i >= (nt + 1u) * stride) return;
    const uint32_t T = i / stride, e = i % stride;
    ts[i] = e < E ? ex[e].rptr[min(16u * T, I)] : 0u;
}

}  // namespace hk

using namespace hk;

struct hk_moe15_layer {
    M15Dims d{};
    M15Dev dev{};
    M15Ws ws{};
    void* mem = nullptr;
    float* hbuf = nullptr;  // this layer's output inside a stack
    size_t lds_route = 0, lds_gu = 0, lds_dr = 0, lds_dl = 0;
    uint32_t dl_img_stride = 0, n_route_blocks = 0, n_dr_blocks = 0;
};

static inline size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }
static inline size_t align16(size_t n) { return (n + 15) & ~(size_t)15; }

static bool same_shape(const OrganView& a, const OrganView& b) {
    return a.kind == b.kind && a.rows == b.rows && a.cols == b.cols && a.group == b.group;
}

extern "C" int hk_moe15_layer_create(hk_ctx* ctx, const hk_moe15_layer_src* s, hk_moe15_layer** out) {
    if (!ctx || !out) return HK_E_INVALID_ARG;
    *out = nullptr;
    if (!s || !s->norm_w || !s->router || !s->gate || !s->up || !s->down_left || !s->down_right)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_layer_create: NULL argument");
    const uint32_t H = s->hidden, I = s->inter, SI = s->shared_inter, E = s->n_experts, K = s->top_k;
    if (!H || !I || !E || !K || K > E || K > M15_MAX_K || E > 512)
        return set_error(ctx, HK_E_UNSUPPORTED,
                         "mixed-1p5 layer: need 0 < top_k <= min(n_experts, 16), n_experts <= 512");
    if (!(s->route_tie_eps >= 0.0f) || !std::isfinite(s->route_tie_eps))
        return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: route_tie_eps must be finite and >= 0");
    if (!(s->eps >= 0.0f) || !std::isfinite(s->eps)) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: bad eps");
    const OrganView& rv = s->router->view;
    if (rv.rows != E || rv.cols != H || rv.kind != HK_Q8)
        return set_error(ctx, HK_E_GEOMETRY, "mixed-1p5 layer: router must be a q8 organ of n_experts x hidden");
    if (SI && (!s->shared_gate || !s->shared_gate_proj || !s->shared_up || !s->shared_down))
        return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: shared expert organs are NULL");
    if (SI && (s->shared_gate->view.kind != HK_Q8 || s->shared_gate->view.rows != 1 || s->shared_gate->view.cols != H ||
               s->shared_gate_proj->view.kind != HK_Q8 || s->shared_gate_proj->view.rows != SI ||
               s->shared_gate_proj->view.cols != H || !same_shape(s->shared_gate_proj->view, s->shared_up->view) ||
               s->shared_gate_proj->res_dev || s->shared_up->res_dev || s->shared_down->view.kind != HK_Q8 ||
               s->shared_down->view.rows != H || s->shared_down->view.cols != SI))
        return set_error(ctx, HK_E_GEOMETRY,
                         "mixed-1p5 layer: shared expert organs must be q8 of shapes 1 x hidden, shared_inter x "
                         "hidden (twice) and hidden x shared_inter");
    const hk_organ *g0 = s->gate[0], *u0 = s->up[0], *l0 = s->down_left[0], *r0 = s->down_right[0];
    if (!g0 || !u0 || !l0 || !r0) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: NULL expert organ");
    const uint32_t rank = r0->view.rows;
    if (g0->view.kind != HK_BIN || g0->view.rows != I || g0->view.cols != H || u0->kind != HK_BIN_RICE ||
        !same_shape(g0->view, u0->view) || l0->view.kind != HK_U3 || r0->view.kind != HK_U3 || l0->view.rows != H ||
        l0->view.cols != rank || r0->view.cols != I || H % 64 || H > 8192 || I % 4)
        return set_error(ctx, HK_E_GEOMETRY,
                         "mixed-1p5 layer: experts need a binary gate and an HGRAVR02 up of inter x hidden, and "
                         "3-bit down factors hidden x rank, rank x inter (hidden a multiple of 64, at most 8192)");
    std::vector<OrganView> gv(E), uv(E), lv(E), rvv(E);
    std::vector<ResView> res(E);
    for (uint32_t e = 0; e < E; ++e) {
        const hk_organ *g = s->gate[e], *u = s->up[e], *l = s->down_left[e], *r = s->down_right[e];
        if (!g || !u || !l || !r) return set_error(ctx, HK_E_INVALID_ARG, "mixed-1p5 layer: NULL expert organ");
        if (!same_shape(g->view, g0->view) || !same_shape(u->view, u0->view) || u->kind != HK_BIN_RICE ||
            !same_shape(l->view, l0->view) || !same_shape(r->view, r0->view) || g->res_dev)
            return set_error(ctx, HK_E_GEOMETRY, "mixed-1p5 layer: experts must share kinds and shapes");
        gv[e] = g->view;
        uv[e] = u->view;
        lv[e] = l->view;
        rvv[e] = r->view;
        res[e] = u->res;
    }
    // the compact gate/up records: scales and residual records must sit at
    // the same offsets from the data and the row pointers in every expert
    auto byte_off = [](const void* a, const void* b) {
        return (int64_t)(reinterpret_cast<uintptr_t>(a) - reinterpret_cast<uintptr_t>(b));
    };
    const int64_t g_soff = byte_off(gv[0].scales, gv[0].data), u_soff = byte_off(uv[0].scales, uv[0].data),
                  rec_off = byte_off(res[0].recs, res[0].row_ptr);
    std::vector<M15Expert> exv(E);
    for (uint32_t e = 0; e < E; ++e) {
        if (byte_off(gv[e].scales, gv[e].data) != g_soff || byte_off(uv[e].scales, uv[e].data) != u_soff ||
            byte_off(res[e].recs, res[e].row_ptr) != rec_off)
            return set_error(ctx, HK_E_UNSUPPORTED,
                             "mixed-1p5 layer: expert organs must come from the library's uploads (same layout)");
        exv[e] = M15Expert{gv[e].data, uv[e].data, res[e].row_ptr, res[e].scale, 0u};
    }
    if (g_soff < 0 || u_soff < 0 || rec_off < 0 || g_soff > 0xFFFFFFFF || u_soff > 0xFFFFFFFF || rec_off > 0xFFFFFFFF)
        return set_error(ctx, HK_E_UNSUPPORTED, "mixed-1p5 layer: unexpected organ layout");
    std::unique_ptr<hk_moe15_layer> L(new hk_moe15_layer());
    L->d = M15Dims{H, I, SI, E, K, rank, s->eps, s->route_tie_eps};
    // dynamic LDS of the four kernels (each within 64 KB)
    const uint32_t Sb = n_steps_for(HK_BIN, H), Sq = n_steps_for(HK_Q8, H), Sr = n_steps_for(HK_U3, I),
                   Sl = n_steps_for(HK_U3, rank), Ss = SI ? n_steps_for(HK_Q8, SI) : 0u;
    L->lds_route = x_lds_bytes<HK_Q8>(Sq);
    const uint32_t nti = n_tiles_for(I), tstride = (E + 3u) & ~3u;
    L->lds_gu = align16(x_lds_bytes<HK_BIN>(Sb)) + (size_t)H * 4u + (size_t)RICE_BATCH * 4u +
                (size_t)E * sizeof(M15Expert) + (size_t)2u * tstride * 4u;
    L->lds_dr = std::max(x_lds_bytes<HK_U3>(Sr), SI ? x_lds_bytes<HK_Q8>(Ss) : (size_t)0);
    L->dl_img_stride = (uint32_t)align16(x_lds_bytes<HK_U3>(Sl));
    L->lds_dl = (size_t)K * L->dl_img_stride + (size_t)K * 16u * 4u;
    if (std::max({L->lds_route, L->lds_gu, L->lds_dr, L->lds_dl}) > 64u * 1024u)
        return set_error(ctx, HK_E_UNSUPPORTED, "mixed-1p5 layer: shapes need more than 64 KB of LDS per workgroup");
    L->n_route_blocks = rv.n_tiles + (SI ? 1u + 2u * s->shared_gate_proj->view.n_tiles : 0u) + Sb;
    L->n_dr_blocks = K * n_tiles_for(rank) + (SI ? n_tiles_for(H) : 0u);
    // one allocation: tables and workspace (each section 256-B aligned)
    size_t off = 0;
    auto take = [&](size_t bytes) {
        const size_t o = off;
        off += align256(bytes);
        return o;
    };
    const size_t o_norm = take(H * 4), o_gate = take(E * sizeof(OrganView)), o_up = take(E * sizeof(OrganView)),
                 o_res = take(E * sizeof(ResView)), o_dr = take(E * sizeof(OrganView)),
                 o_dl = take(E * sizeof(OrganView)), o_ex = take(E * sizeof(M15Expert)),
                 o_ts = take((size_t)(nti + 1u) * tstride * 4u), o_logits = take(E * 4), o_glogit = take(16), o_xn = take(H * 4),
                 o_img = take(x_lds_bytes<HK_BIN>(Sb)), o_imge = take(4), o_act = take((size_t)K * I * 4),
                 o_acts = take(2 * SI * 4 + 16), o_mid = take((size_t)K * rank * 4), o_ys = take(H * 4),
                 o_ids = take(K * 4), o_w = take(K * 4), o_sel = take(2 * K * sizeof(OrganView)),
                 o_hbuf = take(H * 4);
    if (hipMalloc(&L->mem, off) != hipSuccess) return set_error(ctx, HK_E_NOMEM, "mixed-1p5 layer allocation failed");
    uint8_t* m = static_cast<uint8_t*>(L->mem);
    M15Dev& dv = L->dev;
    dv.norm_w = reinterpret_cast<const float*>(m + o_norm);
    dv.router = rv;
    if (SI) {
        dv.sgate = s->shared_gate->view;
        dv.sg = s->shared_gate_proj->view;
        dv.su = s->shared_up->view;
        dv.sdown = s->shared_down->view;
    }
    dv.gate = reinterpret_cast<const OrganView*>(m + o_gate);
    dv.up = reinterpret_cast<const OrganView*>(m + o_up);
    dv.res = reinterpret_cast<const ResView*>(m + o_res);
    dv.dr = reinterpret_cast<const OrganView*>(m + o_dr);
    dv.dl = reinterpret_cast<const OrganView*>(m + o_dl);
    dv.ex = reinterpret_cast<const M15Expert*>(m + o_ex);
    dv.tstart = reinterpret_cast<const uint32_t*>(m + o_ts);
    dv.tstride = tstride;
    dv.g_soff = (uint32_t)g_soff;
    dv.u_soff = (uint32_t)u_soff;
    dv.rec_off = (uint32_t)rec_off;
    M15Ws& w = L->ws;
    w.logits = reinterpret_cast<float*>(m + o_logits);
    w.gate = reinterpret_cast<float*>(m + o_glogit);
    w.xn = reinterpret_cast<float*>(m + o_xn);
    w.img = m + o_img;
    w.img_e = reinterpret_cast<int32_t*>(m + o_imge);
    w.act = reinterpret_cast<float*>(m + o_act);
    w.act_s = reinterpret_cast<float*>(m + o_acts);
    w.mid = reinterpret_cast<float*>(m + o_mid);
    w.ys = reinterpret_cast<float*>(m + o_ys);
    w.ids = reinterpret_cast<int32_t*>(m + o_ids);
    w.w = reinterpret_cast<float*>(m + o_w);
    w.sel = reinterpret_cast<OrganView*>(m + o_sel);
    w.status = ctx->dev_status;
    L->hbuf = reinterpret_cast<float*>(m + o_hbuf);
    auto up_copy = [&](const void* dst, const void* src, size_t bytes) {
        return check_hip(ctx, hipMemcpy(const_cast<void*>(dst), src, bytes, hipMemcpyDefault), "mixed-1p5 layer upload");
    };
    int rc = check_hip(ctx, hipMemset(L->mem, 0, off), "mixed-1p5 layer clear");
    if (!rc) rc = up_copy(dv.norm_w, s->norm_w, H * 4);
    if (!rc) rc = up_copy(dv.gate, gv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(dv.up, uv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(dv.res, res.data(), E * sizeof(ResView));
    if (!rc) rc = up_copy(dv.dr, rvv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(dv.dl, lv.data(), E * sizeof(OrganView));
    if (!rc) rc = up_copy(dv.ex, exv.data(), E * sizeof(M15Expert));
    if (!rc) {
        const uint32_t n = (nti + 1u) * tstride;
        hipLaunchKernelGGL(m15_tile_starts_kernel, dim3((n + 255u) / 256u), dim3(256), 0, 0, dv.ex, E, I, nti, tstride,
                           const_cast<uint32_t*>(dv.tstart));
        rc = check_hip(ctx, hipGetLastError(), "mixed-1p5 tile starts");
        if (!rc) rc = check_hip(ctx, hipDeviceSynchronize(), "mixed-1p5 tile starts");
    }
    if (rc) {
        (void)hipFree(L->mem);
        return rc;
    }
    *out = L.release();
    return HK_OK;
}

extern "C" int hk_moe15_layer_free(hk_ctx* ctx, hk_moe15_layer* L) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!L) return HK_OK;
    int rc = check_hip(ctx, hipFree(L->mem), "hipFree (mixed-1p5 layer)");
    delete L;
    return rc;
}

extern "C" int hk_moe15_decode_layer(hk_ctx* ctx, hk_moe15_layer* L, const float* h, float* out, int32_t* ids,
                                     float* weights, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!L || !h || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_decode_layer: NULL argument");
    if ((reinterpret_cast<uintptr_t>(h) & 15u) != 0)
        return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_decode_layer: h must be 16-byte aligned");
    hipStream_t s = static_cast<hipStream_t>(stream);
    const M15Dims& d = L->d;
    hipLaunchKernelGGL(m15_route_kernel, dim3(L->n_route_blocks), dim3(256), L->lds_route, s, d, L->dev, h, L->ws);
    const dim3 gg(n_tiles_for(d.I), d.K);
    if (d.E <= 64)
        hipLaunchKernelGGL((m15_gate_up_kernel<1>), gg, dim3(256), L->lds_gu, s, d, L->dev, L->ws, ids, weights);
    else if (d.E <= 256)
        hipLaunchKernelGGL((m15_gate_up_kernel<4>), gg, dim3(256), L->lds_gu, s, d, L->dev, L->ws, ids, weights);
    else
        hipLaunchKernelGGL((m15_gate_up_kernel<8>), gg, dim3(256), L->lds_gu, s, d, L->dev, L->ws, ids, weights);
    hipLaunchKernelGGL(m15_down_r_kernel, dim3(L->n_dr_blocks), dim3(256), L->lds_dr, s, d, L->dev, L->ws);
    hipLaunchKernelGGL(m15_down_l_kernel, dim3(n_tiles_for(d.H)), dim3(64u * d.K), L->lds_dl, s, d, h, out, L->ws,
                       L->dl_img_stride);
    return check_hip(ctx, hipGetLastError(), "mixed-1p5 layer launch");
}

extern "C" int hk_moe15_decode_stack(hk_ctx* ctx, hk_moe15_layer* const* layers, uint32_t n_layers, const float* h,
                                     float* out, int32_t* ids, float* weights, hk_stream stream) {
    if (!ctx) return HK_E_INVALID_ARG;
    if (!layers || !n_layers || !h || !out) return set_error(ctx, HK_E_INVALID_ARG, "hk_moe15_decode_stack: NULL argument");
    for (uint32_t l = 0; l < n_layers; ++l)
        if (!layers[l] || layers[l]->d.H != layers[0]->d.H || layers[l]->d.K != layers[0]->d.K)
            return set_error(ctx, HK_E_GEOMETRY, "hk_moe15_decode_stack: layers must share hidden and top_k");
    const uint32_t K = layers[0]->d.K;
    const float* cur = h;
    for (uint32_t l = 0; l < n_layers; ++l) {
        float* dst = l + 1 == n_layers ? out : layers[l]->hbuf;
        const int rc = hk_moe15_decode_layer(ctx, layers[l], cur, dst, ids ? ids + (size_t)l * K : nullptr,
                                             weights ? weights + (size_t)l * K : nullptr, stream);
        if (rc) return rc;
        cur = dst;
    }
    return HK_OK;
}
