// hk_gemv2.hip -- GEMV over sets of packed organs on the int8 matrix cores
// (engine in hk_mfma.h), plus the dense f32 GEMV used for the router.
//
// Grid: (workgroups per organ, organs).  A workgroup of 4 waves loads x once
// (ahead of its first weight loads), builds the x image in LDS, then each wave
// walks groups of R consecutive row tiles
// (16 rows each) of its slice of the organ; one LDS operand fetch feeds the R
// tiles' MFMAs and the next step's weight loads are in flight while the
// current step computes.
#include "hk_mfma.h"

namespace hk {

// The item sequence of one wave: groups k = 0..ng-1 of R tiles starting at
// g0 + k*gstride, each over steps 0..S-1.
struct WaveItems {
    uint32_t g0, gstride, t1, steps, n;
    __device__ void at(uint32_t it, uint32_t* T, int R, int* nvalid, uint32_t* t) const {
        const uint32_t k = it / steps, g = g0 + k * gstride;
        *t = it % steps;
        for (int r = 0; r < R; ++r) T[r] = g + (uint32_t)r;
        *nvalid = (int)min((uint32_t)R, t1 - g);
    }
};

// A pipeline slot's walk over a wave's items: D items ahead at a time
// without a division per item (D / steps and D % steps once), clamped at
// the last item (past the end a slot re-reads it).  g = the slot's tile
// group start, t = its step.
template <int D>
struct ItemStride {
    uint32_t dq, dr, glast, tlast;
    __device__ __forceinline__ void init(const WaveItems& W, uint32_t last) {
        dq = (uint32_t)D / W.steps;
        dr = (uint32_t)D % W.steps;
        glast = W.g0 + (last / W.steps) * W.gstride;
        tlast = last % W.steps;
    }
    // slot (g, t) from item nx - D to item nx (nx > last: the last item)
    __device__ __forceinline__ void next(const WaveItems& W, uint32_t nx, uint32_t last, uint32_t* T, int R,
                                         int* nvalid, uint32_t* t) const {
        uint32_t g = T[0], s = *t + dr;
        g += dq * W.gstride;
        if (s >= W.steps) {
            s -= W.steps;
            g += W.gstride;
        }
        g = nx > last ? glast : g;
        s = nx > last ? tlast : s;
        *t = s;
        for (int r = 0; r < R; ++r) T[r] = g + (uint32_t)r;
        *nvalid = (int)min((uint32_t)R, W.t1 - g);
    }
};

// Row totals of a finished group of R tiles into the workgroup's LDS row
// buffer (unscaled; tiles r >= nvalid alias T[0] and are skipped).
template <int R>
__device__ __forceinline__ void flush_group(float* acc, const uint32_t* T, int nvalid, uint32_t t0, int lane,
                                            float* ysh) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const float v = tile_row_sum(acc[r]);
        if (r < nvalid && lane < 16) ysh[(T[r] - t0) * 16u + (uint32_t)lane] = v;
        acc[r] = 0.0f;
    }
}

// Mixed step headers staged per workgroup: tiles x steps <= 32 x 24.
constexpr uint32_t GEMV_MAX_MIXED_TILES_PER_WG = 32;
constexpr int GEMV_HDR_PER_THREAD = 3;
constexpr uint32_t GEMV_MAX_MIXED_STEPS = GEMV_HDR_PER_THREAD * 256 / GEMV_MAX_MIXED_TILES_PER_WG;

// Tiles per workgroup of a launch: narrow 3-bit factors (<= 4 steps, e.g. the
// rank-160 left factor) take 128 tiles so the x image is built once per 128
// tiles; every other launch at most 32.
__host__ __device__ inline uint32_t gemv_max_tiles(int kind, uint32_t steps) {
    return kind == HK_U3 && steps <= 4 ? 128u : 32u;
}

// Dynamic LDS: x image, one quantization window (2048 columns), (mixed) the
// headers of the workgroup's tiles, then the workgroup's row outputs.
template <int KIND>
__host__ __device__ constexpr size_t gemv_hdr_offset(uint32_t steps) {
    return x_lds_bytes<KIND>(steps);
}

// The terminal head's extras (HEAD launches): x = RMSNorm(1+w)(h) is formed
// from the register chunks before the image is built (workgroup 0 also
// stores it), and the epilogue reduces the greedy key of the logits below
// n_valid into key[0] (one 64-bit atomic max per workgroup); a non-finite x
// sets the low word of key[1].
struct HeadArgs {
    const float* norm_w;
    float eps;
    float* xn;
    uint32_t n_valid;
    uint64_t* key;
};

// The greedy order of a logit: larger value first, then lower index; NaN
// never wins (key 0) and -0 ranks as +0.
__device__ __forceinline__ uint64_t greedy_key(float v, uint32_t i) {
    if (v != v) return 0ull;
    const uint32_t b = __float_as_uint(v == 0.0f ? 0.0f : v);
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return ((uint64_t)ord << 32) | (uint64_t)(~i);
}

// Block-wide sum (every thread gets it); red: one float per wave.
__device__ __forceinline__ float block_sum_f(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (uint32_t w = 0; w < (blockDim.x >> 6); ++w) t += red[w];
    __syncthreads();
    return t;
}

// xn = h * (1 / sqrt(mean(h^2) + eps)) * (1 + w) on this thread's register
// chunks of h (source_qwen80_residual_rms_norm,
// model/qwen80_complete_runtime.rs:6778-6797); every chunk of h must be in
// registers (cols <= 8 * 256 * NC), and gw holds the same chunks of w
// (loaded with h, before the first weight steps: vector loads retire in
// issue order, so a w load issued after them would hold the norm until the
// weights land).
template <int NC>
__device__ __forceinline__ void head_norm_chunks(XChunks<NC>& xc, const XChunks<NC>& gw, uint32_t cols,
                                                 const HeadArgs& ha, float* red) {
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NC; ++j)
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const float4 v = xc.v[j][k];
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
    const float sum = block_sum_f(ss, red);
    const float inv = 1.0f / sqrtf(sum / (float)cols + ha.eps);
#pragma unroll
    for (int j = 0; j < NC; ++j) {
        const uint32_t c0 = 8u * (threadIdx.x + 256u * (uint32_t)j);
        if (c0 < cols) {
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const float4 g = gw.v[j][k];
                float4& v = xc.v[j][k];
                v = make_float4(v.x * inv * (1.0f + g.x), v.y * inv * (1.0f + g.y), v.z * inv * (1.0f + g.z),
                                v.w * inv * (1.0f + g.w));
                if (blockIdx.x == 0) reinterpret_cast<float4*>(ha.xn + c0)[k] = v;
            }
        }
    }
}

// The HGRAVR02 residual added in the binary GEMV's epilogue (RES): views
// per organ, and the most 16-byte record pieces any workgroup's rows span.
struct ResArgs {
    const ResView* views;
    uint32_t pieces;
};
constexpr int GEMV_RES_NP = 12;  // record pieces per thread (pieces <= 12 * 256)

// Where the workgroup's row totals sit in LDS: after the x image (and the
// mixed headers), and with RES after the epilogue's residual table and
// records, which reuse the image's bytes.
template <int KIND, bool RES>
__host__ __device__ inline size_t gemv_ysh_offset(uint32_t steps, uint32_t tpw, uint32_t cols, uint32_t pieces) {
    size_t off = gemv_hdr_offset<KIND>(steps) + (KIND == HK_MIXED ? (size_t)tpw * steps * sizeof(uint4) : 0);
    if (RES) off = std::max(off, (rice_table3_bytes(cols) + (size_t)pieces * 16u + 15u) & ~(size_t)15);
    return off;
}

// D-deep software pipeline: D fetched steps are in flight while one is
// consumed; slot d of the rotating buffer holds item it+d.  The loop body is
// branch-free in memory operations (refetches are unconditional, past the end
// they re-read the last item; y goes out through LDS after the loop) so the
// compiler can wait for exactly the slot being consumed.
//
// RES (binary, at most 512 rows per workgroup): y = base + the HGRAVR02
// residual, to the bit what rice_apply does after the plain GEMV.  The row
// pointers load with the first weights; after the main loop the image's
// LDS takes the product table of three entries per column (from the x
// chunks still in registers) and the workgroup's byte-step record pieces
// (loaded in one round), and each row's thread steps through its records,
// adding its products to the row total in index order.
// Where a pipeline's fetches past its last item go: with the weights' loads
// non-temporal, a re-read of the last item (the refetches stay unconditional,
// a branch around them measured slower) would come from HBM again (6.5 %
// more read traffic on the headline stream); pointed at this small buffer,
// which every wave's refetches keep in the caches, they cost no HBM bytes.
// Nothing fetched from it is ever consumed.
__device__ __align__(256) uint8_t g_refetch_dummy[4096];

// fetch_step, or the same loads from g_refetch_dummy when past (uniform):
// tile 0, step 0 of a view whose sections start there (offsets below 4 KiB).
template <int KIND, int R, bool NT>
__device__ __forceinline__ void fetch_step_or_dummy(const OrganView& o, const uint32_t* T, int nvalid, uint32_t t,
                                                    int lane, Frag<KIND, R>& f, bool past) {
    OrganView op = o;
    op.data = past ? g_refetch_dummy : o.data;
    op.scales = past ? reinterpret_cast<const uint16_t*>(g_refetch_dummy) : o.scales;
    uint32_t Tz[R];
#pragma unroll
    for (int r = 0; r < R; ++r) Tz[r] = past ? 0u : T[r];
    fetch_step<KIND, R, NT>(op, Tz, nvalid, past ? 0u : t, lane, f);
}

template <int KIND, int R, int D, int NC, bool HEAD, bool RES = false>
__global__ void __launch_bounds__(256)
gemv_tiled_kernel(const OrganView* __restrict__ organs, uint32_t n_organs, const float* __restrict__ xall,
                  size_t x_stride, float* __restrict__ yall, size_t y_stride, uint32_t tiles_per_wg, uint32_t parts,
                  uint32_t* status, HeadArgs ha, ResArgs ra) {
    static_assert(!RES || (KIND == HK_BIN && NC == 1 && !HEAD), "the fused residual is for binary organs");
    extern __shared__ __align__(16) uint8_t lds[];
    __shared__ float red[4];
    __shared__ uint64_t kred[HEAD ? 4 : 1];
    uint32_t oi, part;
    organ_part(blockIdx.x, parts, n_organs, &oi, &part);
    const OrganView o = organs[oi];
    const float* __restrict__ x = xall + (size_t)oi * x_stride;
    float* __restrict__ y = yall + (size_t)oi * y_stride;
    const int lane = threadIdx.x & 63, q = lane >> 4;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t t0 = part * tiles_per_wg, t1 = min(t0 + tiles_per_wg, o.n_tiles);
    WaveItems W{t0 + wave * R, 4u * R, t1, o.steps, 0};
    W.n = W.g0 < t1 ? ((t1 - W.g0 + W.gstride - 1) / W.gstride) * o.steps : 0;
    const uint32_t last = W.n ? W.n - 1u : 0u;

    // x (and for HEAD the norm weight) first, then (mixed) this workgroup's
    // step headers, then the first D steps' weight loads, all before the
    // image build
    XChunks<NC> xc;
    load_x<NC>(BlockTeam{}, x, o.cols, xc);
    XChunks<HEAD ? NC : 1> gw;  // HEAD: the norm weight's chunks, with x
    if constexpr (HEAD) load_x<NC>(BlockTeam{}, ha.norm_w, o.cols, gw);
    const uint32_t nh = (t1 - t0) * o.steps;
    uint4 hreg[GEMV_HDR_PER_THREAD];
    uint4* hsh = reinterpret_cast<uint4*>(lds + gemv_hdr_offset<KIND>(o.steps));
    float* ysh = reinterpret_cast<float*>(lds + gemv_ysh_offset<KIND, RES>(o.steps, tiles_per_wg, o.cols, ra.pieces));
    if constexpr (KIND == HK_MIXED) {
#pragma unroll
        for (int k = 0; k < GEMV_HDR_PER_THREAD; ++k) {
            const uint32_t i = threadIdx.x + 256u * k;
            if (i < nh) hreg[k] = ldg(o.hdr + (size_t)t0 * o.steps + i);
        }
    }
    Frag<KIND, R> f[D];
    uint32_t T[D][R], ts[D];
    int nv[D];
    {
        // unconditional, so the x wait below counts exactly these loads; a
        // wave without items re-reads the workgroup's first tile
        const WaveItems P = W.n ? W : WaveItems{t0, 4u * R, t0 + 1u, o.steps, 1u};
#pragma unroll
        for (int d = 0; d < D; ++d) {
            P.at(min((uint32_t)d, last), T[d], R, &nv[d], &ts[d]);
            if constexpr (KIND == HK_MIXED) fetch_step<KIND, R, !HEAD>(o, T[d], nv[d], ts[d], lane, f[d]);
            else fetch_step_or_dummy<KIND, R, !HEAD>(o, T[d], nv[d], ts[d], lane, f[d], (uint32_t)d > last);
        }
    }
    if constexpr (KIND == HK_MIXED) {
#pragma unroll
        for (int k = 0; k < GEMV_HDR_PER_THREAD; ++k) {
            const uint32_t i = threadIdx.x + 256u * k;
            if (i < nh) hsh[i] = hreg[k];
        }
    }
    // RES: the residual's view and the row pointers of this workgroup's rows
    // (two rows a thread), issued after the first weights
    ResView rv{};
    uint32_t rp0 = 0, my0[2] = {0u, 0u}, my1[2] = {0u, 0u};
    if constexpr (RES) {
        rv = ra.views[oi];
        const uint32_t r0 = t0 * 16u, r1 = min(t1 * 16u, o.rows);
        rp0 = ldg(rv.row_ptr8 + r0) / 16u;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t row = min(r0 + threadIdx.x + 256u * (uint32_t)h, r1);
            my0[h] = ldg(rv.row_ptr8 + row);
            my1[h] = ldg(rv.row_ptr8 + min(row + 1u, r1));
        }
    }
    if constexpr (HEAD) head_norm_chunks<NC>(xc, gw, o.cols, ha, red);
    // the x image with E = 0: every thread scatters its own chunks (no
    // block-wide maximum, no gather pass); a unit's chunks are consecutive
    // threads, active together
    bool bad = false;
    {
        const uint32_t nch = o.steps * (uint32_t)Kcfg<KIND>::STEP_COLS / 8u;
        float* sxw = reinterpret_cast<float*>(lds + (size_t)o.steps * Kcfg<KIND>::P * A_TILE_STRIDE);
        if (threadIdx.x < 64u) image_zero_blocks<KIND>(threadIdx.x, lds, o.steps);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const uint32_t ch = threadIdx.x + 256u * (uint32_t)j;
            if (ch < nch) bad |= image_chunk<KIND>(ch, xc.v[j], lds, sxw, 0u, 0u);
        }
        for (uint32_t ch = threadIdx.x + 256u * NC; ch < nch; ch += 256u) {
            float4 v[2];
            load_chunk(x, 8u * ch, o.cols, v);
            bad |= image_chunk<KIND>(ch, v, lds, sxw, 0u, 0u);
        }
        __syncthreads();
    }
    const int E = 0;
    if (bad && status) atomicOr(status, 1u);
    if constexpr (HEAD)
        if (bad) atomicOr(reinterpret_cast<uint32_t*>(ha.key + 1), 1u);

    const ImageA A{lds, a_lane_offset(lane)};
    const float* SX = reinterpret_cast<const float*>(lds + (size_t)o.steps * Kcfg<KIND>::P * A_TILE_STRIDE);

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.0f;
    ItemStride<D> adv;
    adv.init(W, last);
    uint32_t it = 0;
    for (; it + D <= W.n; it += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            compute_step<KIND, R>(f[d], ts[d], A, SX, q, acc);
            if (ts[d] + 1 == o.steps) flush_group<R>(acc, T[d], nv[d], t0, lane, ysh);
            adv.next(W, it + D + d, last, T[d], R, &nv[d], &ts[d]);
            if constexpr (KIND == HK_MIXED) {
                // headers from LDS: the data loads wait for an LDS read, not
                // for every load in flight before them
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    const uint32_t Tr = r < nv[d] ? T[d][r] : T[d][0];
                    fetch_mixed<R>(o, hsh[(Tr - t0) * o.steps + ts[d]], lane, f[d], r);
                }
            } else {
                fetch_step_or_dummy<KIND, R, !HEAD>(o, T[d], nv[d], ts[d], lane, f[d], it + D + d > last);
            }
        }
    }
#pragma unroll
    for (int d = 0; d < D; ++d) {
        if (it + d >= W.n) break;
        compute_step<KIND, R>(f[d], ts[d], A, SX, q, acc);
        if (ts[d] + 1 == o.steps) flush_group<R>(acc, T[d], nv[d], t0, lane, ysh);
    }
    __syncthreads();
    const uint32_t nrows = (t1 > t0 ? t1 - t0 : 0u) * 16u;
    if constexpr (RES) {
        // the image is dead: its bytes take the residual's table and records
        const uint32_t np = (ra.pieces + 255u) / 256u;
        const uint4* recs = reinterpret_cast<const uint4*>(rv.recs8);
        const uint32_t plast = (rv.count8 + 15u) / 16u - 1u;
        uint4 rr[GEMV_RES_NP];
#pragma unroll
        for (int j = 0; j < GEMV_RES_NP; ++j)
            if ((uint32_t)j < np) rr[j] = ldg(recs + min(rp0 + threadIdx.x + 256u * (uint32_t)j, plast));
        float* T3 = reinterpret_cast<float*>(lds);
        {
            const uint32_t c0 = 8u * threadIdx.x;
            if (c0 < o.cols) {
                const float xv[8] = {xc.v[0][0].x, xc.v[0][0].y, xc.v[0][0].z, xc.v[0][0].w,
                                     xc.v[0][1].x, xc.v[0][1].y, xc.v[0][1].z, xc.v[0][1].w};
#pragma unroll
                for (int k = 0; k < 8; ++k) {
                    const float p = rv.scale * xv[k];
                    T3[3u * (c0 + (uint32_t)k)] = -p;
                    T3[3u * (c0 + (uint32_t)k) + 1u] = p;
                    T3[3u * (c0 + (uint32_t)k) + 2u] = -0.0f;
                }
            }
        }
        if (threadIdx.x < 8u) T3[3u * o.cols + threadIdx.x] = -0.0f;
        uint4* Rr = reinterpret_cast<uint4*>(lds + rice_table3_bytes(o.cols));
#pragma unroll
        for (int j = 0; j < GEMV_RES_NP; ++j)
            if ((uint32_t)j < np && threadIdx.x + 256u * (uint32_t)j < ra.pieces) Rr[threadIdx.x + 256u * j] = rr[j];
        __syncthreads();
        const uint32_t* R4 = reinterpret_cast<const uint32_t*>(Rr);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t i = threadIdx.x + 256u * (uint32_t)h, row = t0 * 16u + i;
            if (i < nrows && row < o.rows) {
                float acc = ldexpf(ysh[i], -E);
                uint32_t v = 0xFFFFFFFFu;  // -1: a row's first step lands on its first index
#pragma unroll 2
                for (uint32_t e = my0[h]; e < my1[h]; e += 4u) {
                    const uint32_t w = R4[(e - 16u * rp0) / 4u];
                    v += w & 0xFFu;
                    acc += T3[v];
                    v += (w >> 8) & 0xFFu;
                    acc += T3[v];
                    v += (w >> 16) & 0xFFu;
                    acc += T3[v];
                    v += w >> 24;
                    acc += T3[v];
                }
                y[row] = acc;
            }
        }
        return;
    }
    uint64_t best = 0;
    for (uint32_t i = threadIdx.x; i < nrows; i += blockDim.x) {
        const uint32_t row = t0 * 16u + i;
        if (row < o.rows) {
            const float v = ldexpf(ysh[i], -E);
            y[row] = v;
            if constexpr (HEAD)
                if (row < ha.n_valid) best = max(best, greedy_key(v, row));
        }
    }
    if constexpr (HEAD) {
        for (int off = 32; off; off >>= 1) best = max(best, (uint64_t)__shfl_xor((unsigned long long)best, off, 64));
        if ((threadIdx.x & 63) == 0) kred[threadIdx.x >> 6] = best;
        __syncthreads();
        if (threadIdx.x == 0) {
            best = max(max(kred[0], kred[1]), max(kred[2], kred[3]));
            if (best) atomicMax(reinterpret_cast<unsigned long long*>(ha.key), (unsigned long long)best);
        }
    }
}

// One wave's walk over the row tiles [t0, t1) of organ o in groups of R tiles
// (stride 4R over the block's four waves), every step of each, D steps in
// flight -- the main loop of gemv_tiled_kernel for the non-mixed kinds.
// start() issues the first D fetches (before the caller builds its x image);
// run() consumes the walk against an x image, leaving the unscaled row totals
// in ysh[(tile - t0) * 16 + row].
template <int KIND, int R, int D>
struct TileWalk {
    WaveItems W;
    uint32_t last;
    Frag<KIND, R> f[D];
    uint32_t T[D][R], ts[D];
    int nv[D];

    __device__ __forceinline__ void start(const OrganView& o, uint32_t t0, uint32_t t1, uint32_t wave, int lane) {
        W = WaveItems{t0 + wave * R, 4u * R, t1, o.steps, 0};
        W.n = W.g0 < t1 ? ((t1 - W.g0 + W.gstride - 1) / W.gstride) * o.steps : 0;
        last = W.n ? W.n - 1u : 0u;
        // a wave without items re-reads tile t0 (its results are never used)
        const WaveItems P = W.n ? W : WaveItems{t0, 4u * R, t0 + 1u, o.steps, 1u};
#pragma unroll
        for (int d = 0; d < D; ++d) {
            P.at(min((uint32_t)d, last), T[d], R, &nv[d], &ts[d]);
            fetch_step<KIND, R>(o, T[d], nv[d], ts[d], lane, f[d]);
        }
    }

    __device__ __forceinline__ void run(const OrganView& o, uint32_t t0, const uint8_t* img, int lane, float* ysh) {
        const ImageA A{img, a_lane_offset(lane)};
        const float* SX = reinterpret_cast<const float*>(img + (size_t)o.steps * Kcfg<KIND>::P * A_TILE_STRIDE);
        const int q = lane >> 4;
        float acc[R];
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r] = 0.0f;
        ItemStride<D> adv;
        adv.init(W, last);
        uint32_t it = 0;
        for (; it + D <= W.n; it += D) {
#pragma unroll
            for (int d = 0; d < D; ++d) {
                compute_step<KIND, R>(f[d], ts[d], A, SX, q, acc);
                if (ts[d] + 1 == o.steps) flush_group<R>(acc, T[d], nv[d], t0, lane, ysh);
                adv.next(W, it + D + d, last, T[d], R, &nv[d], &ts[d]);
                fetch_step<KIND, R>(o, T[d], nv[d], ts[d], lane, f[d]);
            }
        }
#pragma unroll
        for (int d = 0; d < D; ++d) {
            if (it + d >= W.n) break;
            compute_step<KIND, R>(f[d], ts[d], A, SX, q, acc);
            if (ts[d] + 1 == o.steps) flush_group<R>(acc, T[d], nv[d], t0, lane, ysh);
        }
    }
};

// LDS layout of the low-rank kernel: the right factor's x image, mid (16
// floats per right tile), the left factor's image, then the left rows.
struct LowrankLds {
    size_t img_r, win_r, mid, img_l, win_l, ysh, total;
};
__host__ __device__ inline LowrankLds lowrank_lds(const OrganView& l, const OrganView& r) {
    LowrankLds L{};
    L.img_r = 0;
    L.win_r = L.img_r + x_lds_bytes<HK_U3>(r.steps);
    L.mid = L.win_r;
    L.img_l = L.mid + ((size_t)r.n_tiles * 16u * 4u + 15u) / 16u * 16u;
    L.win_l = L.img_l + x_lds_bytes<HK_U3>(l.steps);
    L.ysh = L.win_l;
    L.total = L.ysh + (size_t)l.n_tiles * 16u * 4u;
    return L;
}

// (build-time overrides for launch-shape sweeps: tile groups and steps in
// flight of the right and the left factor's walks)
#ifndef HK_LR_RR
#define HK_LR_RR 1
#define HK_LR_RD 3
#define HK_LR_LR 2
#define HK_LR_LD 3
#endif

// HGRAVS01 pairs y_i = L_i (R_i x_i), one workgroup per pair: the right
// factor's rows (mid, kept in LDS) and then the left factor's, whose first
// weight steps are issued as soon as the right factor's walk ends (in flight
// while mid's x image is built).  Issued at the start instead, they hold
// their registers through the right walk: 74 VGPRs and 6 workgroups per CU
// against 56 and 8 (4,096 pairs then run in exactly two rounds; r160 pairs
// 164 against 161 us).  The arithmetic
// is that of two gemv_tiled_kernel launches (mid rounded to f32, then its own
// x image), so the result is the same bits.  mid_all (may be null) also
// receives mid.
#ifndef HK_LR_MINW
#define HK_LR_MINW 1
#endif
template <int NC>
__global__ void __launch_bounds__(256, HK_LR_MINW)
lowrank_kernel(const OrganView* __restrict__ lefts, const OrganView* __restrict__ rights, uint32_t n,
               const float* __restrict__ xall, size_t x_stride, float* __restrict__ mid_all, size_t mid_stride,
               float* __restrict__ yall, size_t y_stride, uint32_t* status) {
    extern __shared__ __align__(16) uint8_t lds[];
    uint32_t oi, part;
    organ_part(blockIdx.x, 1, n, &oi, &part);
    const OrganView rv = rights[oi], lv = lefts[oi];
    const float* __restrict__ x = xall + (size_t)oi * x_stride;
    float* __restrict__ y = yall + (size_t)oi * y_stride;
    const int lane = threadIdx.x & 63;
    const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const LowrankLds M = lowrank_lds(lv, rv);
    float* mid = reinterpret_cast<float*>(lds + M.mid);
    float* ysh = reinterpret_cast<float*>(lds + M.ysh);

    XChunks<NC> xc;
    load_x<NC>(BlockTeam{}, x, rv.cols, xc);
    TileWalk<HK_U3, HK_LR_RR, HK_LR_RD> wr;
    wr.start(rv, 0, rv.n_tiles, wave, lane);
    TileWalk<HK_U3, HK_LR_LR, HK_LR_LD> wl;
    // both x images with E = 0, scattered from each thread's chunks (the
    // two launches' images to the bit: the GEMV builds them the same way)
    bool bad = false;
    {
        uint8_t* img = lds + M.img_r;
        float* sx = reinterpret_cast<float*>(img + (size_t)rv.steps * Kcfg<HK_U3>::P * A_TILE_STRIDE);
        const uint32_t nch = rv.steps * (uint32_t)Kcfg<HK_U3>::STEP_COLS / 8u;
        if (threadIdx.x < 64u) image_zero_blocks<HK_U3>(threadIdx.x, img, rv.steps);
#pragma unroll
        for (int j = 0; j < NC; ++j) {
            const uint32_t ch = threadIdx.x + 256u * (uint32_t)j;
            if (ch < nch) bad |= image_chunk<HK_U3>(ch, xc.v[j], img, sx, 0u, 0u);
        }
        for (uint32_t ch = threadIdx.x + 256u * NC; ch < nch; ch += 256u) {
            float4 v[2];
            load_chunk(x, 8u * ch, rv.cols, v);
            bad |= image_chunk<HK_U3>(ch, v, img, sx, 0u, 0u);
        }
        __syncthreads();
    }
    wr.run(rv, 0, lds + M.img_r, lane, mid);
    wl.start(lv, 0, lv.n_tiles, wave, lane);
    __syncthreads();
    if (mid_all)
        for (uint32_t i = threadIdx.x; i < rv.rows; i += blockDim.x) mid_all[(size_t)oi * mid_stride + i] = mid[i];
    {
        uint8_t* img = lds + M.img_l;
        float* sx = reinterpret_cast<float*>(img + (size_t)lv.steps * Kcfg<HK_U3>::P * A_TILE_STRIDE);
        const uint32_t nch = lv.steps * (uint32_t)Kcfg<HK_U3>::STEP_COLS / 8u;
        if (threadIdx.x < 64u) image_zero_blocks<HK_U3>(threadIdx.x, img, lv.steps);
        for (uint32_t ch = threadIdx.x; ch < nch; ch += 256u) {
            float4 v[2];
            load_chunk(mid, 8u * ch, rv.rows, v);
            bad |= image_chunk<HK_U3>(ch, v, img, sx, 0u, 0u);
        }
        __syncthreads();
    }
    wl.run(lv, 0, lds + M.img_l, lane, ysh);
    __syncthreads();
    for (uint32_t i = threadIdx.x; i < lv.rows; i += blockDim.x) y[i] = ysh[i];
    if (bad && status) atomicOr(status, 1u);
}

bool lowrank_fusable(const OrganView& l, const OrganView& r) {
    return l.kind == HK_U3 && r.kind == HK_U3 && r.rows == l.cols && r.cols <= 8192u && r.rows <= 2048u &&
           lowrank_lds(l, r).total <= GEMV_LDS_LIMIT;
}

hipError_t launch_lowrank(const OrganView* lefts, const OrganView* rights, uint32_t n, const OrganView& l,
                          const OrganView& r, const float* x, size_t x_stride, float* mid, size_t mid_stride, float* y,
                          size_t y_stride, uint32_t* status, hipStream_t s) {
    if (!lowrank_fusable(l, r)) return hipErrorInvalidValue;
    const size_t lds = lowrank_lds(l, r).total;
    if (x_image_cols<HK_U3>(r.steps) <= 2048u)
        hipLaunchKernelGGL(lowrank_kernel<1>, dim3(n), dim3(256), lds, s, lefts, rights, n, x, x_stride, mid,
                           mid_stride, y, y_stride, status);
    else
        hipLaunchKernelGGL(lowrank_kernel<4>, dim3(n), dim3(256), lds, s, lefts, rights, n, x, x_stride, mid,
                           mid_stride, y, y_stride, status);
    return hipGetLastError();
}

// Dense f32 rows (router, shared-expert gate): one wave per row, float4 loads.
__global__ void __launch_bounds__(256) gemv_f32_kernel(const OrganView* __restrict__ organs,
                                                       const float* __restrict__ xall, size_t x_stride,
                                                       float* __restrict__ yall, size_t y_stride) {
    const OrganView o = organs[blockIdx.y];
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= o.rows) return;
    const float4* w = reinterpret_cast<const float4*>(o.dense + (size_t)row * o.cols);
    const float4* xv = reinterpret_cast<const float4*>(xall + (size_t)blockIdx.y * x_stride);
    float acc = 0.f;
    for (uint32_t j = lane; j < o.cols / 4; j += 64) {
        const float4 a = w[j], b = xv[j];
        acc += a.x * b.x + a.y * b.y + a.z * b.z + a.w * b.w;
    }
    acc = wave_sum(acc);
    if (lane == 0) yall[(size_t)blockIdx.y * y_stride + row] = acc;
}

size_t gemv_lds_bytes(int kind, uint32_t cols) {
    const uint32_t S = n_steps_for(kind, cols);
    const size_t ysh = (size_t)gemv_max_tiles(kind, S) * 16u * sizeof(float);
    if (kind == HK_Q4) return gemv_hdr_offset<HK_Q4>(S) + ysh;
    if (kind == HK_U3) return gemv_hdr_offset<HK_U3>(S) + ysh;
    if (kind == HK_BIN) return gemv_hdr_offset<HK_BIN>(S) + ysh;
    if (kind == HK_Q8) return gemv_hdr_offset<HK_Q8>(S) + ysh;
    if (S > GEMV_MAX_MIXED_STEPS) return SIZE_MAX;
    return gemv_hdr_offset<HK_MIXED>(S) + (size_t)GEMV_MAX_MIXED_TILES_PER_WG * S * sizeof(uint4) + ysh;
}

template <int KIND, int R, int D, bool HEAD = false, bool RES = false>
static hipError_t launch_kind(const OrganView* organs, uint32_t n, const OrganView& sh, const float* x,
                              size_t xs, float* y, size_t ys, uint32_t tpw, hipStream_t s, const HeadArgs& ha = {},
                              uint32_t* status = nullptr, const ResArgs& ra = {}) {
    const uint32_t parts = (sh.n_tiles + tpw - 1) / tpw;
    const dim3 grid(parts * n);
    // image + one quantization window (2048 columns); x chunks held in
    // registers: one per thread up to 2048 columns, else four
    const uint32_t kc = x_image_cols<KIND>(sh.steps);
    const size_t lds = gemv_ysh_offset<KIND, RES>(sh.steps, tpw, sh.cols, ra.pieces) + (size_t)tpw * 16u * sizeof(float);
    if (kc <= 2048u)
        hipLaunchKernelGGL((gemv_tiled_kernel<KIND, R, D, 1, HEAD, RES>), grid, dim3(256), lds, s, organs, n, x, xs, y,
                           ys, tpw, parts, status, ha, ra);
    else if constexpr (!RES)
        hipLaunchKernelGGL((gemv_tiled_kernel<KIND, R, D, 4, HEAD>), grid, dim3(256), lds, s, organs, n, x, xs, y, ys,
                           tpw, parts, status, ha, ra);
    return hipGetLastError();
}

// Launch shape (R tiles per wave group, D steps in flight, tiles per
// workgroup) by kind and size, from sweeps over the streamed workloads:
// binary 2-tile groups 5 deep, over 16 tiles when the organ has >= 4 steps
// (also with the fused residual), else over 32; Q4 and Q8 2 over 32, 3 deep;
// 3-bit factors 2 over 16, or over 128 when narrow; mixed (large fragments)
// 1 over 16 (1 over 32 and 1 over 64 measured 1.3 % slower on 6,144 organs of
// 512 x 2048).  With the weights' non-temporal loads (fetch_one) the wide
// binary shape moved from 4-tile groups 3 deep (0.73 of 8 TB/s with the hint,
// 0.756 without) to 2-tile groups 5 deep (0.78-0.80; 4 deep 0.70, 6 deep
// 0.71, 4-tile groups 4 deep 0.56), and the fused residual's with it (0.69
// -> 0.73).
// (build-time overrides for launch-shape sweeps)
#ifndef HK_BIN_NARROW_R
#define HK_BIN_NARROW_R 2
#define HK_BIN_NARROW_D 5
#define HK_BIN_NARROW_TPW 32
#endif
#ifndef HK_BIN_WIDE_R
#define HK_BIN_WIDE_R 2
#define HK_BIN_WIDE_D 5
#endif
#ifndef HK_Q_R
#define HK_Q_R 2
#define HK_Q_D 3
#endif
#ifndef HK_RES_R
#define HK_RES_R 2
#define HK_RES_D 5
#endif
#ifndef HK_BIN_WIDE_TPW
#define HK_BIN_WIDE_TPW 16
#endif
#ifndef HK_Q_TPW
#define HK_Q_TPW 32
#endif
#ifndef HK_HEAD_R
#define HK_HEAD_R 2
#define HK_HEAD_D 3
#define HK_HEAD_TPW 5
#endif
#ifndef HK_MIX_R
#define HK_MIX_R 1
#define HK_MIX_D 3
#define HK_MIX_TPW 16
#endif
template <int KIND>
static hipError_t launch_r(const OrganView* organs, uint32_t n, const OrganView& sh, const float* x, size_t xs,
                           float* y, size_t ys, hipStream_t s) {
    const uint64_t tiles = (uint64_t)n * sh.n_tiles;
    if (tiles >= 16384) {
        if constexpr (KIND == HK_BIN) {
            if (sh.steps >= 4)
                return launch_kind<KIND, HK_BIN_WIDE_R, HK_BIN_WIDE_D>(organs, n, sh, x, xs, y, ys, HK_BIN_WIDE_TPW, s);
            return launch_kind<KIND, HK_BIN_NARROW_R, HK_BIN_NARROW_D>(organs, n, sh, x, xs, y, ys, HK_BIN_NARROW_TPW, s);
        } else if constexpr (KIND == HK_U3) {
            return launch_kind<KIND, 2, 3>(organs, n, sh, x, xs, y, ys, gemv_max_tiles(KIND, sh.steps) == 128u ? 128 : 16, s);
        } else if constexpr (KIND == HK_Q4 || KIND == HK_Q8) {
            return launch_kind<KIND, HK_Q_R, HK_Q_D>(organs, n, sh, x, xs, y, ys, HK_Q_TPW, s);
        } else {
            return launch_kind<KIND, HK_MIX_R, HK_MIX_D>(organs, n, sh, x, xs, y, ys, HK_MIX_TPW, s);
        }
    }
    if (tiles >= 4096) return launch_kind<KIND, 2, 2>(organs, n, sh, x, xs, y, ys, 8, s);
    const uint32_t tpw = (uint64_t)n * ((sh.n_tiles + 3) / 4) >= 256 ? 4 : 1;
    return launch_kind<KIND, 1, 2>(organs, n, sh, x, xs, y, ys, tpw, s);
}

// The terminal head on a q8 lm_head (cols <= 8192): one GEMV launch with the
// norm prologue and the greedy-key epilogue, then the one-thread pick (which
// also clears the key for the next call).  Launch shapes as for one q8 organ,
// except 4,096-16,383 tiles (a 65k-262k vocabulary), where 2-tile groups, 3
// steps in flight, over 5 tiles per workgroup measured fastest (151,936 x
// 2048: 1,900 workgroups, under the 2,048 resident at once; 56.5 us against
// 57.6 for 6 tiles, 59.3 for 8, 64.0 for 4).
__global__ void head_pick_fused_kernel(uint64_t* __restrict__ key, int32_t* __restrict__ token, uint32_t* status) {
    if (threadIdx.x == 0) {
        const uint64_t best = key[0];
        const uint32_t flag = reinterpret_cast<const uint32_t*>(key + 1)[0];
        const uint32_t ord = (uint32_t)(best >> 32);
        const float v = __uint_as_float((ord & 0x80000000u) ? (ord & 0x7FFFFFFFu) : ~ord);
        const bool ok = best != 0ull && isfinite(v) && flag == 0u;
        token[0] = ok ? (int32_t)(~(uint32_t)best) : -1;
        if (!ok) atomicOr(status, 1u);
        key[0] = 0ull;
        key[1] = 0ull;
    }
}

bool head_gemv_fusable(const OrganView& sh) { return sh.kind == HK_Q8 && x_image_cols<HK_Q8>(sh.steps) <= 8192u; }

hipError_t launch_head_fused(const OrganView* organ_dev, const OrganView& sh, const float* h, const float* norm_w,
                             float eps, float* xn, float* logits, uint32_t n_valid, uint64_t* key, int32_t* token,
                             uint32_t* status, hipStream_t s) {
    if (!head_gemv_fusable(sh)) return hipErrorInvalidValue;
    const HeadArgs ha{norm_w, eps, xn, n_valid, key};
    hipError_t e;
    if (sh.n_tiles >= 16384u)
        e = launch_kind<HK_Q8, 2, 3, true>(organ_dev, 1, sh, h, 0, logits, 0, 16, s, ha, status);
    else if (sh.n_tiles >= 4096u)
        e = launch_kind<HK_Q8, HK_HEAD_R, HK_HEAD_D, true>(organ_dev, 1, sh, h, 0, logits, 0, HK_HEAD_TPW, s, ha, status);
    else
        e = launch_kind<HK_Q8, 1, 2, true>(organ_dev, 1, sh, h, 0, logits, 0, (sh.n_tiles + 3) / 4 >= 256 ? 4 : 1, s,
                                          ha, status);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(head_pick_fused_kernel, dim3(1), dim3(64), 0, s, key, token, status);
    return hipGetLastError();
}

hipError_t launch_gemv_rice(const OrganView* organs_dev, const ResView* res_dev, uint32_t n, const OrganView& sh,
                            uint32_t pieces256, uint32_t pieces512, const float* x, size_t x_stride, float* y,
                            size_t y_stride, hipStream_t s, bool* fused) {
    *fused = false;
    // the streamed binary shapes (launch_r), with x in one register chunk
    if (sh.kind != HK_BIN || (uint64_t)n * sh.n_tiles < 16384 || x_image_cols<HK_BIN>(sh.steps) > 2048u)
        return hipSuccess;
    const bool wide = sh.steps >= 4;
    const uint32_t tpw = wide ? HK_BIN_WIDE_TPW : HK_BIN_NARROW_TPW, pieces = wide ? pieces256 : pieces512;
    static_assert(HK_BIN_WIDE_TPW * 16 == 256 && HK_BIN_NARROW_TPW * 16 == 512, "RES rows per workgroup");
    // the fused kernel runs 4 workgroups per CU (its registers): LDS up to a
    // quarter of the CU's 160 KiB costs no occupancy
    if (pieces == 0 || pieces > 256u * GEMV_RES_NP ||
        gemv_ysh_offset<HK_BIN, true>(sh.steps, tpw, sh.cols, pieces) + (size_t)tpw * 64u > 40u * 1024u)
        return hipSuccess;
    const ResArgs ra{res_dev, pieces};
    *fused = true;
    if (wide)
        return launch_kind<HK_BIN, HK_RES_R, HK_RES_D, false, true>(organs_dev, n, sh, x, x_stride, y, y_stride, tpw, s, {},
                                                                   nullptr, ra);
    return launch_kind<HK_BIN, HK_BIN_NARROW_R, HK_BIN_NARROW_D, false, true>(organs_dev, n, sh, x, x_stride, y,
                                                                              y_stride, tpw, s, {}, nullptr, ra);
}

hipError_t launch_gemv_tiled(const OrganView* organs_dev, uint32_t n, const OrganView& sh, const float* x,
                             size_t x_stride, float* y, size_t y_stride, hipStream_t s) {
    switch (sh.kind) {
    case HK_F32:
        hipLaunchKernelGGL(gemv_f32_kernel, dim3((sh.rows + 3) / 4, n), dim3(256), 0, s, organs_dev, x, x_stride,
                           y, y_stride);
        return hipGetLastError();
    case HK_BIN: return launch_r<HK_BIN>(organs_dev, n, sh, x, x_stride, y, y_stride, s);
    case HK_Q4: return launch_r<HK_Q4>(organs_dev, n, sh, x, x_stride, y, y_stride, s);
    case HK_MIXED: return launch_r<HK_MIXED>(organs_dev, n, sh, x, x_stride, y, y_stride, s);
    case HK_Q8: return launch_r<HK_Q8>(organs_dev, n, sh, x, x_stride, y, y_stride, s);
    case HK_U3: return launch_r<HK_U3>(organs_dev, n, sh, x, x_stride, y, y_stride, s);
    default: return hipErrorInvalidValue;
    }
}

}  // namespace hk
