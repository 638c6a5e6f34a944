// hk_gemv2.hip -- packed-organ GEMV on the int8 matrix cores of gfx950.
//
// Batch-1 GEMV is bandwidth bound, but decoding 1-bit or 4-bit weights to
// floats costs at least one VALU op per weight, more than the VALU can issue
// at HBM speed for binary weights (8 weights per byte).  So the decode is
// moved into v_mfma_i32_16x16x64_i8:
//
//   * x is converted once per workgroup to a fixed-point integer
//     X = rint(x * 2^E) (|X| < 2^23), and X * 2^k is split into four signed
//     base-256 "limbs".  The MFMA A operand (16 x 64) holds, in row
//     m = 4*slot + limb, the limbs of the columns that lane-group `slot` of
//     the B operand covers (zero elsewhere), so one MFMA yields per-group
//     partial sums for 4 column groups x 4 limbs at once, exactly (int32).
//   * The B operand (64 x 16, 16 weight rows) comes straight from the packed
//     bytes with one AND per 4 weights: a binary "bit plane" s is
//     bytes & (0x01 << s) = bit * 2^s, a Q4 nibble plane is bytes & 0x0F, a
//     Q2 field is bytes & (0x03 << 2u); the power of two is folded into the
//     A limbs (X * 2^(7-s) etc.), so no shift is needed.
//   * Per (row, group) the four int32 limbs are combined in f32, the zero
//     point is removed with the group's sum of X (binary: sum(2b-1)X =
//     2 sum bX - sum X; Q4: sum (n-8)X; Q2: sum (c-1.5)X), and the f16 group
//     scale is applied: y = 2^-E * sum_groups scale * (...).
// Weights arrive in the tiled layout (hk_tile.h): one step = one 1 KiB
// coalesced wave load, lane l holding row l%16, column slot l/16.  Numerics:
// the only roundings are X (2^-24 relative to max|x|), the f32 combine, and
// the f32 accumulation over groups; rel-L2 vs the serial f32 reference is
// ~1e-7.
#include "hk_internal.h"
#include "hk_tile.h"

namespace hk {

typedef int v4i __attribute__((ext_vector_type(4)));

__device__ __forceinline__ v4i mfma_i8(const v4i& a, const v4i& b, const v4i& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

template <int KIND>
struct Kcfg;
template <>
struct Kcfg<HK_BIN> {
    static constexpr int P = 8, SC = 4, STEP_COLS = 512;
};
template <>
struct Kcfg<HK_Q4> {
    static constexpr int P = 2, SC = 8, STEP_COLS = 128;
};
template <>
struct Kcfg<HK_MIXED> {
    static constexpr int P = 8, SC = 4, STEP_COLS = 512;
};

constexpr int MAXT = 8;  // tiles per wave

__device__ __forceinline__ float combine_limbs(const v4i& c) {
    return (float)c[0] + 256.0f * (float)c[1] + 65536.0f * (float)c[2] + 16777216.0f * (float)c[3];
}

// Balanced base-256 digit `limb` of Y as an int8 bit pattern.
__device__ __forceinline__ uint32_t limb_byte(int32_t y, int limb) {
    const uint32_t z = (uint32_t)y + 0x80808080u;
    return ((z >> (8 * limb)) & 0xFFu) ^ 0x80u;
}

// Value of A-operand byte i (0..15) for step t, MFMA mu, lane-group q.
template <int KIND>
__device__ __forceinline__ int32_t a_value(const int32_t* X, int t, int mu, int q, int i) {
    if constexpr (KIND == HK_BIN) {
        const int32_t x = X[t * 512 + q * 128 + 8 * i + mu];
        return mu < 7 ? (x << (7 - mu)) : -x;
    } else if constexpr (KIND == HK_Q4) {
        return X[t * 128 + q * 32 + 2 * i + mu];
    } else {
        const int h = mu >> 2, u = mu & 3, r = i >> 2, j = i & 3;
        const int a = r < 2 ? 2 * h + r : 2 * h + 2 + r;
        const int32_t x = X[t * 512 + q * 128 + (int)mixed_q2_col((uint32_t)a, (uint32_t)j, (uint32_t)u)];
        return x << (u < 3 ? 6 - 2 * u : 6);
    }
}

// All threads: A tiles of one K chunk into LDS, [tau][lane][16 B], zeros in
// the lanes whose row slot differs from their column slot.
template <int KIND>
__device__ void build_a_tiles(const int32_t* __restrict__ ldsX, uint32_t* __restrict__ ldsA) {
    constexpr int P = Kcfg<KIND>::P, SC = Kcfg<KIND>::SC;
    for (int d = threadIdx.x; d < SC * P * 256; d += blockDim.x) {
        const int dw = d & 3, lane = (d >> 2) & 63, tau = d >> 8;
        const int t = tau / P, mu = tau % P, slot = (lane & 15) >> 2, limb = lane & 3, q = lane >> 4;
        uint32_t word = 0;
        if (slot == q) {
#pragma unroll
            for (int jb = 0; jb < 4; ++jb)
                word |= limb_byte(a_value<KIND>(ldsX, t, mu, q, 4 * dw + jb), limb) << (8 * jb);
        }
        ldsA[d] = word;
    }
}

// One tile over the steps of one chunk: returns this lane's partial dot
// (row lane%16, column slot lane/16) in units of 2^-E.
template <int KIND>
__device__ __forceinline__ float tile_chunk(const OrganView& o, uint32_t T, uint32_t step0, int nsteps,
                                            const v4i* A, const float* sxa, const float* sxb, int lane) {
    constexpr int SC = Kcfg<KIND>::SC;
    float part = 0.0f;
    if constexpr (KIND == HK_BIN || KIND == HK_Q4) {
        const uint8_t* base = o.data + ((size_t)T * o.steps + step0) * 1024u + 16u * lane;
        const uint16_t* sp = o.scales + ((size_t)T * 64u + lane) * o.steps + step0;
        uint4 v[SC];
        float s[SC];
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t < nsteps) {
                v[t] = *reinterpret_cast<const uint4*>(base + (size_t)t * 1024u);
                s[t] = f16_bits_to_f32(sp[t]);
            }
        }
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t >= nsteps) break;
            v4i c = {0, 0, 0, 0};
            if constexpr (KIND == HK_BIN) {
#pragma unroll
                for (int p = 0; p < 8; ++p) {
                    const uint32_t m = 0x01010101u << p;
                    const v4i b = {(int)(v[t].x & m), (int)(v[t].y & m), (int)(v[t].z & m), (int)(v[t].w & m)};
                    c = mfma_i8(A[t * 8 + p], b, c);
                }
                part += s[t] * (combine_limbs(c) * (1.0f / 64.0f) - sxa[t]);
            } else {
                const uint32_t m = 0x0F0F0F0Fu;
                const v4i lo = {(int)(v[t].x & m), (int)(v[t].y & m), (int)(v[t].z & m), (int)(v[t].w & m)};
                const v4i hi = {(int)((v[t].x >> 4) & m), (int)((v[t].y >> 4) & m), (int)((v[t].z >> 4) & m),
                                (int)((v[t].w >> 4) & m)};
                c = mfma_i8(A[t * 2], lo, c);
                c = mfma_i8(A[t * 2 + 1], hi, c);
                part += s[t] * (combine_limbs(c) - 8.0f * sxa[t]);
            }
        }
    } else {
        uint32_t V[SC][8];
        float s0[SC], s1[SC];
        bool q2[SC];
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t < nsteps) {
                const uint4 h = o.hdr[(size_t)T * o.steps + step0 + t];
                const uint32_t below = __builtin_amdgcn_mbcnt_hi(h.y, __builtin_amdgcn_mbcnt_lo(h.x, 0u));
                const bool isq2 = ((lane < 32 ? (h.x >> lane) : (h.y >> (lane - 32))) & 1u) != 0;
                const uint8_t* p = o.data + h.z + 16u * ((uint32_t)lane + below);
                const uint4 va = *reinterpret_cast<const uint4*>(p);
                const uint4 vb = *reinterpret_cast<const uint4*>(p + (isq2 ? 16 : 0));
                const uint32_t sh = isq2 ? 0u : 1u;  // binary: odd columns are the signs >> 1
                V[t][0] = va.x;
                V[t][1] = va.y;
                V[t][2] = va.z;
                V[t][3] = va.w;
                V[t][4] = vb.x >> sh;
                V[t][5] = vb.y >> sh;
                V[t][6] = vb.z >> sh;
                V[t][7] = vb.w >> sh;
                const uint16_t* sp = o.scales + h.w + (uint32_t)lane + below;
                s0[t] = f16_bits_to_f32(sp[0]);
                s1[t] = isq2 ? f16_bits_to_f32(sp[1]) : s0[t];
                q2[t] = isq2;
            }
        }
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if (t >= nsteps) break;
            const uint32_t bm = q2[t] ? 0x03030303u : 0x01010101u;
            const float alpha = q2[t] ? (1.0f / 64.0f) : (2.0f / 64.0f);
            const float beta = q2[t] ? 1.5f : 1.0f;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                v4i c = {0, 0, 0, 0};
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                    v4i b;
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int a = r < 2 ? 2 * h + r : 2 * h + 2 + r;
                        b[r] = (int)(u < 3 ? (V[t][a] & (bm << (2 * u))) : ((V[t][a] >> 6) & bm));
                    }
                    c = mfma_i8(A[t * 8 + h * 4 + u], b, c);
                }
                const float sx = h ? sxb[t] : sxa[t];
                part += (h ? s1[t] : s0[t]) * (combine_limbs(c) * alpha - beta * sx);
            }
        }
    }
    return part;
}

template <int KIND>
__global__ void __launch_bounds__(256, 2)
gemv_tiled_kernel(const OrganView* __restrict__ organs, const float* __restrict__ xall, size_t x_stride,
                  float* __restrict__ yall, size_t y_stride, uint32_t tiles_per_wg, uint32_t* status) {
    constexpr int P = Kcfg<KIND>::P, SC = Kcfg<KIND>::SC, STEP_COLS = Kcfg<KIND>::STEP_COLS;
    constexpr int CHUNK = SC * STEP_COLS;
    __shared__ __align__(16) uint32_t ldsA[SC * P * 256];
    __shared__ __align__(16) int32_t ldsX[CHUNK];
    __shared__ float ldsSX[CHUNK / 32];
    __shared__ float red[4];

    const OrganView o = organs[blockIdx.y];
    const float* __restrict__ x = xall + (size_t)blockIdx.y * x_stride;
    float* __restrict__ y = yall + (size_t)blockIdx.y * y_stride;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t tile0 = blockIdx.x * tiles_per_wg;
    const int q = lane >> 4;

    // fixed-point exponent from max|x|
    float m = 0.0f;
    for (uint32_t c = threadIdx.x; c < o.cols; c += blockDim.x) m = fmaxf(m, fabsf(x[c]));
    m = wave_max(m);
    if (lane == 0) red[wave] = m;
    __syncthreads();
    m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    if (!isfinite(m)) {
        if (threadIdx.x == 0 && status) atomicOr(status, 1u);
        m = 0.0f;
    }
    int e2 = 0;
    if (m > 0.0f) (void)frexpf(m, &e2);
    const int E = m > 0.0f ? 23 - e2 : 0;

    float acc[MAXT];
#pragma unroll
    for (int j = 0; j < MAXT; ++j) acc[j] = 0.0f;
    const int tiles_here = (int)min(tiles_per_wg, o.n_tiles > tile0 ? o.n_tiles - tile0 : 0u);
    const int my_tiles = tiles_here > wave ? (tiles_here - wave + 3) / 4 : 0;
    const uint32_t n_chunks = (o.steps + SC - 1) / SC;

    for (uint32_t kc = 0; kc < n_chunks; ++kc) {
        __syncthreads();
        const uint32_t cb = kc * CHUNK;
        for (int c = threadIdx.x; c < CHUNK; c += blockDim.x) {
            const uint32_t gc = cb + (uint32_t)c;
            ldsX[c] = gc < o.cols ? __float2int_rn(ldexpf(x[gc], E)) : 0;
        }
        __syncthreads();
        for (int b = threadIdx.x; b < CHUNK / 32; b += blockDim.x) {
            int32_t s = 0;
#pragma unroll 8
            for (int k = 0; k < 32; ++k) s += ldsX[b * 32 + k];
            ldsSX[b] = (float)s;
        }
        build_a_tiles<KIND>(ldsX, ldsA);
        __syncthreads();
        v4i A[SC * P];
#pragma unroll
        for (int tau = 0; tau < SC * P; ++tau) A[tau] = *reinterpret_cast<const v4i*>(&ldsA[tau * 256 + lane * 4]);
        float sxa[SC], sxb[SC];
#pragma unroll
        for (int t = 0; t < SC; ++t) {
            if constexpr (KIND == HK_Q4) {
                sxa[t] = ldsSX[4 * t + q];
                sxb[t] = 0.0f;
            } else if constexpr (KIND == HK_BIN) {
                sxa[t] = (ldsSX[16 * t + 4 * q] + ldsSX[16 * t + 4 * q + 1]) +
                         (ldsSX[16 * t + 4 * q + 2] + ldsSX[16 * t + 4 * q + 3]);
                sxb[t] = 0.0f;
            } else {
                sxa[t] = ldsSX[16 * t + 4 * q] + ldsSX[16 * t + 4 * q + 1];
                sxb[t] = ldsSX[16 * t + 4 * q + 2] + ldsSX[16 * t + 4 * q + 3];
            }
        }
        const int nsteps = (int)min((uint32_t)SC, o.steps - kc * SC);
#pragma unroll
        for (int j = 0; j < MAXT; ++j) {
            if (j >= my_tiles) break;
            const uint32_t T = tile0 + (uint32_t)wave + 4u * (uint32_t)j;
            acc[j] += tile_chunk<KIND>(o, T, kc * SC, nsteps, A, sxa, sxb, lane);
        }
    }
#pragma unroll
    for (int j = 0; j < MAXT; ++j) {
        if (j >= my_tiles) break;
        float v = acc[j];
        v += __shfl_xor(v, 16, 64);
        v += __shfl_xor(v, 32, 64);
        const uint32_t row = (tile0 + (uint32_t)wave + 4u * (uint32_t)j) * 16u + (uint32_t)(lane & 15);
        if (lane < 16 && row < o.rows) y[row] = ldexpf(v, -E);
    }
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

static uint32_t pick_tiles_per_wg(uint32_t n_tiles, uint32_t n) {
    // enough workgroups to fill 256 CUs twice over, as few as possible
    // otherwise (each workgroup rebuilds the x limbs once)
    uint32_t tpw = 32;
    while (tpw > 1 && (uint64_t)n * ((n_tiles + tpw - 1) / tpw) < 1024) tpw >>= 1;
    return tpw;
}

hipError_t launch_gemv_tiled(const OrganView* organs_dev, uint32_t n, const OrganView& sh, const float* x,
                             size_t x_stride, float* y, size_t y_stride, hipStream_t s) {
    if (sh.kind == HK_F32) {
        hipLaunchKernelGGL(gemv_f32_kernel, dim3((sh.rows + 3) / 4, n), dim3(256), 0, s, organs_dev, x, x_stride,
                           y, y_stride);
        return hipGetLastError();
    }
    const uint32_t tpw = pick_tiles_per_wg(sh.n_tiles, n);
    const dim3 grid((sh.n_tiles + tpw - 1) / tpw, n);
    switch (sh.kind) {
    case HK_BIN:
        hipLaunchKernelGGL(gemv_tiled_kernel<HK_BIN>, grid, dim3(256), 0, s, organs_dev, x, x_stride, y, y_stride,
                           tpw, nullptr);
        break;
    case HK_Q4:
        hipLaunchKernelGGL(gemv_tiled_kernel<HK_Q4>, grid, dim3(256), 0, s, organs_dev, x, x_stride, y, y_stride,
                           tpw, nullptr);
        break;
    case HK_MIXED:
        hipLaunchKernelGGL(gemv_tiled_kernel<HK_MIXED>, grid, dim3(256), 0, s, organs_dev, x, x_stride, y,
                           y_stride, tpw, nullptr);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace hk
