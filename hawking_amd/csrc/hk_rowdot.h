// hk_rowdot.h -- per-lane partial row dot products and single-weight decode
// for every organ kind (device code shared by the GEMV and MoE kernels).
//
// A row is processed in 32-column chunks; lane `lane` of a wave (or of a
// segment of `width` lanes) takes chunks lane, lane+width, ...  The caller
// reduces the partial sums across the lanes.
#pragma once

#include "hk_internal.h"

namespace hk {

__device__ __forceinline__ float q4_chunk_dot(uint4 v, float s, const float* __restrict__ xc) {
    const float4* xv = reinterpret_cast<const float4*>(xc);
    const uint32_t w[4] = {v.x, v.y, v.z, v.w};
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float4 xa = xv[2 * q];
        const float4 xb = xv[2 * q + 1];
        const uint32_t u = w[q];
        const float xs[8] = {xa.x, xa.y, xa.z, xa.w, xb.x, xb.y, xb.z, xb.w};
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int nib = (int)((u >> (4 * k)) & 0xFu) - 8;
            acc += ((float)nib * s) * xs[k];
        }
    }
    return acc;
}

__device__ __forceinline__ float bin_chunk_dot(uint32_t bits, float s, const float* __restrict__ xc) {
    const float4* xv = reinterpret_cast<const float4*>(xc);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float4 xa = xv[q];
        const float xs[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float w = ((bits >> (4 * q + k)) & 1u) ? s : -s;
            acc += w * xs[k];
        }
    }
    return acc;
}

// 32 two-bit codes (LSB-first) with one scale.
__device__ __forceinline__ float q2_chunk_dot(uint2 codes, float s, const float* __restrict__ xc) {
    const float4* xv = reinterpret_cast<const float4*>(xc);
    float acc = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const uint32_t word = q < 4 ? codes.x : codes.y;
        const float4 xa = xv[q];
        const float xs[4] = {xa.x, xa.y, xa.z, xa.w};
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const uint32_t c = (word >> (2 * (4 * (q & 3) + k))) & 3u;
            acc += (((float)c - 1.5f) * s) * xs[k];
        }
    }
    return acc;
}

// Number of binary groups among flat groups [first, fg) of a mixed organ.
__device__ __forceinline__ uint32_t mixed_bin_before(const uint8_t* __restrict__ tags,
                                                     uint32_t first, uint32_t fg) {
    uint32_t n = 0;
    for (uint32_t g = first; g < fg; ++g) n += (tags[g >> 3] >> (g & 7u)) & 1u;
    return n;
}

template <int KIND>
__device__ __forceinline__ float row_dot_partial(const CanonView& o, uint32_t row,
                                                 const float* __restrict__ x, int lane,
                                                 int width = 64);

template <>
__device__ __forceinline__ float row_dot_partial<HK_Q4>(const CanonView& o, uint32_t row,
                                                        const float* __restrict__ x, int lane,
                                                        int width) {
    const uint32_t chunks = o.cols >> 5;
    const uint4* codes = reinterpret_cast<const uint4*>(o.codes + (size_t)row * (o.cols >> 1));
    const uint16_t* sc = o.scales + (size_t)row * (o.cols / (uint32_t)o.group);
    float acc = 0.f;
    for (uint32_t j = lane; j < chunks; j += width) {
        const float s = f16_bits_to_f32(sc[(j * 32u) / (uint32_t)o.group]);
        acc += q4_chunk_dot(codes[j], s, x + j * 32u);
    }
    return acc;
}

template <>
__device__ __forceinline__ float row_dot_partial<HK_BIN>(const CanonView& o, uint32_t row,
                                                         const float* __restrict__ x, int lane,
                                                         int width) {
    const uint32_t chunks = o.cols >> 5;
    const uint32_t* sg = reinterpret_cast<const uint32_t*>(o.codes + (size_t)row * (o.cols >> 3));
    const uint16_t* sc = o.scales + (size_t)row * (o.cols >> 7);
    float acc = 0.f;
    for (uint32_t j = lane; j < chunks; j += width) {
        const float s = f16_bits_to_f32(sc[j >> 2]);
        acc += bin_chunk_dot(sg[j], s, x + j * 32u);
    }
    return acc;
}

template <>
__device__ __forceinline__ float row_dot_partial<HK_MIXED>(const CanonView& o, uint32_t row,
                                                           const float* __restrict__ x, int lane,
                                                           int width) {
    const uint32_t chunks = o.cols >> 5;
    const uint32_t gpr = o.cols >> 7;
    const uint32_t first = row * gpr;
    float acc = 0.f;
    for (uint32_t j = lane; j < chunks; j += width) {
        const uint32_t g = j >> 2, sub = j & 3u, fg = first + g;
        const uint32_t nb = mixed_bin_before(o.tags, first, fg);
        if ((o.tags[fg >> 3] >> (fg & 7u)) & 1u) {
            const uint32_t idx = o.row_bin[row] + nb;
            const uint32_t bits = reinterpret_cast<const uint32_t*>(o.codes + (size_t)idx * 16u)[sub];
            acc += bin_chunk_dot(bits, f16_bits_to_f32(o.scales[idx]), x + j * 32u);
        } else {
            const uint32_t idx = o.row_q2[row] + (g - nb);
            const uint2 c = reinterpret_cast<const uint2*>(o.q2_codes + (size_t)idx * 32u)[sub];
            acc += q2_chunk_dot(c, f16_bits_to_f32(o.q2_scales[2u * idx + (sub >> 1)]), x + j * 32u);
        }
    }
    return acc;
}

template <>
__device__ __forceinline__ float row_dot_partial<HK_F32>(const CanonView& o, uint32_t row,
                                                         const float* __restrict__ x, int lane,
                                                         int width) {
    const uint32_t chunks = o.cols >> 2;
    const float4* w = reinterpret_cast<const float4*>(o.dense + (size_t)row * o.cols);
    const float4* xv = reinterpret_cast<const float4*>(x);
    float acc = 0.f;
    for (uint32_t j = lane; j < chunks; j += width) {
        const float4 a = w[j], b = xv[j];
        acc += a.x * b.x;
        acc += a.y * b.y;
        acc += a.z * b.z;
        acc += a.w * b.w;
    }
    return acc;
}

// Decoded weight (r, c), bit-exact with the reference decoders.
__device__ __forceinline__ float decode_weight(const CanonView& o, uint32_t r, uint32_t c) {
    const size_t e = (size_t)r * o.cols + c;
    switch (o.kind) {
    case HK_Q4: {
        const uint8_t b = o.codes[e >> 1];
        const int nib = (e & 1) ? (b >> 4) : (b & 0xF);
        return (float)(nib - 8) * f16_bits_to_f32(o.scales[e / (uint32_t)o.group]);
    }
    case HK_BIN: {
        const float s = f16_bits_to_f32(o.scales[e >> 7]);
        return ((o.codes[e >> 3] >> (e & 7)) & 1u) ? s : -s;
    }
    case HK_MIXED: {
        const uint32_t gpr = o.cols >> 7, first = r * gpr, g = c >> 7, fg = first + g;
        const uint32_t nb = mixed_bin_before(o.tags, first, fg), i = c & 127u;
        if ((o.tags[fg >> 3] >> (fg & 7u)) & 1u) {
            const uint32_t idx = o.row_bin[r] + nb;
            const float s = f16_bits_to_f32(o.scales[idx]);
            return ((o.codes[(size_t)idx * 16u + (i >> 3)] >> (i & 7u)) & 1u) ? s : -s;
        }
        const uint32_t idx = o.row_q2[r] + (g - nb);
        const uint32_t code = (o.q2_codes[(size_t)idx * 32u + (i >> 2)] >> (2u * (i & 3u))) & 3u;
        return ((float)code - 1.5f) * f16_bits_to_f32(o.q2_scales[2u * idx + (i >> 6)]);
    }
    default:
        return o.dense[e];
    }
}

}  // namespace hk
