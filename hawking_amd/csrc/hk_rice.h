// hk_rice.h -- the per-token HGRAVR02 residual step (device).
#pragma once

#include "hk_internal.h"

namespace hk {

constexpr uint32_t RICE_VEC = 2;                      // 8-record loads per thread per batch
constexpr uint32_t RICE_BATCH = 256u * 8u * RICE_VEC; // records staged per batch (floats of LDS)

// acc[h] (row r0 + threadIdx.x + 256 h, h = 0, 1) += the row's outliers, in
// index order, of (+-scale) * x[col].  Rows [r0, r1), r1 - r0 <= 512; every
// thread of the 256-thread workgroup calls this (it synchronises).  LDS: xs
// (cols floats) takes a copy of x, vals (RICE_BATCH floats) the products.
// Each batch is one round of 16-byte record loads (8 records each, issued
// with the x copy for the first batch); the products are formed from the LDS
// copy of x, and each row's thread adds the products of its own records in
// order -- the reference's serial order (binary_rice_q1_matvec_f32,
// q80_mixed_decode.rs:509-527), with the product rounded before the add as
// there.  The records array must be readable in whole 16-byte pieces.
__device__ __forceinline__ void rice_rows(const ResView& v, const float* __restrict__ x, uint32_t r0, uint32_t r1,
                                          float* acc, float* xs, float* vals) {
    const uint32_t tid = threadIdx.x;
    const uint32_t e0 = ldg(v.row_ptr + r0), e1 = ldg(v.row_ptr + r1);
    uint32_t my0[2], my1[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = r0 + tid + 256u * (uint32_t)h;
        my0[h] = my1[h] = 0;
        if (row < r1) {
            my0[h] = ldg(v.row_ptr + row);
            my1[h] = ldg(v.row_ptr + row + 1);
        }
    }
    const uint4* recs = reinterpret_cast<const uint4*>(v.recs);
    uint4 rv[RICE_VEC];
    auto load_batch = [&](uint32_t base) {
#pragma unroll
        for (uint32_t j = 0; j < RICE_VEC; ++j) {
            const uint32_t e = base + 8u * (tid + 256u * j);
            rv[j] = e < e1 ? ldg(recs + e / 8u) : make_uint4(0, 0, 0, 0);
        }
    };
    // the first batch's records are in flight with the copy of x; each later
    // batch's loads are issued before the previous batch's row sums
    load_batch(e0 & ~7u);
    copy16_to_lds<4>(reinterpret_cast<uint4*>(xs), reinterpret_cast<const uint4*>(x), v.cols / 4u, tid, 256u);
    for (uint32_t base = e0 & ~7u; base < e1; base += RICE_BATCH) {
        __syncthreads();  // xs (first batch) and the previous batch's readers
#pragma unroll
        for (uint32_t j = 0; j < RICE_VEC; ++j) {
            const uint32_t e = base + 8u * (tid + 256u * j);
            const uint32_t w[4] = {rv[j].x, rv[j].y, rv[j].z, rv[j].w};
            float p[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t rec = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu;
                const bool in = e + (uint32_t)k >= e0 && e + (uint32_t)k < e1;
                const float xv = xs[in ? (rec & 0x7FFFu) : 0u];
                p[k] = in ? ((rec >> 15) ? v.scale : -v.scale) * xv : 0.0f;
            }
            float4* o = reinterpret_cast<float4*>(vals + 8u * (tid + 256u * j));
            o[0] = make_float4(p[0], p[1], p[2], p[3]);
            o[1] = make_float4(p[4], p[5], p[6], p[7]);
        }
        load_batch(base + RICE_BATCH);
        __syncthreads();
#pragma unroll
        for (int h = 0; h < 2; ++h) {
            const uint32_t lo = max(my0[h], base), hi = min(my1[h], base + RICE_BATCH);
            uint32_t e = lo;
            for (; e + 8 <= hi; e += 8) {  // eight reads in flight, adds in order
                float t[8];
#pragma unroll
                for (int k = 0; k < 8; ++k) t[k] = vals[e - base + (uint32_t)k];
#pragma unroll
                for (int k = 0; k < 8; ++k) acc[h] += t[k];
            }
            for (; e < hi; ++e) acc[h] += vals[e - base];
        }
    }
}

}  // namespace hk
