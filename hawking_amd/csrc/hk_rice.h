// hk_rice.h -- the per-token HGRAVR02 residual step (device).
#pragma once

#include "hk_internal.h"

namespace hk {

constexpr uint32_t RICE_VEC = 2;                      // 8-record loads per thread per batch
constexpr uint32_t RICE_BATCH = 256u * 8u * RICE_VEC; // records staged per batch (floats of LDS)

// The loads rice_rows starts with: the rows' record ranges and the first
// batch of records (one round of 16-byte loads, 8 records each).
struct RiceTile {
    uint32_t e0, e1, my0[2], my1[2];
    uint4 rv[RICE_VEC];
};

__device__ __forceinline__ void rice_load_batch(const ResView& v, uint32_t base, uint32_t e1, uint4* rv) {
    const uint4* recs = reinterpret_cast<const uint4*>(v.recs);
#pragma unroll
    for (uint32_t j = 0; j < RICE_VEC; ++j) {
        const uint32_t e = base + 8u * (threadIdx.x + 256u * j);
        rv[j] = e < e1 ? ldg(recs + e / 8u) : make_uint4(0, 0, 0, 0);
    }
}

// rice_prefetch in two parts, so that loads issued between them (weights)
// do not hold back the first records: rice_ranges loads the row pointers,
// rice_first_records (which waits for them) the first batch of records.
__device__ __forceinline__ void rice_ranges(const ResView& v, uint32_t r0, uint32_t r1, RiceTile& t) {
    t.e0 = ldg(v.row_ptr + r0);
    t.e1 = ldg(v.row_ptr + r1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = min(r0 + threadIdx.x + 256u * (uint32_t)h, r1);
        t.my0[h] = ldg(v.row_ptr + row);
        t.my1[h] = ldg(v.row_ptr + min(row + 1u, r1));
    }
}
// rice_ranges for a caller that already holds the range (e0 = row_ptr[r0],
// e1 = row_ptr[r1], say from a table in LDS): only the rows' own pointers
// are loaded, and the first records need not wait for any global load.
__device__ __forceinline__ void rice_ranges_known(const ResView& v, uint32_t r0, uint32_t r1, uint32_t e0,
                                                  uint32_t e1, RiceTile& t) {
    t.e0 = e0;
    t.e1 = e1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = min(r0 + threadIdx.x + 256u * (uint32_t)h, r1);
        t.my0[h] = ldg(v.row_ptr + row);
        t.my1[h] = ldg(v.row_ptr + min(row + 1u, r1));
    }
}
__device__ __forceinline__ void rice_first_records(const ResView& v, RiceTile& t) {
    rice_load_batch(v, t.e0 & ~7u, t.e1, t.rv);
}

__device__ __forceinline__ void rice_prefetch(const ResView& v, uint32_t r0, uint32_t r1, RiceTile& t) {
    t.e0 = ldg(v.row_ptr + r0);
    t.e1 = ldg(v.row_ptr + r1);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = r0 + threadIdx.x + 256u * (uint32_t)h;
        t.my0[h] = t.my1[h] = 0;
        if (row < r1) {
            t.my0[h] = ldg(v.row_ptr + row);
            t.my1[h] = ldg(v.row_ptr + row + 1);
        }
    }
    rice_load_batch(v, t.e0 & ~7u, t.e1, t.rv);
}

// The products of the batch of records at base (staged in t.rv by
// rice_load_batch) into vals: each record's (+-scale) * xs[col], rounded as
// the reference rounds it; a record outside [e0, e1) or a row's padding
// record (column cols) gives -0, which leaves every sum as it is.
__device__ __forceinline__ void rice_products(const ResView& v, const RiceTile& t, uint32_t base, const float* xs,
                                              float* vals) {
    const uint32_t tid = threadIdx.x;
#pragma unroll
    for (uint32_t j = 0; j < RICE_VEC; ++j) {
        const uint32_t e = base + 8u * (tid + 256u * j);
        const uint32_t w[4] = {t.rv[j].x, t.rv[j].y, t.rv[j].z, t.rv[j].w};
        float p[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const uint32_t rec = (w[k >> 1] >> (16 * (k & 1))) & 0xFFFFu, col = rec >> 1;
            const bool in = e + (uint32_t)k >= t.e0 && e + (uint32_t)k < t.e1 && col < v.cols;
            const float xv = xs[in ? col : 0u];
            p[k] = in ? ((rec & 1u) ? v.scale : -v.scale) * xv : -0.0f;
        }
        float4* o = reinterpret_cast<float4*>(vals + 8u * (tid + 256u * j));
        o[0] = make_float4(p[0], p[1], p[2], p[3]);
        o[1] = make_float4(p[4], p[5], p[6], p[7]);
    }
}

// acc[h] += the products in vals (the batch at base) of row h's records, in
// index order.  Rows start at multiples of four records and batches at
// multiples of eight, so a row's products are whole 16-byte pieces: four per
// LDS read, added in order.
__device__ __forceinline__ void rice_row_sums(const RiceTile& t, uint32_t base, const float* vals, float* acc) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t lo = max(t.my0[h], base), hi = min(t.my1[h], base + RICE_BATCH);
        const float4* v4 = reinterpret_cast<const float4*>(vals + (lo - base));
        const uint32_t n4 = hi > lo ? (hi - lo) / 4u : 0u;
#pragma unroll 4
        for (uint32_t j = 0; j < n4; ++j) {
            const float4 q = v4[j];
            acc[h] = (((acc[h] + q.x) + q.y) + q.z) + q.w;
        }
    }
}

// The batches from `first` on (a multiple of eight, its records staged in
// t.rv): products, then each row's sums; every thread of the 256-thread
// workgroup calls this (it synchronises before each batch).
__device__ __forceinline__ void rice_batches_from(const ResView& v, RiceTile& t, uint32_t first, float* acc,
                                                  const float* xs, float* vals) {
    for (uint32_t base = first; base < t.e1; base += RICE_BATCH) {
        __syncthreads();  // xs (first batch) and the previous batch's readers
        rice_products(v, t, base, xs, vals);
        // the next batch's loads are issued before this batch's row sums
        rice_load_batch(v, base + RICE_BATCH, t.e1, t.rv);
        __syncthreads();
        rice_row_sums(t, base, vals, acc);
    }
}

// acc[h] (row r0 + threadIdx.x + 256 h, h = 0, 1) += the row's outliers, in
// index order, of (+-scale) * x[col], for the rows rice_prefetch(v, r0, r1, t)
// started; r1 - r0 <= 512; every thread of the 256-thread workgroup calls
// this (it synchronises).  LDS: xs (cols floats) holds a copy of x -- made
// here unless x_in_lds (the caller copied it and synchronised) -- and vals
// (RICE_BATCH floats) the products.  Each batch is one round of 16-byte
// record loads; the products are formed from the LDS copy of x, and each
// row's thread adds the products of its own records in order -- the
// reference's serial order (binary_rice_q1_matvec_f32,
// q80_mixed_decode.rs:509-527), with the product rounded before the add as
// there.  The records array must be readable in whole 16-byte pieces.
__device__ __forceinline__ void rice_rows_from(const ResView& v, const float* __restrict__ x, RiceTile& t, float* acc,
                                               float* xs, float* vals, bool x_in_lds) {
    if (!x_in_lds)
        copy16_to_lds<4>(reinterpret_cast<uint4*>(xs), reinterpret_cast<const uint4*>(x), v.cols / 4u, threadIdx.x,
                         256u);
    rice_batches_from(v, t, t.e0 & ~7u, acc, xs, vals);
}

// rice_prefetch then rice_rows_from, the first batch's records in flight
// with the copy of x.
__device__ __forceinline__ void rice_rows(const ResView& v, const float* __restrict__ x, uint32_t r0, uint32_t r1,
                                          float* acc, float* xs, float* vals) {
    RiceTile t;
    rice_prefetch(v, r0, r1, t);
    rice_rows_from(v, x, t, acc, xs, vals, false);
}

}  // namespace hk
