// hk_rice.hip -- HGRAVR02 organs: a binary group-128 base plus the global
// top-2% residual stored as Rice-coded index gaps and one sign bit each,
// every outlier worth +-(f16 RMS of the selected residuals)
// (pack_binary_rice_q1 / binary_rice_q1_matvec_f32,
// model/qwen_complete_binary/q80_mixed_decode.rs:260-527).
//
// The Rice stream is decoded once at bind time (on the host, in hk_api.cpp)
// into a CSR over rows (row_ptr plus one u16 record per outlier:
// column << 1 | sign, each row padded to a multiple of four records).  Per
// token the base runs on the tiled binary GEMV and rice_apply adds the
// outliers, each row's thread adding its products in index order -- the
// reference's serial apply order, so given the same base the correction is
// bit-exact.
#include <rocprim/device/device_radix_sort.hpp>
#include <rocprim/device/device_scan.hpp>

#include "hk_internal.h"
#include "hk_rice.h"
#include "hk_synth.h"

namespace hk {

// ------------------------------------------------------------------ bind time

__global__ void f16_check_kernel(const uint16_t* __restrict__ v, size_t n, uint32_t* status) {
    bool bad = false;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
        bad |= (v[i] & 0x7C00u) == 0x7C00u;
    if (__any(bad) && (threadIdx.x & 63) == 0) atomicOr(status, 16u);
}

hipError_t launch_f16_check(const uint16_t* v, size_t n, uint32_t* status, hipStream_t s) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(f16_check_kernel, dim3((unsigned)std::min<size_t>((n + 255) / 256, 1024)), dim3(256), 0, s, v,
                       n, status);
    return hipGetLastError();
}

// ------------------------------------------------------------------ per token

constexpr uint32_t RICE_ROWS_PER_WG = 256;  // at most 512 (two rows per thread)
constexpr size_t RICE_APPLY_LDS_MAX = 64u * 1024u;

// y[row] += sum over the row's outliers, in index order, of (+-scale) * x[col]
// (the apply on its own, for a base computed elsewhere).
// Dynamic LDS: x (cols floats), then RICE_BATCH products.
__global__ void __launch_bounds__(256) rice_apply_kernel(const ResView* __restrict__ views, uint32_t n,
                                                         const float* __restrict__ xall, size_t x_stride,
                                                         float* __restrict__ yall, size_t y_stride, uint32_t parts) {
    extern __shared__ __align__(16) float rice_lds[];
    uint32_t oi, part;
    organ_part(blockIdx.x, parts, n, &oi, &part);
    const ResView v = views[oi];
    const float* __restrict__ x = xall + (size_t)oi * x_stride;
    float* __restrict__ y = yall + (size_t)oi * y_stride;
    const uint32_t r0 = part * RICE_ROWS_PER_WG;
    if (r0 >= v.rows) return;  // uniform over the workgroup
    const uint32_t r1 = min(r0 + RICE_ROWS_PER_WG, v.rows);
    float acc[2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = r0 + threadIdx.x + 256u * (uint32_t)h;
        acc[h] = row < r1 ? y[row] : 0.0f;
    }
    rice_rows(v, x, r0, r1, acc, rice_lds, rice_lds + v.cols);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint32_t row = r0 + threadIdx.x + 256u * (uint32_t)h;
        if (row < r1) y[row] = acc[h];
    }
}

// The apply with one thread per row: a workgroup of RICE_APPLY_ROWS threads
// owns that many rows of one residual, loads every record piece its rows
// span in one round (part 0 starts at record 0, so its loads wait for
// nothing but the residual's view), stages them in LDS next to the signed
// product table T[2 c + sign] = (sign ? scale : -scale) * x[c] (T[2 cols] =
// -0, the padding records' entry: x + -0 is x for every x), and each thread
// adds its row's products in index order, four records per LDS read (rows
// are padded to multiples of four).  Same sums as rice_apply_kernel, to the
// bit: (-scale) * x is -(scale * x) exactly.  NP pieces per thread cover
// `pieces` (<= NP * RICE_APPLY_ROWS).
template <int NP>
__global__ void __launch_bounds__(RICE_APPLY_ROWS)
rice_apply_rows_kernel(const ResView* __restrict__ views, uint32_t n, const float* __restrict__ xall, size_t x_stride,
                       float* __restrict__ yall, size_t y_stride, uint32_t parts, uint32_t pieces) {
    extern __shared__ __align__(16) uint8_t rl[];
    uint32_t oi, part;
    organ_part(blockIdx.x, parts, n, &oi, &part);
    const ResView v = views[oi];
    const uint32_t tid = threadIdx.x, r0 = part * RICE_APPLY_ROWS;
    if (r0 >= v.rows || v.count == 0u) return;  // uniform over the workgroup
    const uint32_t r1 = min(r0 + RICE_APPLY_ROWS, v.rows);
    const float* __restrict__ x = xall + (size_t)oi * x_stride;
    float* __restrict__ y = yall + (size_t)oi * y_stride;
    uint32_t p0 = 0;
    if (part) p0 = ldg(v.row_ptr + r0) / 8u;
    // unconditional loads, clamped to the residual's last piece: a load under
    // a per-lane condition would wait for the ones before it
    const uint4* recs = reinterpret_cast<const uint4*>(v.recs);
    const uint32_t plast = (v.count + 7u) / 8u - 1u;
    uint4 rv[NP];
#pragma unroll
    for (int j = 0; j < NP; ++j) rv[j] = ldg(recs + min(p0 + tid + RICE_APPLY_ROWS * (uint32_t)j, plast));
    const bool mine = tid < r1 - r0;
    const uint32_t row = mine ? r0 + tid : r0;
    const uint32_t my0 = ldg(v.row_ptr + row), my1 = mine ? ldg(v.row_ptr + row + 1u) : my0;
    float acc = ldg(y + row);
    float2* T = reinterpret_cast<float2*>(rl);
#pragma unroll 4
    for (uint32_t c = tid; c < v.cols; c += RICE_APPLY_ROWS) {
        const float p = v.scale * ldg(x + c);
        T[c] = make_float2(-p, p);
    }
    if (tid == 0) T[v.cols] = make_float2(-0.0f, -0.0f);
    uint4* R = reinterpret_cast<uint4*>(rl + rice_table_bytes(v.cols));
#pragma unroll
    for (int j = 0; j < NP; ++j)
        if (tid + RICE_APPLY_ROWS * (uint32_t)j < pieces) R[tid + RICE_APPLY_ROWS * j] = rv[j];
    __syncthreads();
    const float* Tf = reinterpret_cast<const float*>(rl);
    const uint2* R2 = reinterpret_cast<const uint2*>(R);
#pragma unroll 2
    for (uint32_t e = my0; e < my1; e += 4u) {
        const uint2 w = R2[(e - 8u * p0) / 4u];
        acc += Tf[w.x & 0xFFFFu];
        acc += Tf[w.x >> 16];
        acc += Tf[w.y & 0xFFFFu];
        acc += Tf[w.y >> 16];
    }
    if (mine) y[row] = acc;
}

uint32_t rice_part_pieces(const uint32_t* row_ptr, uint32_t rows, uint32_t part_rows) {
    uint32_t most = 0;
    for (uint32_t r0 = 0; r0 < rows; r0 += part_rows) {
        const uint32_t r1 = std::min(r0 + part_rows, rows);
        most = std::max(most, (row_ptr[r1] + 7u) / 8u - row_ptr[r0] / 8u);
    }
    return most;
}

uint32_t rice_part_pieces8(const uint32_t* row_ptr8, uint32_t rows, uint32_t part_rows) {
    uint32_t most = 0;
    for (uint32_t r0 = 0; r0 < rows; r0 += part_rows) {
        const uint32_t r1 = std::min(r0 + part_rows, rows);
        most = std::max(most, (row_ptr8[r1] + 15u) / 16u - row_ptr8[r0] / 16u);
    }
    return most;
}

hipError_t launch_rice_apply(const ResView* res_dev, uint32_t n, uint32_t rows, uint32_t cols, uint32_t pieces,
                             const float* x, size_t x_stride, float* y, size_t y_stride, hipStream_t s) {
    if (n == 0 || rows == 0) return hipSuccess;
    const uint32_t np = (pieces + RICE_APPLY_ROWS - 1u) / RICE_APPLY_ROWS;
    const size_t lds_rows = rice_table_bytes(cols) + (size_t)pieces * 16u;
    if (np >= 1u && np <= 8u && lds_rows <= RICE_APPLY_LDS_MAX) {
        const uint32_t parts = (rows + RICE_APPLY_ROWS - 1u) / RICE_APPLY_ROWS;
        const dim3 g(parts * n), b(RICE_APPLY_ROWS);
#define HK_RICE_ROWS(NP)                                                                                            \
    case NP:                                                                                                        \
        hipLaunchKernelGGL(rice_apply_rows_kernel<NP>, g, b, lds_rows, s, res_dev, n, x, x_stride, y, y_stride, parts, \
                           pieces);                                                                                 \
        break;
        switch (np) {
            HK_RICE_ROWS(1)
            HK_RICE_ROWS(2)
            HK_RICE_ROWS(3)
            HK_RICE_ROWS(4)
            HK_RICE_ROWS(5)
            HK_RICE_ROWS(6)
            HK_RICE_ROWS(7)
            HK_RICE_ROWS(8)
        }
#undef HK_RICE_ROWS
        return hipGetLastError();
    }
    const uint32_t parts = (rows + RICE_ROWS_PER_WG - 1) / RICE_ROWS_PER_WG;
    const size_t lds = ((size_t)cols + RICE_BATCH) * sizeof(float);
    hipLaunchKernelGGL(rice_apply_kernel, dim3(parts * n), dim3(256), lds, s, res_dev, n, x, x_stride, y, y_stride,
                       parts);
    return hipGetLastError();
}

// Decode probe: out[(row - row0) * cols + col] += +-scale for every outlier of
// rows [row0, row0 + nrows) (out already holds the decoded base).
__global__ void rice_decode_add_kernel(ResView v, uint32_t row0, uint32_t nrows, float* __restrict__ out) {
    const uint32_t e0 = v.row_ptr[row0], e1 = v.row_ptr[row0 + nrows];
    for (uint32_t e = e0 + blockIdx.x * blockDim.x + threadIdx.x; e < e1; e += gridDim.x * blockDim.x) {
        // the outlier's row: the last r with row_ptr[r] <= e
        uint32_t lo = row0, hi = row0 + nrows;
        while (hi - lo > 1) {
            const uint32_t mid = (lo + hi) >> 1;
            if (v.row_ptr[mid] <= e) lo = mid;
            else hi = mid;
        }
        const uint32_t rec = v.recs[e], col = rec >> 1;
        if (col < v.cols) atomicAdd(out + (size_t)(lo - row0) * v.cols + col, (rec & 1u) ? v.scale : -v.scale);
    }
}

hipError_t launch_rice_decode_add(const ResView& v, uint32_t row0, uint32_t nrows, float* out, hipStream_t s) {
    if (!nrows) return hipSuccess;
    hipLaunchKernelGGL(rice_decode_add_kernel, dim3(256), dim3(256), 0, s, v, row0, nrows, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------ packer

// Residual against the binary base and the sort keys: ascending ~bits(|r|)
// is descending |r|, and the stable sort keeps ties in index order.
__global__ void rice_residual_kernel(const float* __restrict__ w, size_t n, const uint16_t* __restrict__ bs,
                                     const uint8_t* __restrict__ bg, float* __restrict__ r, uint32_t* __restrict__ key,
                                     uint32_t* __restrict__ val) {
    for (size_t f = (size_t)blockIdx.x * blockDim.x + threadIdx.x; f < n; f += (size_t)gridDim.x * blockDim.x) {
        const float s = f16_bits_to_f32(bs[f / 128]);
        const float rv = w[f] - (((bg[f >> 3] >> (f & 7u)) & 1u) ? s : -s);
        r[f] = rv;
        key[f] = ~__float_as_uint(fabsf(rv));
        val[f] = (uint32_t)f;
    }
}

struct RiceStats {
    uint32_t k;
    uint32_t pad;
    uint64_t bits;
    uint16_t scale;
};

// One block: the selected residuals in index order (sel, count floats,
// 16-byte aligned), their sign bits, best_rice_k over the gaps (first
// minimum), and the f16 RMS scale: the f64 sum of squares in index order on
// one thread, as the reference (each square of an f32 is exact in f64, so a
// fused multiply-add rounds the same as the reference's multiply then add).
__global__ void __launch_bounds__(256) rice_stats_kernel(const float* __restrict__ r, const uint32_t* __restrict__ idx,
                                                         size_t count, float* __restrict__ sel,
                                                         uint8_t* __restrict__ signs, RiceStats* __restrict__ out) {
    __shared__ uint64_t part[16][256 / 64];
    const uint32_t tid = threadIdx.x;
    for (size_t b = tid; b < (count + 7) / 8; b += 256) {
        uint32_t byte = 0;
        for (uint32_t i = 0; i < 8 && 8 * b + i < count; ++i) {
            const float v = r[idx[8 * b + i]];
            sel[8 * b + i] = v;
            byte |= (v >= 0.0f ? 1u : 0u) << i;
        }
        signs[b] = (uint8_t)byte;
    }
    uint64_t q[16];
#pragma unroll
    for (int k = 0; k < 16; ++k) q[k] = 0;
    for (size_t i = 1 + tid; i < count; i += 256) {
        const uint32_t d = idx[i] - idx[i - 1];
#pragma unroll
        for (int k = 0; k < 16; ++k) q[k] += d >> k;
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        uint64_t v = q[k];
        for (int off = 32; off; off >>= 1) v += __shfl_xor(v, off, 64);
        if ((tid & 63) == 0) part[k][tid >> 6] = v;
    }
    __syncthreads();
    if (tid == 0) {
        const uint64_t nd = count > 0 ? count - 1 : 0;
        uint32_t best_k = 0;
        uint64_t best = ~0ull;
        for (int k = 0; k < 16 && nd; ++k) {
            const uint64_t bits = part[k][0] + part[k][1] + part[k][2] + part[k][3] + nd * (1u + (uint64_t)k);
            if (bits < best) {
                best = bits;
                best_k = (uint32_t)k;
            }
        }
        double sum_sq = 0.0;
        size_t i = 0;
        for (; i + 16 <= count; i += 16) {  // 16 values in flight per round
            float4 v[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = reinterpret_cast<const float4*>(sel + i)[j];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                sum_sq += (double)v[j].x * (double)v[j].x;
                sum_sq += (double)v[j].y * (double)v[j].y;
                sum_sq += (double)v[j].z * (double)v[j].z;
                sum_sq += (double)v[j].w * (double)v[j].w;
            }
        }
        for (; i < count; ++i) sum_sq += (double)sel[i] * (double)sel[i];
        float scale = (float)sqrt(sum_sq / (double)count);
        if (!isfinite(scale) || scale <= 0.0f) scale = 1.0f;
        out->k = best_k;
        out->bits = nd ? best : 0;
        out->scale = f32_to_f16_bits(scale);
    }
}

// Rice code length of gap i (pack_rice, q80_mixed_decode.rs:335-346).
__global__ void rice_len_kernel(const uint32_t* __restrict__ idx, size_t nd, const RiceStats* __restrict__ st,
                                uint64_t* __restrict__ len) {
    const uint32_t k = st->k;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nd; i += (size_t)gridDim.x * blockDim.x)
        len[i] = (uint64_t)((idx[i + 1] - idx[i]) >> k) + 1u + k;
}

__device__ __forceinline__ void or_bits(uint32_t* words, uint64_t pos, uint32_t n, uint32_t value) {
    // n <= 32 bits of value at bit pos, LSB first
    const uint64_t v = (uint64_t)value << (pos & 31u);
    atomicOr(words + (pos >> 5), (uint32_t)v);
    if ((pos & 31u) + n > 32u) atomicOr(words + (pos >> 5) + 1, (uint32_t)(v >> 32));
}

// Each gap writes its own bits: q ones, a zero, k remainder bits.
__global__ void rice_write_kernel(const uint32_t* __restrict__ idx, size_t nd, const RiceStats* __restrict__ st,
                                  const uint64_t* __restrict__ off, uint32_t* __restrict__ words) {
    const uint32_t k = st->k;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < nd; i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t d = idx[i + 1] - idx[i];
        uint64_t pos = off[i];
        for (uint32_t q = d >> k; q;) {
            const uint32_t take = min(q, 32u - (uint32_t)(pos & 31u));
            or_bits(words, pos, take, take == 32u ? 0xFFFFFFFFu : ((1u << take) - 1u));
            pos += take;
            q -= take;
        }
        pos += 1;  // the terminating zero
        if (k) or_bits(words, pos, k, d & ((1u << k) - 1u));
    }
}

static unsigned grid_n(size_t n) { return (unsigned)std::min<size_t>((n + 255) / 256 ? (n + 255) / 256 : 1, 4096); }

hipError_t pack_binary_rice_device(const float* w, uint32_t rows, uint32_t cols, double ratio, uint16_t* bin_scales,
                                   uint8_t* bin_signs, uint8_t* res_signs, uint8_t* rice, size_t rice_cap,
                                   RicePackResult* out, hipStream_t s) {
    const size_t n = (size_t)rows * cols;
    size_t count = (size_t)ceil((double)n * ratio);
    count = count < 1 ? 1 : (count > n ? n : count);
    *out = RicePackResult{};
    out->count = count;
    hipError_t e = hipSuccess;
    // layout of one temporary allocation
    size_t sort_tmp = 0, sort_tmp2 = 0, scan_tmp = 0;
    if ((e = rocprim::radix_sort_pairs(nullptr, sort_tmp, (const uint32_t*)nullptr, (uint32_t*)nullptr,
                                       (const uint32_t*)nullptr, (uint32_t*)nullptr, n, 0u, 32u, s)))
        return e;
    if ((e = rocprim::radix_sort_keys(nullptr, sort_tmp2, (const uint32_t*)nullptr, (uint32_t*)nullptr, count, 0u, 32u,
                                      s)))
        return e;
    const size_t nd = count - 1;
    if (nd && (e = rocprim::exclusive_scan(nullptr, scan_tmp, (const uint64_t*)nullptr, (uint64_t*)nullptr, (uint64_t)0,
                                           nd, rocprim::plus<uint64_t>(), s)))
        return e;
    auto al = [](size_t b) { return (b + 255) & ~(size_t)255; };
    const size_t tmp_bytes = std::max(sort_tmp, std::max(sort_tmp2, scan_tmp));
    const size_t total =
        al(n * 4) * 5 + al(count * 4) * 2 + al(nd * 8) * 2 + al(sizeof(RiceStats)) + al(tmp_bytes) + 256;
    uint8_t* mem = nullptr;
    if ((e = hipMalloc(&mem, total))) return e;
    uint8_t* p = mem;
    auto take = [&](size_t b) {
        uint8_t* q = p;
        p += al(b);
        return q;
    };
    float* r = (float*)take(n * 4);
    uint32_t* key = (uint32_t*)take(n * 4);
    uint32_t* key2 = (uint32_t*)take(n * 4);
    uint32_t* val = (uint32_t*)take(n * 4);
    uint32_t* val2 = (uint32_t*)take(n * 4);
    uint32_t* idx = (uint32_t*)take(count * 4);
    float* sel = (float*)take(count * 4);
    uint64_t* len = (uint64_t*)take(nd * 8);
    uint64_t* off = (uint64_t*)take(nd * 8);
    RiceStats* st = (RiceStats*)take(sizeof(RiceStats));
    void* tmp = take(tmp_bytes);
    uint32_t* bad = (uint32_t*)take(4);
    RiceStats hs{};
    uint32_t hbad = 0;
    do {
        if ((e = hipMemsetAsync(bad, 0, 4, s))) break;
        if ((e = launch_pack_bin(w, n / 128, bin_scales, bin_signs, bad, s))) break;
        hipLaunchKernelGGL(rice_residual_kernel, dim3(grid_n(n)), dim3(256), 0, s, w, n, bin_scales, bin_signs, r, key,
                           val);
        if ((e = hipGetLastError())) break;
        size_t tb = tmp_bytes;
        if ((e = rocprim::radix_sort_pairs(tmp, tb, key, key2, val, val2, n, 0u, 32u, s))) break;
        tb = tmp_bytes;
        if ((e = rocprim::radix_sort_keys(tmp, tb, val2, idx, count, 0u, 32u, s))) break;
        hipLaunchKernelGGL(rice_stats_kernel, dim3(1), dim3(256), 0, s, r, idx, count, sel, res_signs, st);
        if ((e = hipGetLastError())) break;
        if ((e = hipMemcpyAsync(&hs, st, sizeof(hs), hipMemcpyDeviceToHost, s))) break;
        if ((e = hipMemcpyAsync(&out->first, idx, 4, hipMemcpyDeviceToHost, s))) break;
        if ((e = hipMemcpyAsync(&hbad, bad, 4, hipMemcpyDeviceToHost, s))) break;
        if ((e = hipStreamSynchronize(s))) break;
        out->k = hs.k;
        out->scale = hs.scale;
        out->bad = hbad;
        out->rice_bytes = (size_t)((hs.bits + 7) / 8);
        if (!nd) break;
        // the writer ors whole words: the buffer must hold them
        if (((hs.bits + 31) / 32) * 4 > rice_cap) {
            e = hipErrorInvalidValue;
            break;
        }
        hipLaunchKernelGGL(rice_len_kernel, dim3(grid_n(nd)), dim3(256), 0, s, idx, nd, st, len);
        if ((e = hipGetLastError())) break;
        tb = tmp_bytes;
        if ((e = rocprim::exclusive_scan(tmp, tb, len, off, (uint64_t)0, nd, rocprim::plus<uint64_t>(), s))) break;
        if ((e = hipMemsetAsync(rice, 0, ((hs.bits + 31) / 32) * 4, s))) break;
        hipLaunchKernelGGL(rice_write_kernel, dim3(grid_n(nd)), dim3(256), 0, s, idx, nd, st, off,
                           reinterpret_cast<uint32_t*>(rice));
        if ((e = hipGetLastError())) break;
        e = hipStreamSynchronize(s);
    } while (false);
    (void)hipStreamSynchronize(s);
    (void)hipFree(mem);
    return e;
}

}  // namespace hk
