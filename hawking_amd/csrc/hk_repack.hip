// hk_repack.hip -- load-time repack of canonical organs into the wavefront-
// tiled layout (hk_tile.h), and the bit-exact decode probe over that layout.
#include <algorithm>

#include "hk_internal.h"
#include "hk_tile.h"

namespace hk {

static inline size_t a256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t tiled_bytes(int kind, int group, uint32_t rows, uint32_t cols, uint32_t n_bin, uint32_t n_q2,
                   size_t* packed_bytes) {
    const size_t nt = n_tiles_for(rows), S = n_steps_for(kind, cols), n = (size_t)rows * cols;
    size_t data = 0, scales = 0, hdr = 0, dense = 0, packed = 0;
    switch (kind) {
    case HK_BIN:
        data = nt * S * 1024;
        scales = nt * 64 * S * 2 + 16;
        packed = n / 8 + n / 128 * 2;
        break;
    case HK_Q4:
        data = nt * S * 1024;
        scales = nt * 64 * S * 2 + 16;
        packed = n / 2 + n / (size_t)group * 2;
        break;
    case HK_Q8:
        data = nt * S * 1024;
        scales = nt * 16 * S * 2 + 16;
        packed = n + n / 64 * 2;
        break;
    case HK_U3: {
        const size_t groups = (n + 63) / 64;
        data = nt * u3_tile_data((uint32_t)S, u3_tail_q(cols));
        scales = nt * u3_tile_scales((uint32_t)S, u3_tail_q(cols)) * 2 + 16;
        packed = groups * 24 + groups * 2;
        break;
    }
    case HK_MIXED: {
        const size_t items = nt * S * 64, pad = items - (size_t)n_bin - n_q2;
        data = ((size_t)n_bin + pad) * 16 + (size_t)n_q2 * 32;
        // each step's scales padded to whole 4-byte words (at most one u16 per step)
        scales = ((size_t)n_bin + pad + 2 * (size_t)n_q2 + nt * S) * 2 + 16;
        hdr = nt * S * 16;
        packed = (n / 128 + 7) / 8 + (size_t)n_bin * 18 + (size_t)n_q2 * 36;
        break;
    }
    default:
        dense = n * 4;
        packed = n * 4;
    }
    if (packed_bytes) *packed_bytes = packed;
    return a256(data) + a256(scales) + a256(hdr) + a256(dense);
}

OrganView tiled_place(int kind, int group, uint32_t rows, uint32_t cols, uint32_t n_bin, uint32_t n_q2,
                      uint8_t* base) {
    OrganView v{};
    v.kind = kind;
    v.group = group;
    v.rows = rows;
    v.cols = cols;
    v.n_tiles = n_tiles_for(rows);
    v.steps = kind == HK_F32 ? 0 : n_steps_for(kind, cols);
    const size_t nt = v.n_tiles, S = v.steps, n = (size_t)rows * cols;
    size_t data = 0, scales = 0, hdr = 0;
    if (kind == HK_BIN || kind == HK_Q4) {
        data = nt * S * 1024;
        scales = nt * 64 * S * 2 + 16;
    } else if (kind == HK_U3) {
        v.tail_q = u3_tail_q(cols);
        data = nt * u3_tile_data((uint32_t)S, v.tail_q);
        scales = nt * u3_tile_scales((uint32_t)S, v.tail_q) * 2 + 16;
    } else if (kind == HK_Q8) {
        data = nt * S * 1024;
        scales = nt * 16 * S * 2 + 16;
    } else if (kind == HK_MIXED) {
        const size_t items = nt * S * 64, pad = items - (size_t)n_bin - n_q2;
        data = ((size_t)n_bin + pad) * 16 + (size_t)n_q2 * 32;
        scales = ((size_t)n_bin + pad + 2 * (size_t)n_q2 + nt * S) * 2 + 16;
        hdr = nt * S * 16;
    }
    uint8_t* p = base;
    v.data = p;
    p += a256(data);
    v.scales = reinterpret_cast<const uint16_t*>(p);
    p += a256(scales);
    v.hdr = reinterpret_cast<const uint4*>(p);
    p += a256(hdr);
    v.dense = reinterpret_cast<const float*>(p);
    (void)n;
    return v;
}

// ------------------------------------------------------------------ BIN / Q4

// Code e of a 3-bit LSB-first stream (extract_unsigned, q80_mixed_decode.rs:579-589).
__device__ inline uint32_t get_code3(const uint8_t* codes, size_t e) {
    const size_t b = 3 * e;
    uint32_t two = codes[b >> 3];
    if ((b & 7u) > 5u) two |= (uint32_t)codes[(b >> 3) + 1] << 8;  // the code straddles a byte
    return (two >> (b & 7u)) & 7u;
}

// One thread per (tile, step, lane) item: copy its 16 bytes and its scale.
__device__ void repack_fixed_body(const CanonView& src, const OrganView& dst) {
    const size_t total = (size_t)dst.n_tiles * dst.steps * 64;
    for (size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (size_t)gridDim.x * blockDim.x) {
        const uint32_t l = (uint32_t)(it & 63), ts = (uint32_t)(it >> 6);
        const uint32_t T = ts / dst.steps, t = ts % dst.steps, n = l & 15u, q = l >> 4;
        const uint32_t r = T * 16u + n;
        uint4 v = make_uint4(0, 0, 0, 0);
        uint16_t s = 0;
        if (src.kind == HK_BIN) {
            const uint32_t g = 4u * t + q;
            if (r < src.rows && g < src.cols / 128u) {
                v = *reinterpret_cast<const uint4*>(src.codes + (size_t)r * (src.cols / 8u) + 16u * g);
                s = src.scales[(size_t)r * (src.cols / 128u) + g];
            }
        } else if (src.kind == HK_Q8) {
            // padding (rows past the end) holds code 127 = 0 with scale 0
            v = make_uint4(0x7F7F7F7Fu, 0x7F7F7F7Fu, 0x7F7F7F7Fu, 0x7F7F7F7Fu);
            if (r < src.rows && t < src.cols / 64u) {
                const size_t e = (size_t)r * src.cols + 64u * t + 16u * q;
                v = *reinterpret_cast<const uint4*>(src.codes + e);
                s = src.scales[e / 64u];
            }
            *reinterpret_cast<uint4*>(const_cast<uint8_t*>(dst.data) + (size_t)ts * 1024u + 16u * l) = v;
            if (q == 0) const_cast<uint16_t*>(dst.scales)[(size_t)ts * 16u + n] = s;
            continue;
        } else {
            const uint32_t c = 4u * t + q;
            if (r < src.rows && c < src.cols / 32u) {
                const size_t e = (size_t)r * src.cols + 32u * c;
                v = *reinterpret_cast<const uint4*>(src.codes + e / 2);
                s = src.scales[e / (uint32_t)src.group];
            }
        }
        *reinterpret_cast<uint4*>(const_cast<uint8_t*>(dst.data) + (size_t)ts * 1024u + 16u * l) = v;
        const_cast<uint16_t*>(dst.scales)[(size_t)ts * 64u + l] = s;
    }
}

// One thread per stored (tile, step, lane) item of a U3 organ: split the 32
// codes of its chunk into the low 2-bit fields and the high bits, copy the
// scale of the flat group holding the chunk.  Padding rows get scale 0.
__device__ void repack_u3_body(const CanonView& src, const OrganView& dst) {
    const uint32_t S = dst.steps, nql = dst.tail_q;
    const size_t per_tile = (size_t)64 * (S - 1) + 16u * nql, total = dst.n_tiles * per_tile;
    const size_t tile_data = u3_tile_data(S, nql), tile_sc = u3_tile_scales(S, nql);
    for (size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (size_t)gridDim.x * blockDim.x) {
        const uint32_t T = (uint32_t)(it / per_tile), rem = (uint32_t)(it % per_tile);
        const uint32_t t = rem / 64u, l = rem % 64u, n = l & 15u, q = l >> 4;
        const uint32_t nq = t + 1 == S ? nql : 4u, r = T * 16u + n;
        uint32_t lo0 = 0, lo1 = 0, hi = 0;
        uint16_t s = 0;
        if (r < src.rows) {
            const size_t e0 = (size_t)r * src.cols + 128u * t + 32u * q;
            for (uint32_t k = 0; k < 32; ++k) {
                const uint32_t code = get_code3(src.codes, e0 + k);
                if (k < 16) lo0 |= (code & 3u) << (2u * k);
                else lo1 |= (code & 3u) << (2u * (k - 16u));
                hi |= (code >> 2) << k;
            }
            s = src.scales[e0 / 64u];
        }
        uint8_t* base = const_cast<uint8_t*>(dst.data) + (size_t)T * tile_data + 768u * t;
        (void)nq;
        uint32_t* lane_words = reinterpret_cast<uint32_t*>(base + 12u * l);
        lane_words[0] = lo0;
        lane_words[1] = lo1;
        lane_words[2] = hi;
        const_cast<uint16_t*>(dst.scales)[(size_t)T * tile_sc + 64u * t + l] = s;
    }
}

// ------------------------------------------------------------------ MIXED

__device__ inline bool canon_is_q2(const CanonView& s, uint32_t r, uint32_t g, bool* valid) {
    *valid = r < s.rows && g < s.cols / 128u;
    if (!*valid) return false;
    const uint32_t fg = r * (s.cols / 128u) + g;
    return !((s.tags[fg >> 3] >> (fg & 7u)) & 1u);
}

// Pass 1: one thread per (tile, step) block: Q2 mask and count.
__device__ void repack_mixed_mask_body(const CanonView& src, const OrganView& dst, uint32_t* counts) {
    const uint32_t nb = dst.n_tiles * dst.steps;
    for (uint32_t b = blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += gridDim.x * blockDim.x) {
        const uint32_t T = b / dst.steps, t = b % dst.steps;
        uint64_t mask = 0;
        for (uint32_t l = 0; l < 64; ++l) {
            bool valid;
            if (canon_is_q2(src, T * 16u + (l & 15u), 4u * t + (l >> 4), &valid)) mask |= 1ull << l;
        }
        uint4* h = const_cast<uint4*>(dst.hdr) + b;
        h->x = (uint32_t)mask;
        h->y = (uint32_t)(mask >> 32);
        counts[b] = __popcll(mask);
    }
}

// Pass 2 (one thread per organ): exclusive prefix of Q2 counts -> data
// offsets; scale offsets advance by 64 + nq2 u16s rounded up to even.
__device__ void repack_mixed_offsets_body(const OrganView& dst, const uint32_t* counts) {
    const uint32_t nb = dst.n_tiles * dst.steps;
    uint32_t q2 = 0, so = 0;
    for (uint32_t b = 0; b < nb; ++b) {
        uint4* h = const_cast<uint4*>(dst.hdr) + b;
        h->z = 16u * (64u * b + q2);
        h->w = so;
        q2 += counts[b];
        so += (64u + counts[b] + 1u) & ~1u;
    }
}

// Pass 3: one thread per item: copy binary signs, or reorder Q2 codes.
__device__ void repack_mixed_items_body(const CanonView& src, const OrganView& dst) {
    const size_t total = (size_t)dst.n_tiles * dst.steps * 64;
    const uint32_t gpr = src.cols / 128u;
    for (size_t it = (size_t)blockIdx.x * blockDim.x + threadIdx.x; it < total;
         it += (size_t)gridDim.x * blockDim.x) {
        const uint32_t l = (uint32_t)(it & 63), b = (uint32_t)(it >> 6);
        const uint32_t T = b / dst.steps, t = b % dst.steps, r = T * 16u + (l & 15u), g = 4u * t + (l >> 4);
        const uint4 h = dst.hdr[b];
        const uint64_t mask = (uint64_t)h.x | ((uint64_t)h.y << 32);
        const uint32_t below = __popcll(mask & ((1ull << l) - 1ull)), nq2 = __popcll(mask);
        uint8_t* item = const_cast<uint8_t*>(dst.data) + h.z + 16u * (l + below);
        bool valid;
        const bool q2 = canon_is_q2(src, r, g, &valid);
        // Q2 pairs first, then the binary (and padding) lanes' scales
        uint16_t* sc = const_cast<uint16_t*>(dst.scales) + h.w + (q2 ? 2u * below : 2u * nq2 + l - below);
        if (!valid) {
            *reinterpret_cast<uint4*>(item) = make_uint4(0, 0, 0, 0);
            sc[0] = 0;
            continue;
        }
        const uint32_t fg = r * gpr + g;
        uint32_t nbin = 0;
        for (uint32_t k = r * gpr; k < fg; ++k) nbin += (src.tags[k >> 3] >> (k & 7u)) & 1u;
        if (!q2) {
            const uint32_t idx = src.row_bin[r] + nbin;
            *reinterpret_cast<uint4*>(item) = *reinterpret_cast<const uint4*>(src.codes + (size_t)idx * 16u);
            sc[0] = src.scales[idx];
        } else {
            const uint32_t idx = src.row_q2[r] + (g - nbin);
            const uint8_t* cs = src.q2_codes + (size_t)idx * 32u;
            uint32_t w[8];
            for (uint32_t a = 0; a < 8; ++a) {
                uint32_t word = 0;
                for (uint32_t j = 0; j < 4; ++j)
                    for (uint32_t u = 0; u < 4; ++u) {
                        const uint32_t e = mixed_q2_col(a, j, u);
                        const uint32_t code = (cs[e >> 2] >> (2u * (e & 3u))) & 3u;
                        word |= code << (8u * j + 2u * u);
                    }
                w[a] = word ^ 0x80808080u;  // top field's high bit inverted (read as code - 2)
            }
            reinterpret_cast<uint4*>(item)[0] = make_uint4(w[0], w[1], w[2], w[3]);
            reinterpret_cast<uint4*>(item)[1] = make_uint4(w[4], w[5], w[6], w[7]);
            sc[0] = src.q2_scales[2u * idx];
            sc[1] = src.q2_scales[2u * idx + 1u];
        }
    }
}

static unsigned grid1(size_t n) {
    size_t b = (n + 255) / 256;
    return (unsigned)(b == 0 ? 1 : (b > 65536 ? 65536 : b));
}

// Single organ (arguments by value) and batched (blockIdx.y = job) forms.
__global__ void repack_fixed_kernel(CanonView src, OrganView dst) { repack_fixed_body(src, dst); }
__global__ void repack_u3_kernel(CanonView src, OrganView dst) { repack_u3_body(src, dst); }
__global__ void repack_u3_batch_kernel(const RepackJob* __restrict__ jobs) {
    repack_u3_body(jobs[blockIdx.y].src, jobs[blockIdx.y].dst);
}
__global__ void repack_mixed_mask_kernel(CanonView src, OrganView dst, uint32_t* counts) {
    repack_mixed_mask_body(src, dst, counts);
}
__global__ void repack_mixed_offsets_kernel(OrganView dst, const uint32_t* counts) {
    if (threadIdx.x == 0) repack_mixed_offsets_body(dst, counts);
}
__global__ void repack_mixed_items_kernel(CanonView src, OrganView dst) { repack_mixed_items_body(src, dst); }

__global__ void repack_fixed_batch_kernel(const RepackJob* __restrict__ jobs) {
    repack_fixed_body(jobs[blockIdx.y].src, jobs[blockIdx.y].dst);
}
__global__ void repack_mixed_mask_batch_kernel(const RepackJob* __restrict__ jobs) {
    repack_mixed_mask_body(jobs[blockIdx.y].src, jobs[blockIdx.y].dst, jobs[blockIdx.y].counts);
}
__global__ void repack_mixed_offsets_batch_kernel(const RepackJob* __restrict__ jobs, uint32_t n) {
    const uint32_t j = blockIdx.x * blockDim.x + threadIdx.x;
    if (j < n) repack_mixed_offsets_body(jobs[j].dst, jobs[j].counts);
}
__global__ void repack_mixed_items_batch_kernel(const RepackJob* __restrict__ jobs) {
    repack_mixed_items_body(jobs[blockIdx.y].src, jobs[blockIdx.y].dst);
}

hipError_t launch_repack(const CanonView& src, const OrganView& dst, void* scratch, hipStream_t s) {
    const size_t items = (size_t)dst.n_tiles * dst.steps * 64;
    if (src.kind == HK_BIN || src.kind == HK_Q4 || src.kind == HK_Q8) {
        hipLaunchKernelGGL(repack_fixed_kernel, dim3(grid1(items)), dim3(256), 0, s, src, dst);
    } else if (src.kind == HK_U3) {
        hipLaunchKernelGGL(repack_u3_kernel, dim3(grid1(items)), dim3(256), 0, s, src, dst);
    } else if (src.kind == HK_MIXED) {
        uint32_t* counts = static_cast<uint32_t*>(scratch);
        hipLaunchKernelGGL(repack_mixed_mask_kernel, dim3(grid1(items / 64)), dim3(256), 0, s, src, dst, counts);
        hipLaunchKernelGGL(repack_mixed_offsets_kernel, dim3(1), dim3(64), 0, s, dst, counts);
        hipLaunchKernelGGL(repack_mixed_items_kernel, dim3(grid1(items)), dim3(256), 0, s, src, dst);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_repack_batch(int kind, const RepackJob* jobs_dev, uint32_t n, size_t max_items, hipStream_t s) {
    if (n == 0) return hipSuccess;
    if (n > 65535) return hipErrorInvalidValue;
    const unsigned gx = std::min(grid1(max_items), 1024u);
    if (kind == HK_BIN || kind == HK_Q4 || kind == HK_Q8) {
        hipLaunchKernelGGL(repack_fixed_batch_kernel, dim3(gx, n), dim3(256), 0, s, jobs_dev);
    } else if (kind == HK_U3) {
        hipLaunchKernelGGL(repack_u3_batch_kernel, dim3(gx, n), dim3(256), 0, s, jobs_dev);
    } else if (kind == HK_MIXED) {
        hipLaunchKernelGGL(repack_mixed_mask_batch_kernel, dim3(std::min(grid1(max_items / 64), 1024u), n), dim3(256),
                           0, s, jobs_dev);
        hipLaunchKernelGGL(repack_mixed_offsets_batch_kernel, dim3((n + 63) / 64), dim3(64), 0, s, jobs_dev, n);
        hipLaunchKernelGGL(repack_mixed_items_batch_kernel, dim3(gx, n), dim3(256), 0, s, jobs_dev);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ------------------------------------------------------------------ decode probe

__global__ void decode_tiled_kernel(OrganView o, uint32_t row0, uint32_t nrows, float* __restrict__ out) {
    const size_t total = (size_t)nrows * o.cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = tiled_weight(o, row0 + (uint32_t)(i / o.cols), (uint32_t)(i % o.cols));
}

hipError_t launch_decode_rows(const OrganView& o, uint32_t row0, uint32_t nrows, float* out, hipStream_t s) {
    const size_t total = (size_t)nrows * o.cols;
    if (!total) return hipSuccess;
    hipLaunchKernelGGL(decode_tiled_kernel, dim3(grid1(total)), dim3(256), 0, s, o, row0, nrows, out);
    return hipGetLastError();
}

}  // namespace hk
