// hk_pack.hip -- device packers and the synthetic weight generator.
//
// Bit-exact with the reference packers: every f32 step is a separate IEEE
// operation (FP contraction is off for this file), divisions are correctly
// rounded (__fdiv_rn), f32->f16 is the hardware round-to-nearest-even
// conversion, rint is roundTiesToEven, and the binary scale is the f64 mean
// rounded to f32 and then to f16 (two roundings), as in pack_binary_group
// (crates/hawking-core/src/model/qwen_complete_binary/q80_mixed_decode.rs:185-230).
#pragma clang fp contract(off)

#include "hk_internal.h"
#include "hk_synth.h"

namespace hk {

// ------------------------------------------------------------------ one group

// pack_uniform_q4_group64 (qwen80_uniform_q4.rs:190-278), one group of G.
template <typename Src>
__device__ void q4_pack_group(const Src& src, int G, uint16_t* scale_out, uint8_t* codes_out,
                              uint32_t* bad) {
    float max_abs = 0.0f;
    for (int i = 0; i < G; ++i) {
        const float v = src(i);
        if (!isfinite(v)) *bad = 1u;
        max_abs = fmaxf(max_abs, fabsf(v));
    }
    const uint16_t sb = f32_to_f16_bits(__fdiv_rn(max_abs, 7.0f));
    if ((sb & 0x7C00u) == 0x7C00u) *bad = 1u;
    const float rs = f16_bits_to_f32(sb);
    *scale_out = sb;
    for (int i = 0; i < G; i += 8) {
        uint32_t word = 0;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            int q = 0;
            if (rs != 0.0f) {
                float r = rintf(__fdiv_rn(src(i + k), rs));
                r = fminf(fmaxf(r, -8.0f), 7.0f);
                q = (int)r;
            }
            word |= (uint32_t)(q + 8) << (4 * k);
        }
        reinterpret_cast<uint32_t*>(codes_out)[i >> 3] = word;
    }
}

// pack_binary_group (q80_mixed_decode.rs:185-230), one group of 128.
template <typename Src>
__device__ void bin_pack_group(const Src& src, uint16_t* scale_out, uint8_t* signs_out,
                               uint32_t* bad) {
    double sum_abs = 0.0;
    uint32_t words[4] = {0, 0, 0, 0};
    for (int i = 0; i < 128; ++i) {
        const float v = src(i);
        if (!isfinite(v)) *bad = 1u;
        sum_abs += (double)fabsf(v);
        if (v >= 0.0f) words[i >> 5] |= 1u << (i & 31);
    }
    const double mean = sum_abs / 128.0;
    *scale_out = f32_to_f16_bits((float)mean);
    *reinterpret_cast<uint4*>(signs_out) = make_uint4(words[0], words[1], words[2], words[3]);
}

// Q2 base stage (ascension_dual_gravity_worker.py:898-911), one group of 64.
template <typename Src>
__device__ void q2_pack_group(const Src& src, uint16_t* scale_out, uint8_t* codes_out,
                              uint32_t* bad) {
    float max_abs = 0.0f;
    for (int i = 0; i < 64; ++i) {
        const float v = src(i);
        if (!isfinite(v)) *bad = 1u;
        max_abs = fmaxf(max_abs, fabsf(v));
    }
    const uint16_t sb = f32_to_f16_bits(__fdiv_rn(max_abs, 1.5f));
    const float sf = f16_bits_to_f32(sb);
    const float denom = sf > 0.0f ? sf : 1.0f;
    *scale_out = sb;
    uint32_t words[4] = {0, 0, 0, 0};
    for (int i = 0; i < 64; ++i) {
        const float n = __fdiv_rn(src(i), denom);
        float r = rintf(n + 1.5f);
        r = fminf(fmaxf(r, 0.0f), 3.0f);
        words[i >> 4] |= (uint32_t)r << (2 * (i & 15));
    }
    *reinterpret_cast<uint4*>(codes_out) = make_uint4(words[0], words[1], words[2], words[3]);
}

// pack_uniform_factor at 8 bits (q80_mixed_decode.rs:529-577), one group of
// 64: scale = f16(max|w| / 127); the quantizer divides by the f32 scale (1 if
// it is 0) and rounds half away from zero (Rust f32::round); code = q + 127.
template <typename Src>
__device__ void q8_pack_group(const Src& src, uint16_t* scale_out, uint8_t* codes_out, uint32_t* bad) {
    float max_abs = 0.0f;
    for (int i = 0; i < 64; ++i) {
        const float v = src(i);
        if (!isfinite(v)) *bad = 1u;
        max_abs = fmaxf(max_abs, fabsf(v));
    }
    const float scale = __fdiv_rn(max_abs, 127.0f);
    const uint16_t sb = f32_to_f16_bits(scale);
    if ((sb & 0x7C00u) == 0x7C00u) *bad = 1u;
    *scale_out = sb;
    const float denom = scale > 0.0f ? scale : 1.0f;
    for (int i = 0; i < 64; i += 16) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const float r = fminf(fmaxf(roundf(__fdiv_rn(src(i + k), denom)), -127.0f), 127.0f);
            w[k >> 2] |= (uint32_t)((int)r + 127) << (8 * (k & 3));
        }
        reinterpret_cast<uint4*>(codes_out)[i >> 4] = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// One flat 64-group of a 3-bit uniform factor (pack_uniform_factor at 3 bits,
// q80_mixed_decode.rs:529-577): bound 3, values past n_valid pack as 0, and the
// 64 codes q + 3 are written LSB-first as 24 bytes.
template <class Src>
__device__ void u3_pack_group(const Src& src, uint32_t n_valid, uint16_t* scale_out, uint8_t* codes_out,
                              uint32_t* bad) {
    float max_abs = 0.0f;
    for (uint32_t i = 0; i < n_valid; ++i) {
        const float v = src((int)i);
        if (!isfinite(v)) *bad = 1u;
        max_abs = fmaxf(max_abs, fabsf(v));
    }
    const float scale = __fdiv_rn(max_abs, 3.0f);
    const uint16_t sb = f32_to_f16_bits(scale);
    if ((sb & 0x7C00u) == 0x7C00u) *bad = 1u;
    *scale_out = sb;
    const float denom = scale > 0.0f ? scale : 1.0f;
    uint64_t w[3] = {0, 0, 0};
#pragma unroll
    for (uint32_t i = 0; i < 64; ++i) {
        const float v = i < n_valid ? src((int)i) : 0.0f;
        const uint64_t code = (uint64_t)((int)fminf(fmaxf(roundf(__fdiv_rn(v, denom)), -3.0f), 3.0f) + 3);
        const uint32_t p = 3u * i;
        w[p >> 6] |= code << (p & 63u);
        if ((p & 63u) > 61u) w[(p >> 6) + 1] |= code >> (64u - (p & 63u));
    }
    uint64_t* o = reinterpret_cast<uint64_t*>(codes_out);
    o[0] = w[0];
    o[1] = w[1];
    o[2] = w[2];
}

struct BufSrc {
    const float* p;
    __device__ float operator()(int i) const { return p[i]; }
};

struct SynthSrc {
    uint64_t key;
    uint64_t base;
    float sigma;
    __device__ float operator()(int i) const { return synth_normal(key, base + (uint64_t)i, sigma); }
};

// ------------------------------------------------------------------ packers over f32 buffers

__global__ void pack_q4_kernel(const float* __restrict__ w, size_t groups, int G,
                               uint16_t* __restrict__ scales, uint8_t* __restrict__ codes,
                               uint32_t* bad) {
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        q4_pack_group(BufSrc{w + g * G}, G, scales + g, codes + g * (G / 2), &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void pack_bin_kernel(const float* __restrict__ w, size_t groups,
                                uint16_t* __restrict__ scales, uint8_t* __restrict__ signs,
                                uint32_t* bad) {
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        bin_pack_group(BufSrc{w + g * 128}, scales + g, signs + g * 16, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void pack_q2_kernel(const float* __restrict__ w, size_t groups,
                               uint16_t* __restrict__ scales, uint8_t* __restrict__ codes,
                               uint32_t* bad) {
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        q2_pack_group(BufSrc{w + g * 64}, scales + g, codes + g * 16, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void pack_q8_kernel(const float* __restrict__ w, size_t groups, uint16_t* __restrict__ scales,
                               uint8_t* __restrict__ codes, uint32_t* bad) {
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        q8_pack_group(BufSrc{w + g * 64}, scales + g, codes + g * 64, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void pack_u3_kernel(const float* __restrict__ w, size_t count, uint16_t* __restrict__ scales,
                               uint8_t* __restrict__ codes, uint32_t* bad) {
    const size_t groups = (count + 63) / 64;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        const uint32_t nv = (uint32_t)(count - g * 64 < 64 ? count - g * 64 : 64);
        u3_pack_group(BufSrc{w + g * 64}, nv, scales + g, codes + g * 24, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void synth_normal_kernel(uint64_t key, uint64_t first, size_t count, float sigma,
                                    float* __restrict__ out) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < count;
         i += (size_t)gridDim.x * blockDim.x)
        out[i] = synth_normal(key, first + i, sigma);
}

static unsigned grid_for(size_t n, unsigned block) {
    size_t b = (n + block - 1) / block;
    if (b > 1u << 20) b = 1u << 20;
    return (unsigned)(b ? b : 1);
}

hipError_t launch_pack_q4(const float* w, size_t groups, int G, uint16_t* scales, uint8_t* codes,
                          uint32_t* bad, hipStream_t s) {
    hipLaunchKernelGGL(pack_q4_kernel, dim3(grid_for(groups, 256)), dim3(256), 0, s, w, groups, G,
                       scales, codes, bad);
    return hipGetLastError();
}

hipError_t launch_pack_bin(const float* w, size_t groups, uint16_t* scales, uint8_t* signs,
                           uint32_t* bad, hipStream_t s) {
    hipLaunchKernelGGL(pack_bin_kernel, dim3(grid_for(groups, 256)), dim3(256), 0, s, w, groups,
                       scales, signs, bad);
    return hipGetLastError();
}

hipError_t launch_pack_q8(const float* w, size_t groups, uint16_t* scales, uint8_t* codes, uint32_t* bad,
                          hipStream_t s) {
    hipLaunchKernelGGL(pack_q8_kernel, dim3(grid_for(groups, 256)), dim3(256), 0, s, w, groups, scales, codes, bad);
    return hipGetLastError();
}

hipError_t launch_pack_u3(const float* w, size_t count, uint16_t* scales, uint8_t* codes, uint32_t* bad,
                          hipStream_t s) {
    hipLaunchKernelGGL(pack_u3_kernel, dim3(grid_for((count + 63) / 64, 256)), dim3(256), 0, s, w, count, scales,
                       codes, bad);
    return hipGetLastError();
}

hipError_t launch_pack_q2(const float* w, size_t groups, uint16_t* scales, uint8_t* codes,
                          uint32_t* bad, hipStream_t s) {
    hipLaunchKernelGGL(pack_q2_kernel, dim3(grid_for(groups, 256)), dim3(256), 0, s, w, groups,
                       scales, codes, bad);
    return hipGetLastError();
}

hipError_t launch_synth_normal(uint64_t key, uint64_t first, size_t count, float sigma, float* out,
                               hipStream_t s) {
    hipLaunchKernelGGL(synth_normal_kernel, dim3(grid_for(count, 256)), dim3(256), 0, s, key, first,
                       count, sigma, out);
    return hipGetLastError();
}

// ------------------------------------------------------------------ synthetic organs
// Generate-and-pack without materialising f32 weights: element e of organ
// (key) is synth_normal(key, e, sigma), so the host oracle regenerates any
// single organ bit for bit.

__global__ void synth_pack_q4_kernel(const SynthJob* __restrict__ jobs, uint32_t njobs,
                                     uint32_t* bad) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t groups = (size_t)j.rows * j.cols / (uint32_t)j.group;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        q4_pack_group(SynthSrc{j.key, g * (uint32_t)j.group, j.sigma}, j.group, j.scales + g,
                      j.codes + g * (uint32_t)(j.group / 2), &b);
        if (b) atomicOr(bad, 1u);
    }
    (void)njobs;
}

__global__ void synth_pack_bin_kernel(const SynthJob* __restrict__ jobs, uint32_t* bad) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t groups = (size_t)j.rows * j.cols / 128;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        bin_pack_group(SynthSrc{j.key, g * 128, j.sigma}, j.scales + g, j.codes + g * 16, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void synth_pack_q8_kernel(const SynthJob* __restrict__ jobs, uint32_t* bad) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t groups = (size_t)j.rows * j.cols / 64;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        q8_pack_group(SynthSrc{j.key, g * 64, j.sigma}, j.scales + g, j.codes + g * 64, &b);
        if (b) atomicOr(bad, 1u);
    }
}

__global__ void synth_pack_u3_kernel(const SynthJob* __restrict__ jobs, uint32_t* bad) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t n = (size_t)j.rows * j.cols, groups = (n + 63) / 64;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x) {
        uint32_t b = 0;
        const uint32_t nv = (uint32_t)(n - g * 64 < 64 ? n - g * 64 : 64);
        u3_pack_group(SynthSrc{j.key, g * 64, j.sigma}, nv, j.scales + g, j.codes + g * 24, &b);
        if (b) atomicOr(bad, 1u);
    }
}

// Mixed, pass 1: tag words (32 flat groups per thread).
__global__ void synth_mixed_tags_kernel(const SynthJob* __restrict__ jobs) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t groups = (size_t)j.rows * j.cols / 128;
    const size_t words = (groups + 31) / 32;
    for (size_t w = (size_t)blockIdx.x * blockDim.x + threadIdx.x; w < words;
         w += (size_t)gridDim.x * blockDim.x) {
        uint32_t t = 0;
        for (uint32_t b = 0; b < 32; ++b) {
            const size_t g = w * 32 + b;
            if (g < groups && synth_coin(j.coin_key, g)) t |= 1u << b;
        }
        reinterpret_cast<uint32_t*>(j.tags)[w] = t;
    }
}

// Mixed, pass 2 (one block per organ): per-row prefix counts.
__global__ void __launch_bounds__(1024) mixed_row_scan_kernel(const SynthJob* __restrict__ jobs) {
    const SynthJob j = jobs[blockIdx.x];
    __shared__ uint32_t part[1024];
    const uint32_t gpr = j.cols / 128;
    const uint32_t tid = threadIdx.x, nt = blockDim.x;
    // rows handled by this thread: contiguous chunk
    const uint32_t per = (j.rows + nt - 1) / nt;
    const uint32_t r0 = tid * per, r1 = min(j.rows, r0 + per);
    uint32_t local = 0;
    for (uint32_t r = r0; r < r1; ++r)
        for (uint32_t g = r * gpr; g < (r + 1) * gpr; ++g) local += (j.tags[g >> 3] >> (g & 7u)) & 1u;
    part[tid] = local;
    __syncthreads();
    if (tid == 0) {
        uint32_t run = 0;
        for (uint32_t t = 0; t < nt; ++t) {
            const uint32_t v = part[t];
            part[t] = run;
            run += v;
        }
    }
    __syncthreads();
    uint32_t run = part[tid];
    for (uint32_t r = r0; r < r1; ++r) {
        j.row_bin[r] = run;
        j.row_q2[r] = r * gpr - run;
        for (uint32_t g = r * gpr; g < (r + 1) * gpr; ++g) run += (j.tags[g >> 3] >> (g & 7u)) & 1u;
    }
    if (r1 == j.rows && r0 < r1) {
        j.row_bin[j.rows] = run;
        j.row_q2[j.rows] = j.rows * gpr - run;
    }
    if (j.rows == 0 && tid == 0) {
        j.row_bin[0] = 0;
        j.row_q2[0] = 0;
    }
}

// Mixed, pass 3: thread per (row, group) generates (or reads, for a job
// with dense weights: hk_pack_mixed) and packs its group.
__global__ void synth_mixed_pack_kernel(const SynthJob* __restrict__ jobs, uint32_t* bad) {
    const SynthJob j = jobs[blockIdx.y];
    const bool buf = j.w != nullptr;
    const uint32_t gpr = j.cols / 128;
    const size_t groups = (size_t)j.rows * gpr;
    for (size_t fg = (size_t)blockIdx.x * blockDim.x + threadIdx.x; fg < groups;
         fg += (size_t)gridDim.x * blockDim.x) {
        const uint32_t r = (uint32_t)(fg / gpr), g = (uint32_t)(fg % gpr);
        uint32_t nb = 0;
        for (uint32_t h = r * gpr; h < (uint32_t)fg; ++h) nb += (j.tags[h >> 3] >> (h & 7u)) & 1u;
        uint32_t b = 0;
        if ((j.tags[fg >> 3] >> (fg & 7u)) & 1u) {
            const uint32_t idx = j.row_bin[r] + nb;
            if (buf)
                bin_pack_group(BufSrc{j.w + fg * 128}, j.scales + idx, j.codes + (size_t)idx * 16, &b);
            else
                bin_pack_group(SynthSrc{j.key, fg * 128, j.sigma}, j.scales + idx, j.codes + (size_t)idx * 16, &b);
        } else {
            const uint32_t idx = j.row_q2[r] + (g - nb);
            for (int half = 0; half < 2; ++half) {
                uint16_t* so = j.q2_scales + 2 * idx + half;
                uint8_t* co = j.q2_codes + (size_t)idx * 32 + 16 * half;
                if (buf)
                    q2_pack_group(BufSrc{j.w + fg * 128 + 64 * half}, so, co, &b);
                else
                    q2_pack_group(SynthSrc{j.key, fg * 128 + 64 * (uint64_t)half, j.sigma}, so, co, &b);
            }
        }
        if (b) atomicOr(bad, 1u);
    }
}

// hk_pack_mixed, pass 1: tag bytes from a per-group selector (8 groups per
// thread) and the binary-group count.
__global__ void mixed_tags_from_sel_kernel(const uint8_t* __restrict__ sel, size_t groups, uint8_t* __restrict__ tags,
                                           uint32_t* count) {
    uint32_t local = 0;
    for (size_t b = (size_t)blockIdx.x * blockDim.x + threadIdx.x; b < (groups + 7) / 8;
         b += (size_t)gridDim.x * blockDim.x) {
        uint32_t t = 0;
        for (uint32_t k = 0; k < 8; ++k) {
            const size_t g = b * 8 + k;
            if (g < groups && sel[g]) t |= 1u << k;
        }
        tags[b] = (uint8_t)t;
        local += (uint32_t)__builtin_popcount(t);
    }
    for (int off = 32; off >= 1; off >>= 1) local += __shfl_xor(local, off, 64);
    if ((threadIdx.x & 63) == 0 && local) atomicAdd(count, local);
}

hipError_t launch_mixed_tags_from_sel(const uint8_t* sel, size_t groups, uint8_t* tags, uint32_t* count,
                                      hipStream_t s) {
    hipLaunchKernelGGL(mixed_tags_from_sel_kernel, dim3(grid_for((groups + 7) / 8, 256)), dim3(256), 0, s, sel,
                       groups, tags, count);
    return hipGetLastError();
}

// hk_pack_mixed, passes 2-3 on one job (tags, row tables, w).
hipError_t launch_mixed_pack_buffer(const SynthJob* job_dev, size_t groups, uint32_t* bad, hipStream_t s) {
    hipLaunchKernelGGL(mixed_row_scan_kernel, dim3(1), dim3(1024), 0, s, job_dev);
    hipLaunchKernelGGL(synth_mixed_pack_kernel, dim3(grid_for(groups, 256) < 4096 ? grid_for(groups, 256) : 4096, 1),
                       dim3(256), 0, s, job_dev, bad);
    return hipGetLastError();
}

// Mixed: count binary groups per organ (for exact allocation).
__global__ void synth_mixed_count_kernel(const SynthJob* __restrict__ jobs, uint32_t* counts) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t groups = (size_t)j.rows * j.cols / 128;
    uint32_t local = 0;
    for (size_t g = (size_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
         g += (size_t)gridDim.x * blockDim.x)
        local += synth_coin(j.coin_key, g) ? 1u : 0u;
    for (int off = 32; off >= 1; off >>= 1) local += __shfl_xor(local, off, 64);
    if ((threadIdx.x & 63) == 0 && local) atomicAdd(counts + blockIdx.y, local);
}

__global__ void synth_dense_kernel(const SynthJob* __restrict__ jobs) {
    const SynthJob j = jobs[blockIdx.y];
    const size_t n = (size_t)j.rows * j.cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (size_t)gridDim.x * blockDim.x)
        j.dense[i] = synth_normal(j.key, i, j.sigma);
}

hipError_t launch_synth_jobs(int kind, const SynthJob* jobs_dev, uint32_t njobs,
                             size_t max_groups, uint32_t* bad, hipStream_t s) {
    const unsigned bx = (unsigned)((max_groups + 255) / 256 < 4096 ? (max_groups + 255) / 256 : 4096);
    switch (kind) {
    case HK_Q4:
        hipLaunchKernelGGL(synth_pack_q4_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev,
                           njobs, bad);
        break;
    case HK_BIN:
        hipLaunchKernelGGL(synth_pack_bin_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev, bad);
        break;
    case HK_U3:
        hipLaunchKernelGGL(synth_pack_u3_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev, bad);
        break;
    case HK_Q8:
        hipLaunchKernelGGL(synth_pack_q8_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev, bad);
        break;
    case HK_MIXED: {
        const size_t words = (max_groups + 31) / 32;
        const unsigned tx = (unsigned)((words + 255) / 256 < 4096 ? (words + 255) / 256 : 4096);
        hipLaunchKernelGGL(synth_mixed_tags_kernel, dim3(tx ? tx : 1, njobs), dim3(256), 0, s, jobs_dev);
        hipLaunchKernelGGL(mixed_row_scan_kernel, dim3(njobs), dim3(1024), 0, s, jobs_dev);
        hipLaunchKernelGGL(synth_mixed_pack_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev,
                           bad);
        break;
    }
    case HK_F32:
        hipLaunchKernelGGL(synth_dense_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_synth_mixed_count(const SynthJob* jobs_dev, uint32_t njobs, size_t max_groups,
                                    uint32_t* counts, hipStream_t s) {
    const unsigned bx = (unsigned)((max_groups + 255) / 256 < 1024 ? (max_groups + 255) / 256 : 1024);
    hipLaunchKernelGGL(synth_mixed_count_kernel, dim3(bx ? bx : 1, njobs), dim3(256), 0, s, jobs_dev,
                       counts);
    return hipGetLastError();
}

}  // namespace hk
