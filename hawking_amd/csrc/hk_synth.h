// hk_synth.h -- counter-based synthetic generator (host and device).
//
// Element i of a tensor with key k is N(0, sigma) drawn as Irwin-Hall(12):
// three SplitMix64 words give twelve 16-bit uniforms u_j; the integer
// S = sum(2u_j+1) - 12*2^16 is exact, z = S * 2^-17 is exact in f32, and the
// only rounding step is z * sigma.  Every operation is an integer op or an
// exact f32 op, so the CPU oracle and the GPU produce identical bits.
// Mixed-format coins: group g of a tensor is binary iff the high 32 bits of
// word(coin_key, g) are below floor(0.7 * 2^32).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hk {

__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t stream_key(uint64_t seed, uint64_t stream) {
    return mix64(mix64(seed ^ 0x6A09E667F3BCC909ull) ^ stream);
}

__host__ __device__ __forceinline__ uint64_t stream_word(uint64_t key, uint64_t ctr) {
    return mix64(key + (ctr + 1u) * 0x9E3779B97F4A7C15ull);
}

__host__ __device__ __forceinline__ float synth_normal(uint64_t key, uint64_t index, float sigma) {
    int32_t s = 0;
#pragma unroll
    for (int w = 0; w < 3; ++w) {
        const uint64_t v = stream_word(key, index * 3u + (uint64_t)w);
#pragma unroll
        for (int j = 0; j < 4; ++j) s += (int32_t)((v >> (16 * j)) & 0xFFFFu);
    }
    const int32_t S = 2 * s + 12 - 786432;
    const float z = (float)S * (1.0f / 131072.0f);
    return z * sigma;
}

__host__ __device__ __forceinline__ bool synth_coin(uint64_t coin_key, uint64_t group) {
    return (uint32_t)(stream_word(coin_key, group) >> 32) < 3006477107u;
}

// One organ to generate (device-resident job table entry).
struct SynthJob {
    uint64_t key;
    uint64_t coin_key;
    float sigma;
    int32_t group;
    uint32_t rows;
    uint32_t cols;
    uint16_t* scales;    // Q4 scales / mixed binary scales
    uint8_t* codes;      // Q4 codes / mixed binary signs
    uint8_t* tags;       // mixed
    uint16_t* q2_scales; // mixed
    uint8_t* q2_codes;   // mixed
    uint32_t* row_bin;   // mixed [rows+1]
    uint32_t* row_q2;    // mixed [rows+1]
    float* dense;        // f32
    const float* w;      // mixed: weights to pack instead of generated ones (hk_pack_mixed), or null
};

hipError_t launch_synth_jobs(int kind, const SynthJob* jobs_dev, uint32_t njobs, size_t max_groups,
                             uint32_t* bad, hipStream_t s);
// hk_pack_mixed: tag bytes and the binary count from a per-group selector,
// then the row tables and the packer over the job's dense weights.
hipError_t launch_mixed_tags_from_sel(const uint8_t* sel, size_t groups, uint8_t* tags, uint32_t* count,
                                      hipStream_t s);
hipError_t launch_mixed_pack_buffer(const SynthJob* job_dev, size_t groups, uint32_t* bad, hipStream_t s);
hipError_t launch_synth_mixed_count(const SynthJob* jobs_dev, uint32_t njobs, size_t max_groups,
                                    uint32_t* counts, hipStream_t s);
hipError_t launch_pack_q4(const float* w, size_t groups, int G, uint16_t* scales, uint8_t* codes,
                          uint32_t* bad, hipStream_t s);
hipError_t launch_pack_bin(const float* w, size_t groups, uint16_t* scales, uint8_t* signs,
                           uint32_t* bad, hipStream_t s);
hipError_t launch_pack_q8(const float* w, size_t groups, uint16_t* scales, uint8_t* codes, uint32_t* bad,
                          hipStream_t s);
// 3-bit uniform factor over `count` flat values (groups of 64, the last zero-padded).
hipError_t launch_pack_u3(const float* w, size_t count, uint16_t* scales, uint8_t* codes, uint32_t* bad,
                          hipStream_t s);
hipError_t launch_pack_q2(const float* w, size_t groups, uint16_t* scales, uint8_t* codes,
                          uint32_t* bad, hipStream_t s);
hipError_t launch_synth_normal(uint64_t key, uint64_t first, size_t count, float sigma, float* out,
                               hipStream_t s);

}  // namespace hk
