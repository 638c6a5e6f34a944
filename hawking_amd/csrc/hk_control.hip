// hk_control.hip -- the achievable-bandwidth control: a read-only stream of
// device memory, run beside the organ GEMVs to measure what HBM delivers on
// this box with the same timing method (the reference runs
// q80_geo_stream_control, shaders/q80_matvec_geometry_gen.metal:80-107,
// beside its matvec geometry sweep for the same purpose).
//
// Each workgroup reads one contiguous slice of the buffer in rounds of
// 256 threads x 8 loads x 16 bytes (32 KiB): every thread issues its 8
// loads before it adds any of them, so 2 KiB per wave are in flight, and the
// workgroup writes one float (the sum of what it read) at the end, so the
// writes are negligible.  The loads carry the non-temporal hint, as the
// weight streams' do (ordinary loads read 6.3-6.5 TB/s here, these 7.1).
#include "hk_internal.h"

namespace hk {

constexpr int CTRL_LOADS = 8;  // 16-byte loads in flight per thread

__global__ void __launch_bounds__(256) stream_control_kernel(const uint4* __restrict__ data, size_t n16,
                                                             size_t per_wg, float* __restrict__ out) {
    __shared__ float red[4];
    const size_t b0 = (size_t)blockIdx.x * per_wg, b1 = min(b0 + per_wg, n16);
    float acc = 0.0f;
    for (size_t base = b0; base < b1; base += 256u * CTRL_LOADS) {
        // unconditional loads (index clamped, value dropped past the slice):
        // a load under a per-lane condition would wait for the one before it
        uint4 v[CTRL_LOADS];
#pragma unroll
        for (int k = 0; k < CTRL_LOADS; ++k) v[k] = ldg_nt(data + min(base + threadIdx.x + 256u * (size_t)k, b1 - 1u));
#pragma unroll
        for (int k = 0; k < CTRL_LOADS; ++k)
            if (base + threadIdx.x + 256u * (size_t)k >= b1) v[k] = make_uint4(0u, 0u, 0u, 0u);
#pragma unroll
        for (int k = 0; k < CTRL_LOADS; ++k)
            acc += __uint_as_float(v[k].x) + __uint_as_float(v[k].y) + __uint_as_float(v[k].z) +
                   __uint_as_float(v[k].w);
    }
    acc = wave_sum(acc);
    if ((threadIdx.x & 63u) == 0u) red[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = red[0] + red[1] + red[2] + red[3];
}

hipError_t launch_stream_control(const void* data, size_t nbytes, float* out, uint32_t workgroups, hipStream_t s) {
    const size_t n16 = nbytes / 16u;
    // slices of whole 32 KiB rounds
    const size_t round = 256u * CTRL_LOADS;
    const size_t per_wg = ((n16 + workgroups - 1u) / workgroups + round - 1u) / round * round;
    hipLaunchKernelGGL(stream_control_kernel, dim3(workgroups), dim3(256), 0, s, static_cast<const uint4*>(data),
                       n16, per_wg, out);
    return hipGetLastError();
}

}  // namespace hk
