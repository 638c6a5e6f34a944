// hk_gemv.hip -- packed-organ row dot products, GEMV and decode kernels.
//
// One wave64 computes one output row: the 64 lanes stride over the row in
// 32-column chunks (one 128-bit load of Q4 codes, one 32-bit load of sign
// bits, or 8 bytes of 2-bit Q2 codes), decode in registers, accumulate in
// f32, and reduce across the wave with xor-shuffles.  Scale association
// follows the reference champion kernels, ((q * s) * x)
// (shaders/qwen_uniform_q4.metal:183-221).
#include "hk_internal.h"
#include "hk_rowdot.h"

namespace hk {

template <int KIND>
__global__ void __launch_bounds__(256) gemv_kernel(OrganView o, const float* __restrict__ x,
                                                  float* __restrict__ y) {
    const int lane = threadIdx.x & 63;
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= o.rows) return;
    float acc = row_dot_partial<KIND>(o, row, x, lane);
    acc = wave_sum(acc);
    if (lane == 0) y[row] = acc;
}

template <int KIND>
__global__ void __launch_bounds__(256) gemv_batch_kernel(const OrganView* __restrict__ organs,
                                                        const float* __restrict__ x,
                                                        size_t x_stride, float* __restrict__ y,
                                                        size_t y_stride) {
    const int lane = threadIdx.x & 63;
    const OrganView o = organs[blockIdx.y];
    const uint32_t row = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= o.rows) return;
    const float* xi = x + (size_t)blockIdx.y * x_stride;
    float acc = row_dot_partial<KIND>(o, row, xi, lane);
    acc = wave_sum(acc);
    if (lane == 0) y[(size_t)blockIdx.y * y_stride + row] = acc;
}

__global__ void decode_rows_kernel(OrganView o, uint32_t row0, uint32_t nrows,
                                   float* __restrict__ out) {
    const size_t total = (size_t)nrows * o.cols;
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (size_t)gridDim.x * blockDim.x) {
        const uint32_t r = row0 + (uint32_t)(i / o.cols);
        const uint32_t c = (uint32_t)(i % o.cols);
        out[i] = decode_weight(o, r, c);
    }
}

hipError_t launch_gemv(const OrganView& o, const float* x, float* y, hipStream_t s) {
    dim3 grid((o.rows + 3) / 4), block(256);
    switch (o.kind) {
    case HK_Q4: hipLaunchKernelGGL(gemv_kernel<HK_Q4>, grid, block, 0, s, o, x, y); break;
    case HK_BIN: hipLaunchKernelGGL(gemv_kernel<HK_BIN>, grid, block, 0, s, o, x, y); break;
    case HK_MIXED: hipLaunchKernelGGL(gemv_kernel<HK_MIXED>, grid, block, 0, s, o, x, y); break;
    case HK_F32: hipLaunchKernelGGL(gemv_kernel<HK_F32>, grid, block, 0, s, o, x, y); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_gemv_batch(const OrganView* organs_dev, uint32_t n, int kind, uint32_t rows,
                             uint32_t cols, int group, const float* x, size_t x_stride,
                             float* y, size_t y_stride, hipStream_t s) {
    (void)cols;
    (void)group;
    dim3 grid((rows + 3) / 4, n), block(256);
    switch (kind) {
    case HK_Q4:
        hipLaunchKernelGGL(gemv_batch_kernel<HK_Q4>, grid, block, 0, s, organs_dev, x, x_stride, y, y_stride);
        break;
    case HK_BIN:
        hipLaunchKernelGGL(gemv_batch_kernel<HK_BIN>, grid, block, 0, s, organs_dev, x, x_stride, y, y_stride);
        break;
    case HK_MIXED:
        hipLaunchKernelGGL(gemv_batch_kernel<HK_MIXED>, grid, block, 0, s, organs_dev, x, x_stride, y, y_stride);
        break;
    case HK_F32:
        hipLaunchKernelGGL(gemv_batch_kernel<HK_F32>, grid, block, 0, s, organs_dev, x, x_stride, y, y_stride);
        break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_decode_rows(const OrganView& o, uint32_t row0, uint32_t nrows, float* out,
                              hipStream_t s) {
    size_t total = (size_t)nrows * o.cols;
    unsigned blocks = (unsigned)((total + 255) / 256);
    if (blocks > 65535u * 16u) blocks = 65535u * 16u;
    if (blocks == 0) return hipSuccess;
    hipLaunchKernelGGL(decode_rows_kernel, dim3(blocks), dim3(256), 0, s, o, row0, nrows, out);
    return hipGetLastError();
}

}  // namespace hk
