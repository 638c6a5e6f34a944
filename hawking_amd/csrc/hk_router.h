// hk_router.h -- router launchers and device error bits.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace hk {

// Bits OR-ed into the context's device status word by kernels that detect
// invalid data (read back by hk_check_device_status).
constexpr uint32_t HK_DEVERR_NONFINITE = 1u;
constexpr uint32_t HK_DEVERR_ROUTE = 2u;
constexpr uint32_t HK_DEVERR_STALL = 4u;  // a persistent decode launch gave up waiting for a hand-off

hipError_t launch_softmax_topk(const float* logits, uint32_t n_tokens, uint32_t n, uint32_t k,
                               float tie_eps, int renorm, int32_t* ids, float* weights,
                               uint32_t* status, hipStream_t s);
hipError_t launch_noaux_tc(const float* logits, const float* bias, uint32_t n_tokens, uint32_t n,
                           uint32_t n_group, uint32_t topk_group, uint32_t k, int norm,
                           float scaling, int32_t* ids, float* weights, hipStream_t s);

}  // namespace hk
