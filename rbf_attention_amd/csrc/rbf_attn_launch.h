// Per-dtype launchers (defined in rbf_attn_launch.hip, compiled once per
// element type) used by the C ABI in rbf_attn_capi.hip.
#pragma once

#include <hip/hip_runtime.h>

namespace rbf {

struct Params;

// variant: 0 = softmax, 1 = non-softmax.  Return the launch status.
#define RBF_DECLARE_LAUNCHERS(NAME)                                              \
  hipError_t launch_fwd_##NAME(const Params& p, int variant, hipStream_t st);   \
  hipError_t launch_bwd_dq_##NAME(const Params& p, int variant, hipStream_t st); \
  hipError_t launch_bwd_dkdv_##NAME(const Params& p, int variant, hipStream_t st);

RBF_DECLARE_LAUNCHERS(bf16)
RBF_DECLARE_LAUNCHERS(fp16)
RBF_DECLARE_LAUNCHERS(fp32)

#undef RBF_DECLARE_LAUNCHERS

}  // namespace rbf
