// Per-dtype launchers (defined in rbf_attn_launch.hip, compiled once per
// element type) used by the C ABI in rbf_attn_capi.hip.
#pragma once

#include <hip/hip_runtime.h>

namespace rbf {

struct Params;
struct DecodeParams;

// variant: 0 = softmax, 1 = non-softmax.  Return the launch status.
// launch_bwd_* is the whole backward (dQ, then dK/dV); bwd_kernels_* is the
// number of kernels it enqueues for p (1 or 2).
#define RBF_DECLARE_LAUNCHERS(NAME)                                              \
  hipError_t launch_fwd_##NAME(const Params& p, int variant, hipStream_t st);   \
  hipError_t launch_bwd_dq_##NAME(const Params& p, int variant, hipStream_t st); \
  hipError_t launch_bwd_dkdv_##NAME(const Params& p, int variant, hipStream_t st); \
  hipError_t launch_bwd_##NAME(const Params& p, int variant, hipStream_t st);      \
  int bwd_kernels_##NAME(const Params& p);                                          \
  hipError_t launch_decode_##NAME(const DecodeParams& p, int variant, hipStream_t st);

RBF_DECLARE_LAUNCHERS(bf16)
RBF_DECLARE_LAUNCHERS(fp16)
RBF_DECLARE_LAUNCHERS(fp32)

#undef RBF_DECLARE_LAUNCHERS

// fp32 kernels with 256 features, compiled in a unit of their own
// (rbf_attn_launch.hip with RBF_WIDE, register classes left to the compiler).
hipError_t launch_fwd_wide_fp32(const Params& p, int variant, hipStream_t st);
hipError_t launch_bwd_dq_wide_fp32(const Params& p, int variant, hipStream_t st);
hipError_t launch_bwd_dkdv_wide_fp32(const Params& p, int variant, hipStream_t st);
hipError_t launch_decode_wide_fp32(const DecodeParams& p, int variant, hipStream_t st);

// Head-resident kernels (16-bit elements, 32 < D <= 64, N <= 32 * kHrMaxBlocks;
// defined in rbf_attn_launch_hr.hip).  They return hipErrorInvalidValue for
// shapes they do not cover.
constexpr int kHrMaxBlocks = 18;

#define RBF_DECLARE_HR_LAUNCHERS(NAME)                                                         \
  hipError_t launch_fwd_hr_##NAME(const Params& p, int variant, int waves, hipStream_t st);   \
  hipError_t launch_bwd_dq_hr_##NAME(const Params& p, int variant, hipStream_t st);           \
  hipError_t launch_bwd_dkdv_hr_##NAME(const Params& p, int variant, hipStream_t st);     \
  hipError_t launch_bwd_hr_##NAME(const Params& p, int variant, hipStream_t st);

RBF_DECLARE_HR_LAUNCHERS(bf16)
RBF_DECLARE_HR_LAUNCHERS(fp16)

#undef RBF_DECLARE_HR_LAUNCHERS

// Decode split geometry: waves per work-group (one 32-key block each per
// tile); fp32 tiles need twice the LDS, so fp32 runs half as many.
inline int decode_waves(int dtype_is_fp32) { return dtype_is_fp32 ? 2 : 4; }

}  // namespace rbf
