// Launchers of the head-resident kernels (16-bit elements, 32 < D <= 64,
// N <= 32 * kHrMaxBlocks).  Compiled once per 16-bit element type with
// -DRBF_ELEM_ID=0 (bf16) or 1 (fp16), in a translation unit of their own so
// that these kernels can take the instruction scheduler that suits them
// (the build compiles this unit with the ILP-maximising machine scheduler:
// 3-5 % faster on these kernels, slower on the long-sequence streaming ones).
#include "rbf_attn_hr_kernels.h"
#include "rbf_attn_launch.h"

#ifndef RBF_ELEM_ID
#error "RBF_ELEM_ID must be defined (0 bf16, 1 fp16)"
#endif

namespace rbf {
namespace {

#if RBF_ELEM_ID == 0
typedef __bf16 Elt;
#elif RBF_ELEM_ID == 1
typedef _Float16 Elt;
#else
#error "head-resident kernels are built for 16-bit elements only"
#endif

constexpr int DP = 64;
constexpr int NB = kHrMaxBlocks;

unsigned heads(const Params& p) { return (unsigned)((long long)p.B * p.H); }

template <bool SM, int W, bool POS>
hipError_t fwd_cfg(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((rbf_fwd_hr_kernel<Elt, DP, W, NB, SM, POS>), dim3(heads(p)), dim3(64 * W), 0, st, p);
  return hipGetLastError();
}

template <bool SM, bool POS>
hipError_t dq_cfg(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((rbf_bwd_dq_hr_kernel<Elt, DP, 8, NB, SM, POS>), dim3(heads(p)), dim3(64 * 8), 0, st, p);
  return hipGetLastError();
}

template <bool SM, bool POS>
hipError_t dkdv_cfg(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((rbf_bwd_dkdv_hr_kernel<Elt, DP, 8, NB, SM, POS>), dim3(heads(p)), dim3(64 * 8), 0, st, p);
  return hipGetLastError();
}

template <bool SM, bool POS>
hipError_t bwd_cfg(const Params& p, hipStream_t st) {
  hipLaunchKernelGGL((rbf_bwd_hr_kernel<Elt, DP, 8, NB, SM, POS>), dim3(heads(p)), dim3(64 * 8), 0, st, p);
  return hipGetLastError();
}

bool fits(const Params& p) { return p.D > 32 && p.D <= DP && p.nblk <= NB; }

}  // namespace

#if RBF_ELEM_ID == 0
#define RBF_NAME bf16
#else
#define RBF_NAME fp16
#endif
#define RBF_CAT2(a, b) a##b
#define RBF_CAT(a, b) RBF_CAT2(a, b)

// waves: 8 selects the 8-wave softmax forward (a tuning alternative, without
// a position term); any other value the default: softmax 16 waves,
// non-softmax 12, softmax with a position term 8.
hipError_t RBF_CAT(launch_fwd_hr_, RBF_NAME)(const Params& p, int variant, int waves, hipStream_t st) {
  if (!fits(p)) return hipErrorInvalidValue;
  const bool sm = variant == 0;
  // With a position term the softmax forward needs more registers than 12
  // waves leave (its next Q block and the term's fragments are in flight
  // together): 8 waves, measured as fast as 12 with spills.
  if (p.pos) return sm ? fwd_cfg<true, 8, true>(p, st) : fwd_cfg<false, 12, true>(p, st);
  if (waves == 8 && sm) return fwd_cfg<true, 8, false>(p, st);
  return sm ? fwd_cfg<true, 16, false>(p, st) : fwd_cfg<false, 12, false>(p, st);
}

hipError_t RBF_CAT(launch_bwd_dq_hr_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  if (!fits(p)) return hipErrorInvalidValue;
  const bool sm = variant == 0;
  if (p.pos) return sm ? dq_cfg<true, true>(p, st) : dq_cfg<false, true>(p, st);
  return sm ? dq_cfg<true, false>(p, st) : dq_cfg<false, false>(p, st);
}

hipError_t RBF_CAT(launch_bwd_dkdv_hr_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  if (!fits(p)) return hipErrorInvalidValue;
  const bool sm = variant == 0;
  if (p.pos) return sm ? dkdv_cfg<true, true>(p, st) : dkdv_cfg<false, true>(p, st);
  return sm ? dkdv_cfg<true, false>(p, st) : dkdv_cfg<false, false>(p, st);
}

// dQ then dK/dV of each head in one launch (rbf_bwd_hr_kernel).
hipError_t RBF_CAT(launch_bwd_hr_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  if (!fits(p)) return hipErrorInvalidValue;
  const bool sm = variant == 0;
  if (p.pos) return sm ? bwd_cfg<true, true>(p, st) : bwd_cfg<false, true>(p, st);
  return sm ? bwd_cfg<true, false>(p, st) : bwd_cfg<false, false>(p, st);
}

}  // namespace rbf
