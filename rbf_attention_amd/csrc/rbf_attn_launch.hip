// Launchers for one element type.  Compiled once per dtype with
// -DRBF_ELEM_ID=0 (bf16), 1 (fp16) or 2 (fp32), so the three instantiation
// sets build in parallel.
//
// Tile choices (tokens per LDS tile, waves per work-group) per head dim:
//   fwd:  4 waves x 32 queries; BN = 64 keys (32 for fp32).
//   dQ:   4 waves x 32 queries; BN = 64 keys for D <= 64, 32 for D = 128
//         (three LDS tiles: K, K^T, V), 32 for fp32.
//   dKdV: 4 waves x 32 keys; BM = 64 queries for D <= 64, 32 for D = 128
//         (four LDS tiles: Q, Q^T, dO, dO^T), 32 for fp32.
#include "rbf_attn_kernels.h"
#include "rbf_attn_launch.h"

#ifndef RBF_ELEM_ID
#error "RBF_ELEM_ID must be defined (0 bf16, 1 fp16, 2 fp32)"
#endif

namespace rbf {
namespace {

#if RBF_ELEM_ID == 0
typedef __bf16 Elt;
#elif RBF_ELEM_ID == 1
typedef _Float16 Elt;
#else
typedef float Elt;
#endif

constexpr int kWaves = 4;
constexpr bool kIsF32 = sizeof(Elt) == 4;

inline unsigned grid_of(const Params& p) {
  const int ngrp = (p.nblk + kWaves - 1) / kWaves;
  return (unsigned)((long long)p.B * p.H * ngrp);
}

template <int DP, bool SM>
hipError_t fwd(const Params& p, hipStream_t st) {
  constexpr int BN = kIsF32 ? 32 : 64;
  hipLaunchKernelGGL((rbf_fwd_kernel<Elt, DP, kWaves, BN, SM>), dim3(grid_of(p)), dim3(64 * kWaves), 0, st, p);
  return hipGetLastError();
}

template <int DP, bool SM>
hipError_t dq(const Params& p, hipStream_t st) {
  constexpr int BN = (kIsF32 || DP > 64) ? 32 : 64;
  hipLaunchKernelGGL((rbf_bwd_dq_kernel<Elt, DP, kWaves, BN, SM>), dim3(grid_of(p)), dim3(64 * kWaves), 0, st, p);
  return hipGetLastError();
}

template <int DP, bool SM>
hipError_t dkdv(const Params& p, hipStream_t st) {
  constexpr int BM = (kIsF32 || DP > 64) ? 32 : 64;
  hipLaunchKernelGGL((rbf_bwd_dkdv_kernel<Elt, DP, kWaves, BM, SM>), dim3(grid_of(p)), dim3(64 * kWaves), 0,
                     st, p);
  return hipGetLastError();
}

// Head dim D (a multiple of 8 in [8, 128]) runs on the kernel for the next
// padded width DP in {32, 64, 128}; features D..DP-1 are zero-filled.
#define RBF_DISPATCH(FN)                                               \
  do {                                                                 \
    const bool sm = (variant == 0);                                    \
    if (p.D <= 32) return sm ? FN<32, true>(p, st) : FN<32, false>(p, st); \
    if (p.D <= 64) return sm ? FN<64, true>(p, st) : FN<64, false>(p, st); \
    return sm ? FN<128, true>(p, st) : FN<128, false>(p, st);          \
  } while (0)

hipError_t fwd_any(const Params& p, int variant, hipStream_t st) { RBF_DISPATCH(fwd); }
hipError_t dq_any(const Params& p, int variant, hipStream_t st) { RBF_DISPATCH(dq); }
hipError_t dkdv_any(const Params& p, int variant, hipStream_t st) { RBF_DISPATCH(dkdv); }

#undef RBF_DISPATCH

}  // namespace

#if RBF_ELEM_ID == 0
#define RBF_NAME bf16
#elif RBF_ELEM_ID == 1
#define RBF_NAME fp16
#else
#define RBF_NAME fp32
#endif
#define RBF_CAT2(a, b) a##b
#define RBF_CAT(a, b) RBF_CAT2(a, b)

hipError_t RBF_CAT(launch_fwd_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return fwd_any(p, variant, st);
}
hipError_t RBF_CAT(launch_bwd_dq_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return dq_any(p, variant, st);
}
hipError_t RBF_CAT(launch_bwd_dkdv_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return dkdv_any(p, variant, st);
}

}  // namespace rbf
