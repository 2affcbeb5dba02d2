// Launchers for one element type.  Compiled once per dtype with
// -DRBF_ELEM_ID=0 (bf16), 1 (fp16) or 2 (fp32), so the three instantiation
// sets build in parallel (bf16 as two units, RBF_PART below); once more with
// -DRBF_ELEM_ID=2 -DRBF_WIDE for the fp32 kernels with 256 features
// (launch_*_wide_fp32).
//
// A kernel configuration is (W waves per work-group, blocks of 32 tokens per
// wave, LDS tile of streamed tokens).  Defaults per padded head dim DP are in
// the *_default() functions; for bf16 a few alternatives are also compiled and
// can be chosen with RBF_ATTN_FWD_CFG / RBF_ATTN_DQ_CFG / RBF_ATTN_DKDV_CFG
// (an index into the candidate lists below) for tuning sweeps.
#include <stdlib.h>

#include "rbf_attn_kernels.h"
#include "rbf_attn_launch.h"
#include "rbf_attn_staging.h"
#include "rbf_decode_kernels.h"

#ifndef RBF_ELEM_ID
#error "RBF_ELEM_ID must be defined (0 bf16, 1 fp16, 2 fp32)"
#endif
#if defined(RBF_WIDE) && RBF_ELEM_ID != 2
#error "RBF_WIDE builds the fp32 kernels with 256 features only"
#endif
// RBF_PART splits an element type's launchers over two units, so that the
// dQ kernels can be compiled with a machine-scheduler strategy of their own:
// 0 (default) every launcher; 1 all but dQ (the whole backward calls the
// other unit's launch_bwd_dq_*); 2 the dQ launcher only.  Each kernel is
// instantiated in one unit.
#ifndef RBF_PART
#define RBF_PART 0
#endif
#if RBF_PART != 0 && defined(RBF_WIDE)
#error "RBF_PART applies to the per-element-type units"
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

constexpr bool kIsF32 = sizeof(Elt) == 4;

int env_choice(const char* name) {
  const char* s = getenv(name);
  return s ? atoi(s) : -1;
}

int cu_count() {
  static const int n = [] {
    int dev = 0, v = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
      v = 256;
    return v > 0 ? v : 256;
  }();
  return n;
}

template <typename F>
int wgs_per_cu(F kernel, int threads) {
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, threads, 0) != hipSuccess || n < 1) n = 1;
  return n;
}

// Work-groups per head (Params::nbin) and the grid.  A head has `ngrp`
// groups of `blocks_per_wg` 32-token blocks.  When every group fits on the
// GPU at once each gets its own work-group; otherwise the groups are dealt
// to as many bins per head as keep all work-groups resident together
// (`wgs` per CU), so that the launch runs in one round of near-equal
// work-groups instead of a heavy round followed by a tail of light, short
// ones.  RBF_ATTN_NBIN=n forces n bins per head (0: one group per bin).
// Whether the binned kernels suit this problem: the streamed operands (K and
// V, or Q and dO) of all heads of an XCD stay within about its L2 size.  The
// bins of all heads run at once, so longer heads would stream them from HBM
// instead of sharing them in L2 head by head (the one-group form runs a
// head's groups together, heaviest first).
bool bins_fit(const Params& p) {
  const long long BH = (long long)p.B * p.H;
  return (BH + 7) / 8 * 2LL * p.N * p.D * (long long)sizeof(Elt) <= (16LL << 20);
}

unsigned set_bins(Params& p, int blocks_per_wg, int wgs, bool binned) {
  const int ngrp = (p.nblk + blocks_per_wg - 1) / blocks_per_wg;
  const long long BH = (long long)p.B * p.H;
  static const int forced = env_choice("RBF_ATTN_NBIN");
  long long nbin = ngrp;
  if (!binned) {
    // kernel compiled without the bin loop
  } else if (forced > 0) {
    nbin = forced < ngrp ? forced : ngrp;
  } else if (forced < 0 && BH > 0) {
    const long long slots = (long long)cu_count() * wgs;
    if (BH * ngrp > slots) nbin = slots / BH < 1 ? 1 : (slots / BH < ngrp ? slots / BH : ngrp);
  }
  p.nbin = (int)nbin;
  return (unsigned)(BH * nbin);
}

template <typename F>
hipError_t launch(F kernel, const Params& p, int blocks_per_wg, int threads, int wgs, bool binned, hipStream_t st) {
  Params q = p;
  const unsigned grid = set_bins(q, blocks_per_wg, wgs, binned);
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(threads), 0, st, q);
  return hipGetLastError();
}

// Head-resident launchers of this element type (rbf_attn_launch_hr.hip);
// never reached for fp32.
hipError_t hr_fwd(const Params& p, bool sm, int waves, hipStream_t st) {
#if RBF_ELEM_ID == 0
  return launch_fwd_hr_bf16(p, sm ? 0 : 1, waves, st);
#elif RBF_ELEM_ID == 1
  return launch_fwd_hr_fp16(p, sm ? 0 : 1, waves, st);
#else
  return hipErrorInvalidValue;
#endif
}

hipError_t hr_dq(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 0
  return launch_bwd_dq_hr_bf16(p, sm ? 0 : 1, st);
#elif RBF_ELEM_ID == 1
  return launch_bwd_dq_hr_fp16(p, sm ? 0 : 1, st);
#else
  return hipErrorInvalidValue;
#endif
}

hipError_t hr_dkdv(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 0
  return launch_bwd_dkdv_hr_bf16(p, sm ? 0 : 1, st);
#elif RBF_ELEM_ID == 1
  return launch_bwd_dkdv_hr_fp16(p, sm ? 0 : 1, st);
#else
  return hipErrorInvalidValue;
#endif
}

hipError_t hr_bwd(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 0
  return launch_bwd_hr_bf16(p, sm ? 0 : 1, st);
#elif RBF_ELEM_ID == 1
  return launch_bwd_hr_fp16(p, sm ? 0 : 1, st);
#else
  return hipErrorInvalidValue;
#endif
}

// Head-resident kernels (16-bit): the head's nblk blocks fit the kernel's LDS
// tiles (nb_max blocks) and there are at least as many heads as CUs, so one
// work-group per head fills the GPU.  RBF_ATTN_HR=0 disables them, =1 uses
// them whenever the head fits.
// RBF_ATTN_HR_KERNELS (bits: 1 fwd, 2 dQ, 4 dK/dV; default all) picks which
// kernels take the head-resident form.  The head-resident dK/dV measured
// faster than the binned streaming one at C2 on four MI355X boxes of five
// (41-45 against 45-46 us) and slower on one (50 against 46 us).
bool use_hr(const Params& p, int nb_max, int which) {
  static const int forced = env_choice("RBF_ATTN_HR");
  static const int env_mask = env_choice("RBF_ATTN_HR_KERNELS");
  const int mask = env_mask >= 0 ? env_mask : 7;
  if (kIsF32 || forced == 0 || p.nblk > nb_max || !(mask & which)) return false;
  if (forced > 0) return true;
  return (long long)p.B * p.H >= cu_count();
}
constexpr int kHrBlocks64 = kHrMaxBlocks;  // D <= 64: N <= 576

// LDS-DMA tile staging (16-bit, D = 64 or 128 filling the padded width DP:
// the streaming kernels' tiles go from global memory straight into LDS, three
// tiles in flight), when the rows of both operands a kernel stages are ones
// dma_rows_ok admits (rbf_attn_staging.h); otherwise the kernel is the
// register-staged one.  Each kernel checks only what it stages: the forward
// and dQ kernels stage K and V (and read Q and dO directly), the dK/dV kernels
// Q and dO (and read K and V directly); a forward's dO descriptor is unset.
// RBF_ATTN_DMA=0 keeps the register-staged kernels for every shape.
bool dma_pair_ok(const Params& p, int dp, int64_t stride_a, int64_t stride_b) {
  static const int forced = env_choice("RBF_ATTN_DMA");
  constexpr int64_t esz = sizeof(Elt);
  return !kIsF32 && forced != 0 && p.D == dp && dma_rows_ok(p.N, stride_a, p.D, esz) &&
         dma_rows_ok(p.N, stride_b, p.D, esz);
}
// K and V tiles: the forward and dQ kernels.
bool use_dma_kv(const Params& p, int dp) { return dma_pair_ok(p, dp, p.sk[2], p.sv[2]); }
// Q and dO tiles: the dK/dV kernels.
bool use_dma_qdo(const Params& p, int dp) { return dma_pair_ok(p, dp, p.sq[2], p.sdo[2]); }

template <int DP, bool SM, int W, int BN, bool BIN = false, bool DMA = false>
hipError_t fwd_cfg(const Params& p, hipStream_t st) {
  auto k = rbf_fwd_kernel<Elt, DP, W, BN, SM, BIN, (BIN && sizeof(Elt) == 2 && DP <= 64) ? 3 : 1, DMA>;
  static const int wgs = wgs_per_cu(k, 64 * W);
  return launch(k, p, W, 64 * W, wgs, BIN, st);
}

template <int DP, bool SM, int W, int QPW, int BN, bool EARLY = true, bool BIN = false, bool DMA = false>
hipError_t dq_cfg(const Params& p, hipStream_t st) {
  auto k = rbf_bwd_dq_kernel<Elt, DP, W, QPW, BN, SM, EARLY, BIN, DMA>;
  static const int wgs = wgs_per_cu(k, 64 * W);
  return launch(k, p, W * QPW, 64 * W, wgs, BIN, st);
}

template <int DP, bool SM, int W, int KPW, int BM, bool EARLY = true, bool PIPE = false, bool PRIO = false,
          bool BIN = false, bool DMA = false>
hipError_t dkdv_cfg(const Params& p, hipStream_t st) {
  auto k = rbf_bwd_dkdv_kernel<Elt, DP, W, KPW, BM, SM, EARLY, PIPE, PRIO, BIN, DMA>;
  static const int wgs = wgs_per_cu(k, 64 * W);
  return launch(k, p, W * KPW, 64 * W, wgs, BIN, st);
}

template <int DP, bool SM, int NP, int BM, bool SGB = false, bool BIN = false, bool DMA = false>
hipError_t dkdv_pair_cfg(const Params& p, hipStream_t st) {
  auto k = rbf_bwd_dkdv_pair_kernel<Elt, DP, NP, BM, SM, SGB, BIN, DMA>;
  static const int wgs = wgs_per_cu(k, 128 * NP);
  return launch(k, p, NP, 128 * NP, wgs, BIN, st);
}

// ---- defaults ------------------------------------------------------------
// Chosen from measured sweeps on MI355X (N = 516 and N = 8196, D = 64 / 128).
// Heads whose operands share L2 use the binned kernels (bins_fit,
// set_bins), others the one-group-per-work-group form.
// The forward switches to 8-wave work-groups over longer key tiles once a
// head has enough tokens to keep them busy.
constexpr int kLongSeq = 2048;

// With a position term (Params::pos) only the head-resident kernels apply;
// the C ABI admits it for 16-bit elements, 32 < D <= 64 and N <= 576.
template <int DP, bool SM>
hipError_t fwd_default(const Params& p, hipStream_t st) {
  if (p.pos) {
    if constexpr (!kIsF32 && DP == 64) {
      if (p.nblk <= kHrBlocks64) return hr_fwd(p, SM, 0, st);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (!kIsF32 && DP == 64) {
    if (use_hr(p, kHrBlocks64, 1)) return hr_fwd(p, SM, 0, st);
  }
  if constexpr (kIsF32) return fwd_cfg<DP, SM, 4, 32>(p, st);
  else if constexpr (DP == 256) {
    // 256 features: Q^T fragments and O^T accumulators of a 32-query block
    // take 192 registers, so one wave per SIMD (AGPRs hold the overflow, no
    // scratch); K and V tiles through registers into padded row-major LDS.
    return fwd_cfg<DP, SM, 4, 64>(p, st);
  } else if constexpr (DP <= 64) {
    // LDS-DMA: 4 waves over 64-key tiles at every length, one group per
    // work-group.  The bin loop re-primes the three-tile pipeline for each of
    // its groups with nothing to overlap it; separate work-groups overlap one
    // another's.  Measured against the binned forms (bf16 softmax fwd, us):
    // B63 H8 N1028 149 -> 131, B20 H8 N700 30.4 -> 27.9, B16 H8 N2052 118 ->
    // 108, B15 H8 N4100 382 -> 344, B4 H8 N8196 354 -> 346 (8 waves over
    // 128-key tiles: 374 and 358); B16 H8 N1028 37.8 -> 39.4.
    if (DP == 64 && use_dma_kv(p, DP)) return fwd_cfg<DP, SM, 4, 64, false, true>(p, st);
    // Register staging (padded head dims, or strides past the DMA range): one
    // group per work-group, 4 waves over 64-key tiles up to N = 8192.
    // Measured against the binned forms at D = 48 (bf16 softmax fwd, us): B63
    // H8 N1028 149 -> 117, B20 H8 N700 26.9 -> 23.5, B16 H8 N2052 111 -> 103;
    // at B4 H8 N8196 the binned 8-wave form stays ahead (360 against 366).
    if (p.N >= 4 * kLongSeq) return bins_fit(p) ? fwd_cfg<DP, SM, 8, 128, true>(p, st) : fwd_cfg<DP, SM, 8, 128>(p, st);
    return fwd_cfg<DP, SM, 4, 64>(p, st);
  } else {
    if (use_dma_kv(p, DP)) return bins_fit(p) ? fwd_cfg<DP, SM, 8, 64, true, true>(p, st) : fwd_cfg<DP, SM, 8, 64, false, true>(p, st);
    return bins_fit(p) ? fwd_cfg<DP, SM, 8, 64, true>(p, st) : fwd_cfg<DP, SM, 8, 64>(p, st);
  }
}

template <int DP, bool SM>
hipError_t dq_default(const Params& p, hipStream_t st) {
  if (p.pos) {
    if constexpr (!kIsF32 && DP == 64) {
      if (p.nblk <= kHrBlocks64) return hr_dq(p, SM, st);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (!kIsF32 && DP == 64) {
    if (use_hr(p, kHrBlocks64, 2)) return hr_dq(p, SM, st);
  }
  if constexpr (kIsF32) return dq_cfg<DP, SM, 4, 1, 32, DP != 256>(p, st);
  else if constexpr (DP == 256) {
    // 32-key tiles, K^T read next to the dQ MFMAs (one wave per SIMD)
    return dq_cfg<DP, SM, 4, 1, 32, false>(p, st);
  } else if constexpr (DP <= 64) {
    // (LDS-DMA on 64-key tiles: three 128-key tiles leave room for one
    // four-wave work-group per CU.)  One group per work-group, as for the
    // forward: against the binned form (bf16 softmax dQ, us) B63 H8 N1028 192
    // -> 168, B16 H8 N1028 45.0 -> 43.2, B20 H8 N700 33.5 -> 31.4, B16 H8
    // N2052 140 -> 126, B15 H8 N4100 491 -> 419, B4 H8 N8196 450 -> 414.
    if (DP == 64 && use_dma_kv(p, DP)) return dq_cfg<DP, SM, 4, 1, 64, true, false, true>(p, st);
    // register staging: one group per work-group (D = 48: 1.0-4.7 % faster
    // than binned at N = 700-8196)
    return dq_cfg<DP, SM, 4, 1, 128>(p, st);
  }
  else {
    // Short heads: 4-wave work-groups over 32-key register-staged tiles,
    // K^T read next to the dQ MFMAs.  Measured against the 8-wave LDS-DMA
    // form (bf16 softmax dQ): B63 H16 N516 302 -> 258 us, B8 H16 N516 36.5 ->
    // 33.2, B31 H16 N1028 363 -> 344; slower from N = 1500 (73 -> 80).
    if (p.N < 1200) return dq_cfg<DP, SM, 4, 1, 32, false>(p, st);
    if (use_dma_kv(p, DP))
      return bins_fit(p) ? dq_cfg<DP, SM, 8, 1, 64, true, true, true>(p, st) : dq_cfg<DP, SM, 8, 1, 64, true, false, true>(p, st);
    return bins_fit(p) ? dq_cfg<DP, SM, 8, 1, 32, true, true>(p, st) : dq_cfg<DP, SM, 8, 1, 32>(p, st);
  }
}

template <int DP, bool SM>
hipError_t dkdv_default(const Params& p, hipStream_t st) {
  if (p.pos) {
    if constexpr (!kIsF32 && DP == 64) {
      if (p.nblk <= kHrBlocks64) return hr_dkdv(p, SM, st);
    }
    return hipErrorInvalidValue;
  }
  if constexpr (!kIsF32 && DP == 64) {
    if (use_hr(p, kHrBlocks64, 4)) return hr_dkdv(p, SM, st);
  }
  if constexpr (kIsF32) return dkdv_cfg<DP, SM, 4, 1, 32, DP != 256>(p, st);
  else if constexpr (DP == 256) {
    // the paired kernel with two key blocks (four waves) per work-group over
    // 64-query register-staged tiles: each wave holds one of K, V and one
    // 32 x 256 accumulator
    return dkdv_pair_cfg<DP, SM, 2, 64>(p, st);
  } else if constexpr (DP <= 64) {
    // LDS-DMA from N = 4096 on: at N = 512-2048 the D = 64 dK/dV measured as
    // fast or slower with it (C4 188 -> 191 us), at N = 8192 faster (605 -> 589).
    // With it, one group per work-group (as the forward and dQ): 0.7-3.4 %
    // faster than the binned form at B15 H8 N4100, B4 H8 N8196, B2 H8 N16388.
    if (DP == 64 && p.N >= 2 * kLongSeq && use_dma_qdo(p, DP))
      return dkdv_cfg<DP, SM, 8, 1, 128, true, false, false, false, true>(p, st);
    // Register staging: one group per work-group, 4 waves below N = 4096 and 8
    // above.  Against the binned forms at D = 48 (bf16 softmax dK/dV, us): B63
    // H8 N1028 208 -> 200, B20 H8 N700 38.1 -> 35.9, B16 H8 N2052 169 -> 160,
    // B4 H8 N8196 536 -> 528.
    if (p.N >= 2 * kLongSeq) return dkdv_cfg<DP, SM, 8, 1, 128>(p, st);
    return dkdv_cfg<DP, SM, 4, 1, 128, false>(p, st);
  } else {
    // Four key blocks per work-group, one group each (no bin loop), at every
    // length; LDS-DMA from N = 1024.  Measured against the binned two-block
    // form (bf16 softmax dK/dV): B32 H8 N516 156 -> 114 us, B63 H16 N516 657
    // -> 470, B31 H16 N1028 891 -> 562 (DMA; 585 without), B4 H16 N1500 193
    // -> 114; at B2 H8 N300 18.5 against 18.8.
    if (p.N >= 1024 && use_dma_qdo(p, DP)) return dkdv_pair_cfg<DP, SM, 4, 64, true, false, true>(p, st);
    return dkdv_pair_cfg<DP, SM, 4, 64, true>(p, st);
  }
}

// ---- tuning candidates (bf16, 32 < D <= 64) ------------------------------
template <int DP, bool SM>
hipError_t fwd_any_cfg(const Params& p, hipStream_t st) {
  if (p.pos) return fwd_default<DP, SM>(p, st);  // tuning candidates take no position term
#if RBF_ELEM_ID == 0
  static const int choice = env_choice("RBF_ATTN_FWD_CFG");
  switch (choice) {
    case 0: return fwd_cfg<DP, SM, 4, 64>(p, st);
    case 1: return fwd_cfg<DP, SM, 8, 128>(p, st);
    case 2: return fwd_cfg<DP, SM, 8, 64>(p, st);
    case 3: return fwd_cfg<DP, SM, 4, 128>(p, st);
    case 4: return fwd_cfg<DP, SM, 2, 64>(p, st);
    case 5: return fwd_cfg<DP, SM, 4, 32>(p, st);
    case 6:
      if (use_dma_kv(p, DP)) return fwd_cfg<DP, SM, 4, 64, false, true>(p, st);
      break;
    case 7: return fwd_cfg<DP, SM, 4, 64, true>(p, st);
    case 8:
      if (use_dma_kv(p, DP)) return fwd_cfg<DP, SM, 8, DP == 64 ? 128 : 64, false, true>(p, st);
      break;
    case 10:
      if constexpr (DP == 64) { if (p.nblk <= kHrBlocks64) return hr_fwd(p, SM, 8, st); }
      break;
    case 11:
      if constexpr (DP == 64) { if (p.nblk <= kHrBlocks64) return hr_fwd(p, SM, 0, st); }
      break;
    default: break;
  }
#endif
  return fwd_default<DP, SM>(p, st);
}

template <int DP, bool SM>
hipError_t dq_any_cfg(const Params& p, hipStream_t st) {
  if (p.pos) return dq_default<DP, SM>(p, st);  // tuning candidates take no position term
#if RBF_ELEM_ID == 0
  if constexpr (DP == 128) {
    static const int choice = env_choice("RBF_ATTN_DQ_CFG");
    switch (choice) {
      case 8: return dq_cfg<DP, SM, 4, 1, 64>(p, st);
      case 9: return dq_cfg<DP, SM, 4, 1, 32, false>(p, st);
      case 10: return dq_cfg<DP, SM, 8, 1, 32>(p, st);
      case 11: return dq_cfg<DP, SM, 8, 1, 32, false>(p, st);
      case 14:
        if (use_dma_kv(p, DP)) return dq_cfg<DP, SM, 8, 1, 64, true, false, true>(p, st);
        break;
      default: break;
    }
  }
  if constexpr (DP <= 64) {
  static const int choice = env_choice("RBF_ATTN_DQ_CFG");
  switch (choice) {
    case 0: return dq_cfg<DP, SM, 4, 1, 64>(p, st);
    case 1: return dq_cfg<DP, SM, 2, 2, 64>(p, st);
    case 2: return dq_cfg<DP, SM, 4, 2, 64>(p, st);
    case 3: return dq_cfg<DP, SM, 4, 2, 32>(p, st);
    case 4: return dq_cfg<DP, SM, 4, 1, 32>(p, st);
    case 5: return dq_cfg<DP, SM, 8, 1, 64>(p, st);
    case 6: return dq_cfg<DP, SM, 4, 1, 64, false>(p, st);
    case 8: return dq_cfg<DP, SM, 4, 1, 128>(p, st);
    case 11: return dq_cfg<DP, SM, 8, 1, 64>(p, st);
    case 12:
      if (use_dma_kv(p, DP)) return dq_cfg<DP, SM, 4, 1, 64, true, false, true>(p, st);
      break;
    case 13: return dq_cfg<DP, SM, 4, 1, 64, true, true>(p, st);
    default: break;
  }
  }
#endif
  return dq_default<DP, SM>(p, st);
}

template <int DP, bool SM>
hipError_t dkdv_any_cfg(const Params& p, hipStream_t st) {
  if (p.pos) return dkdv_default<DP, SM>(p, st);  // tuning candidates take no position term
#if RBF_ELEM_ID == 0
  if constexpr (DP == 128) {
    static const int choice = env_choice("RBF_ATTN_DKDV_CFG");
    switch (choice) {
      case 7: return dkdv_cfg<DP, SM, 4, 1, 64, true, true>(p, st);
      case 8: return dkdv_cfg<DP, SM, 4, 1, 64, true, false>(p, st);
      case 9: return dkdv_cfg<DP, SM, 4, 1, 32, false, false>(p, st);
      case 10: return dkdv_cfg<DP, SM, 4, 1, 64, false, false>(p, st);
      case 12: return dkdv_cfg<DP, SM, 4, 1, 64, false, false, true>(p, st);
      case 20: return dkdv_pair_cfg<DP, SM, 4, 64>(p, st);
      case 21: return dkdv_pair_cfg<DP, SM, 4, 32>(p, st);
      case 22: return dkdv_pair_cfg<DP, SM, 2, 64>(p, st);
      case 23: return dkdv_pair_cfg<DP, SM, 2, 32>(p, st);
      case 25: return dkdv_pair_cfg<DP, SM, 4, 64, true>(p, st);
      case 26: return dkdv_pair_cfg<DP, SM, 2, 64, true>(p, st);
      case 27: return dkdv_pair_cfg<DP, SM, 4, 64, false, false, true>(p, st);
      case 28: return dkdv_pair_cfg<DP, SM, 4, 64, true, false, true>(p, st);
      default: break;
    }
  }
  if constexpr (DP <= 64) {
  static const int choice = env_choice("RBF_ATTN_DKDV_CFG");
  switch (choice) {
    case 0: return dkdv_cfg<DP, SM, 4, 1, 64>(p, st);
    case 1: return dkdv_cfg<DP, SM, 2, 2, 64>(p, st);
    case 2: return dkdv_cfg<DP, SM, 4, 2, 64>(p, st);
    case 3: return dkdv_cfg<DP, SM, 4, 2, 32>(p, st);
    case 4: return dkdv_cfg<DP, SM, 4, 1, 32>(p, st);
    case 5: return dkdv_cfg<DP, SM, 8, 1, 64>(p, st);
    case 6: return dkdv_cfg<DP, SM, 4, 1, 64, false>(p, st);
    case 7: return dkdv_cfg<DP, SM, 4, 1, 64, true, true>(p, st);
    case 8: return dkdv_cfg<DP, SM, 4, 1, 128, true, false>(p, st);
    case 10: return dkdv_cfg<DP, SM, 4, 1, 128, false, false>(p, st);
    case 11: return dkdv_cfg<DP, SM, 8, 1, 128, true, false>(p, st);
    case 12: return dkdv_cfg<DP, SM, 4, 1, 128, true, false, true>(p, st);
    case 20: return dkdv_pair_cfg<DP, SM, 4, 64>(p, st);
    case 21: return dkdv_pair_cfg<DP, SM, 4, 32>(p, st);
    case 22: return dkdv_pair_cfg<DP, SM, 4, 128>(p, st);
    case 23: return dkdv_pair_cfg<DP, SM, 2, 64>(p, st);
    case 24: return dkdv_pair_cfg<DP, SM, 2, 128>(p, st);
    default: break;
  }
  }
#endif
  return dkdv_default<DP, SM>(p, st);
}

template <int DP, bool SM>
hipError_t decode_dp(const DecodeParams& p, hipStream_t st) {
  constexpr int W = kIsF32 ? 2 : 4;
  if (p.W != W) return hipErrorInvalidValue;
  hipLaunchKernelGGL((rbf_decode_split_kernel<Elt, DP, W, SM>), dim3(p.B * p.H, p.nsplit), dim3(64 * W), 0, st, p);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((rbf_decode_merge_kernel<Elt, DP, SM>), dim3(p.B * p.H * p.T), dim3(64), 0, st, p);
  return hipGetLastError();
}

#ifndef RBF_WIDE
// 256 features.  The fp32 kernels of that width are built in a unit of their
// own (this file with RBF_WIDE): their register-resident Q/K/V/dO fragments
// and accumulators exceed the 512 registers of a lane, and with the VGPR form
// of the MFMA instructions forced (as for every other kernel) the compiler
// fails on them, so that unit leaves the register classes to the compiler.
#if RBF_PART != 2
hipError_t fwd_256(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 2
  return launch_fwd_wide_fp32(p, sm ? 0 : 1, st);
#else
  return sm ? fwd_default<256, true>(p, st) : fwd_default<256, false>(p, st);
#endif
}
#endif
#if RBF_PART != 1
hipError_t dq_256(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 2
  return launch_bwd_dq_wide_fp32(p, sm ? 0 : 1, st);
#else
  return sm ? dq_default<256, true>(p, st) : dq_default<256, false>(p, st);
#endif
}
#endif
#if RBF_PART != 2
hipError_t dkdv_256(const Params& p, bool sm, hipStream_t st) {
#if RBF_ELEM_ID == 2
  return launch_bwd_dkdv_wide_fp32(p, sm ? 0 : 1, st);
#else
  return sm ? dkdv_default<256, true>(p, st) : dkdv_default<256, false>(p, st);
#endif
}
#endif

// Head dim D (a multiple of 8 in [8, 256]) runs on the kernel for the next
// padded width DP in {32, 64, 128, 256}; features D..DP-1 are zero-filled (as
// the reference pads to BLOCK_DMODEL = next_pow2(D), rbf_attention.py:661).
// Only the softmax bf16 path with D in (32, 128] carries tuning candidates.
#define RBF_DISPATCH(DEF, ANY, W256)                                                \
  do {                                                                              \
    const bool sm = (variant == 0);                                                 \
    if (p.D <= 32) return sm ? DEF<32, true>(p, st) : DEF<32, false>(p, st);        \
    if (p.D <= 64) return sm ? ANY<64, true>(p, st) : DEF<64, false>(p, st);        \
    if (p.D <= 128) return sm ? ANY<128, true>(p, st) : DEF<128, false>(p, st);     \
    return W256(p, sm, st);                                                         \
  } while (0)

#if RBF_PART != 1
hipError_t dq_any(const Params& p, int variant, hipStream_t st) { RBF_DISPATCH(dq_default, dq_any_cfg, dq_256); }
#endif
#if RBF_PART != 2
hipError_t fwd_any(const Params& p, int variant, hipStream_t st) { RBF_DISPATCH(fwd_default, fwd_any_cfg, fwd_256); }
hipError_t dkdv_any(const Params& p, int variant, hipStream_t st) {
  RBF_DISPATCH(dkdv_default, dkdv_any_cfg, dkdv_256);
}

#undef RBF_DISPATCH

// Whole backward.  Where both backward kernels take the head-resident form,
// one launch runs a head's dQ pass and then its dK/dV pass
// (rbf_bwd_hr_kernel): one kernel boundary fewer, and the dK/dV pass's loads
// overlap the end of the dQ pass (C2: 85 against 89.6 us per step).
// RBF_ATTN_BWD_MERGED=0 keeps the two launches.
bool bwd_one_launch(const Params& p) {
  if constexpr (kIsF32) {
    return false;
  } else {
    static const int merged = env_choice("RBF_ATTN_BWD_MERGED");
    if (merged == 0 || p.D <= 32 || p.D > 64) return false;
    return p.pos ? p.nblk <= kHrBlocks64 : use_hr(p, kHrBlocks64, 2) && use_hr(p, kHrBlocks64, 4);
  }
}

hipError_t bwd_any(const Params& p, int variant, hipStream_t st) {
  if (bwd_one_launch(p)) return hr_bwd(p, variant == 0, st);
#if RBF_PART == 1
  static_assert(RBF_ELEM_ID == 0, "the split build is for bf16");
  hipError_t e = launch_bwd_dq_bf16(p, variant, st);
#else
  hipError_t e = dq_any(p, variant, st);
#endif
  if (e != hipSuccess) return e;
  return dkdv_any(p, variant, st);
}

hipError_t decode_any(const DecodeParams& p, int variant, hipStream_t st) {
  const bool sm = variant == 0;
  if (p.D <= 32) return sm ? decode_dp<32, true>(p, st) : decode_dp<32, false>(p, st);
  if (p.D <= 64) return sm ? decode_dp<64, true>(p, st) : decode_dp<64, false>(p, st);
  if (p.D <= 128) return sm ? decode_dp<128, true>(p, st) : decode_dp<128, false>(p, st);
#if RBF_ELEM_ID == 2
  return launch_decode_wide_fp32(p, variant, st);
#else
  return sm ? decode_dp<256, true>(p, st) : decode_dp<256, false>(p, st);
#endif
}
#endif  // RBF_PART != 2
#ifdef RBF_DISPATCH
#undef RBF_DISPATCH
#endif
#endif  // !RBF_WIDE

}  // namespace

#ifdef RBF_WIDE
// fp32 kernels with 256 features (see fwd_256).
hipError_t launch_fwd_wide_fp32(const Params& p, int variant, hipStream_t st) {
  return variant == 0 ? fwd_default<256, true>(p, st) : fwd_default<256, false>(p, st);
}
hipError_t launch_bwd_dq_wide_fp32(const Params& p, int variant, hipStream_t st) {
  return variant == 0 ? dq_default<256, true>(p, st) : dq_default<256, false>(p, st);
}
hipError_t launch_bwd_dkdv_wide_fp32(const Params& p, int variant, hipStream_t st) {
  return variant == 0 ? dkdv_default<256, true>(p, st) : dkdv_default<256, false>(p, st);
}
hipError_t launch_decode_wide_fp32(const DecodeParams& p, int variant, hipStream_t st) {
  return variant == 0 ? decode_dp<256, true>(p, st) : decode_dp<256, false>(p, st);
}
#else
#if RBF_ELEM_ID == 0
#define RBF_NAME bf16
#elif RBF_ELEM_ID == 1
#define RBF_NAME fp16
#else
#define RBF_NAME fp32
#endif
#define RBF_CAT2(a, b) a##b
#define RBF_CAT(a, b) RBF_CAT2(a, b)

#if RBF_PART != 1
hipError_t RBF_CAT(launch_bwd_dq_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return dq_any(p, variant, st);
}
#endif
#if RBF_PART != 2
hipError_t RBF_CAT(launch_fwd_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return fwd_any(p, variant, st);
}
hipError_t RBF_CAT(launch_bwd_dkdv_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return dkdv_any(p, variant, st);
}
hipError_t RBF_CAT(launch_bwd_, RBF_NAME)(const Params& p, int variant, hipStream_t st) {
  return bwd_any(p, variant, st);
}
int RBF_CAT(bwd_kernels_, RBF_NAME)(const Params& p) { return bwd_one_launch(p) ? 1 : 2; }
hipError_t RBF_CAT(launch_decode_, RBF_NAME)(const DecodeParams& p, int variant, hipStream_t st) {
  return decode_any(p, variant, st);
}
#endif  // RBF_PART != 2
#endif  // RBF_WIDE

}  // namespace rbf
