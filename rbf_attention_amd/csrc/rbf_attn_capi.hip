// C ABI of librbfattn.so: argument validation, parameter packing and dispatch
// to the per-dtype launchers.  Nothing here allocates device memory or
// synchronises; every error is detected before the first launch.
#include <math.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include <mutex>

#include <hip/hip_runtime.h>

#include "rbf_attn.h"
#include "rbf_attn_kernels.h"
#include "rbf_attn_launch.h"
#include "rbf_decode_kernels.h"

namespace {

thread_local char g_err[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

size_t elem_size(int dtype) { return dtype == RBF_ATTN_FP32 ? 4 : 2; }

int check_tensor(const char* name, const rbf_attn_tensor& t, size_t esz) {
  if (t.ptr == nullptr) return fail(RBF_ATTN_EINVAL_PTR, "%s: null pointer", name);
  if (reinterpret_cast<uintptr_t>(t.ptr) % 16 != 0)
    return fail(RBF_ATTN_EINVAL_STRIDE, "%s: base pointer not 16-byte aligned", name);
  const int64_t s[3] = {t.stride_b, t.stride_h, t.stride_n};
  for (int i = 0; i < 3; ++i)
    if ((s[i] * (int64_t)esz) % 16 != 0)
      return fail(RBF_ATTN_EINVAL_STRIDE, "%s: stride %d (%lld elements) is not a multiple of 16 bytes", name, i,
                  (long long)s[i]);
  return RBF_ATTN_OK;
}

int check_common(const rbf_attn_args* a) {
  g_err[0] = '\0';
  if (a == nullptr) return fail(RBF_ATTN_EINVAL_ARGS, "args is NULL");
  if (a->abi_version != RBF_ATTN_ABI_VERSION)
    return fail(RBF_ATTN_EINVAL_ARGS, "abi_version %d != library %d", a->abi_version, RBF_ATTN_ABI_VERSION);
  if (a->variant != RBF_ATTN_SOFTMAX && a->variant != RBF_ATTN_NON_SOFTMAX)
    return fail(RBF_ATTN_EINVAL_ARGS, "unknown variant %d", a->variant);
  if (a->dtype != RBF_ATTN_BF16 && a->dtype != RBF_ATTN_FP16 && a->dtype != RBF_ATTN_FP32)
    return fail(RBF_ATTN_EINVAL_DTYPE, "unknown dtype %d", a->dtype);
  if (a->B < 0 || a->H < 0 || a->N < 0)
    return fail(RBF_ATTN_EINVAL_SHAPE, "negative size B=%d H=%d N=%d", a->B, a->H, a->N);
  if (a->D < 8 || a->D > 256 || a->D % 8 != 0)
    return fail(RBF_ATTN_EINVAL_HEADDIM, "head dim D=%d unsupported (need 8 <= D <= 256, D %% 8 == 0)", a->D);
  if (a->causal != 0 && a->causal != 1) return fail(RBF_ATTN_EINVAL_ARGS, "causal must be 0 or 1");
  if (a->num_prefix < 0) return fail(RBF_ATTN_EINVAL_ARGS, "num_prefix must be >= 0");
  if (!(a->gamma > 0.f) || !isfinite(a->gamma))
    return fail(RBF_ATTN_EINVAL_ARGS, "gamma must be finite and > 0 (got %g)", (double)a->gamma);
  // Token indices and the grid are 32-bit.
  if (a->N > (1 << 30)) return fail(RBF_ATTN_EINVAL_SHAPE, "N=%d too large", a->N);
  const long long nblk = (a->N + 31) / 32;
  const long long grid = (long long)a->B * a->H * ((nblk + 3) / 4);
  if (grid > 0x7fffffffLL) return fail(RBF_ATTN_EINVAL_SHAPE, "grid of %lld work-groups too large", grid);
  if ((long long)a->B * a->H * a->N > (1LL << 40)) return fail(RBF_ATTN_EINVAL_SHAPE, "B*H*N too large");
  return RBF_ATTN_OK;
}

int check_f32(const char* name, const float* p) {
  if (p == nullptr) return fail(RBF_ATTN_EINVAL_PTR, "%s: null pointer", name);
  if (reinterpret_cast<uintptr_t>(p) % 4 != 0) return fail(RBF_ATTN_EINVAL_STRIDE, "%s: not 4-byte aligned", name);
  return RBF_ATTN_OK;
}

void copy_strides(int64_t dst[3], const rbf_attn_tensor& t) {
  dst[0] = t.stride_b;
  dst[1] = t.stride_h;
  dst[2] = t.stride_n;
}

rbf::Params make_params(const rbf_attn_args* a) {
  rbf::Params p = {};
  p.q = a->q.ptr;
  p.k = a->k.ptr;
  p.v = a->v.ptr;
  p.o = a->o.ptr;
  p.dout = a->dout.ptr;
  p.dq = a->dq.ptr;
  p.dk = a->dk.ptr;
  p.dv = a->dv.ptr;
  p.lse = a->lse;
  p.delta = a->delta;
  copy_strides(p.sq, a->q);
  copy_strides(p.sk, a->k);
  copy_strides(p.sv, a->v);
  copy_strides(p.so, a->o);
  copy_strides(p.sdo, a->dout);
  copy_strides(p.sdq, a->dq);
  copy_strides(p.sdk, a->dk);
  copy_strides(p.sdv, a->dv);
  p.B = a->B;
  p.H = a->H;
  p.N = a->N;
  p.D = a->D;
  p.causal = a->causal;
  p.num_prefix = a->num_prefix;
  p.gamma = a->gamma;
  p.c = (float)(2.0 * (double)a->gamma * 1.4426950408889634);
  const int rem = a->N % 32;
  p.org = rem == 0 ? 0 : rem - 32;
  p.nblk = (a->N - p.org) / 32;
  // Heaviest-group-first chunks of heads on one XCD: as many heads as have
  // 16 MB of streamed operands (K and V, or Q and dO) between them, rounded
  // up.  Measured on MI355X (bf16, sums of the three streaming kernels):
  // short heads want the whole XCD share in one chunk (no heavy group left
  // for the end of the launch); 4.2 MB heads (N = 8196, D = 128) ran 1.3 %
  // faster in chunks of 4 than of 1, and 6 or 8 were slower again; 8.4 MB
  // heads 0.6 % faster in chunks of 2 than of 1; for 2 MB heads chunks of 4
  // and 8 were within 0.5 %.
  const long long per_head = 2LL * a->N * a->D * (long long)elem_size(a->dtype);
  const long long fit = per_head > 0 ? ((16LL << 20) + per_head - 1) / per_head : 1;
  const long long per_xcd = ((long long)a->B * a->H) / 8;
  p.hchunk = (int)(fit < 1 ? 1 : (fit > per_xcd ? (per_xcd > 0 ? per_xcd : 1) : fit));
  // RBF_ATTN_HCHUNK overrides the chunk size (tuning sweeps).
  static const int forced = getenv("RBF_ATTN_HCHUNK") ? atoi(getenv("RBF_ATTN_HCHUNK")) : 0;
  if (forced > 0) p.hchunk = (int)(forced < per_xcd ? forced : (per_xcd > 0 ? per_xcd : 1));
  return p;
}

int launched(hipError_t e, const char* what) {
  if (e != hipSuccess) return fail(RBF_ATTN_ELAUNCH, "%s launch failed: %s", what, hipGetErrorString(e));
  return RBF_ATTN_OK;
}

// Decode: validation and split geometry (shared by the workspace query and
// the launch, so both agree on the workspace size).
struct DecodeGeom {
  int dp, waves, nsplit, tps;
  uint64_t ws_bytes;
};

int decode_check(const rbf_attn_decode_args* a, DecodeGeom* g) {
  g_err[0] = '\0';
  if (a == nullptr) return fail(RBF_ATTN_EINVAL_ARGS, "args is NULL");
  if (a->abi_version != RBF_ATTN_ABI_VERSION)
    return fail(RBF_ATTN_EINVAL_ARGS, "abi_version %d != library %d", a->abi_version, RBF_ATTN_ABI_VERSION);
  if (a->variant != RBF_ATTN_SOFTMAX && a->variant != RBF_ATTN_NON_SOFTMAX)
    return fail(RBF_ATTN_EINVAL_ARGS, "unknown variant %d", a->variant);
  if (a->dtype != RBF_ATTN_BF16 && a->dtype != RBF_ATTN_FP16 && a->dtype != RBF_ATTN_FP32)
    return fail(RBF_ATTN_EINVAL_DTYPE, "unknown dtype %d", a->dtype);
  if (a->B < 0 || a->H < 0) return fail(RBF_ATTN_EINVAL_SHAPE, "negative size B=%d H=%d", a->B, a->H);
  if (a->T < 1 || a->T > 32) return fail(RBF_ATTN_EINVAL_SHAPE, "T=%d query tokens unsupported (need 1..32)", a->T);
  if (a->L < a->T || a->L > (1 << 30)) return fail(RBF_ATTN_EINVAL_SHAPE, "cache length L=%d must be in [T, 2^30]", a->L);
  if (a->D < 8 || a->D > 256 || a->D % 8 != 0)
    return fail(RBF_ATTN_EINVAL_HEADDIM, "head dim D=%d unsupported (need 8 <= D <= 256, D %% 8 == 0)", a->D);
  if (!(a->gamma > 0.f) || !isfinite(a->gamma))
    return fail(RBF_ATTN_EINVAL_ARGS, "gamma must be finite and > 0 (got %g)", (double)a->gamma);
  const long long bh = (long long)a->B * a->H;
  if (bh > 0x7fffffffLL / 32) return fail(RBF_ATTN_EINVAL_SHAPE, "B*H=%lld too large", bh);
  g->dp = a->D <= 32 ? 32 : a->D <= 64 ? 64 : a->D <= 128 ? 128 : 256;
  // Split the key axis into one round of work-groups: as many as fit on the
  // 256 CUs at once (2 per CU for 128 features, whose split kernel holds 256
  // VGPRs and 68 KB of LDS; 1 for 256 features, whose V tiles take 135 KB;
  // 3 otherwise).  One round measured 7-20 % faster than two or more (no
  // tail).  RBF_ATTN_DECODE_WGS overrides (sweeps).
  g->waves = rbf::decode_waves(a->dtype == RBF_ATTN_FP32);
  const int tile = 32 * g->waves;
  const int ntiles = (a->L + tile - 1) / tile;
  static const long long forced = getenv("RBF_ATTN_DECODE_WGS") ? atoll(getenv("RBF_ATTN_DECODE_WGS")) : 0;
  const long long target =
      forced > 0 ? forced : (g->dp == 256 ? 256 : g->dp == 128 || a->dtype == RBF_ATTN_FP32 ? 512 : 768);
  long long ns = bh > 0 ? (target + bh - 1) / bh : 1;
  if (ns > ntiles) ns = ntiles;
  if (ns < 1) ns = 1;
  g->tps = (int)((ntiles + ns - 1) / ns);
  g->nsplit = (ntiles + g->tps - 1) / g->tps;
  if (g->nsplit > 65535) return fail(RBF_ATTN_EINVAL_SHAPE, "too many key splits");
  const long long P = (long long)g->nsplit * g->waves;
  g->ws_bytes = (uint64_t)rbf::decode_ws_floats((int)bh, (int)P, a->T, g->dp) * 4;
  return RBF_ATTN_OK;
}

}  // namespace

// Workspace of rbf_attn_bwd_noalloc: one fp32 entry per (b, h, n) row.  The
// host-side name `scratch` is only a stand-in for the symbol; the device
// address of each GPU's copy comes from hipGetSymbolAddress (scratch_ptr).
static __device__ __align__(256) float scratch[RBF_ATTN_NOALLOC_MAX_ROWS];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch_ptr[kMaxDevices] = {};

// Device address of `scratch` on the GPU that runs `stream`, looked up once
// per device with that device current.
int scratch_ptr(hipStream_t stream, float** out) {
  int dev = -1, cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return fail(RBF_ATTN_ELAUNCH, "hipGetDevice: %s", hipGetErrorString(e));
  dev = cur;
  if (stream != nullptr && (e = hipStreamGetDevice(stream, &dev)) != hipSuccess)
    return fail(RBF_ATTN_ELAUNCH, "hipStreamGetDevice: %s", hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(RBF_ATTN_ELAUNCH, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    // The first call on a device may come while the caller's stream is being
    // captured into a graph: the lookup (and any device switch) then runs in
    // relaxed capture mode on this thread, which admits calls that global or
    // thread-local capture would reject, and the caller's mode is restored.
    hipStreamCaptureMode mode = hipStreamCaptureModeRelaxed;
    const bool swapped = hipThreadExchangeStreamCaptureMode(&mode) == hipSuccess;
    if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) {
      if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
      return fail(RBF_ATTN_ELAUNCH, "hipSetDevice(%d): %s", dev, hipGetErrorString(e));
    }
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (dev != cur) (void)hipSetDevice(cur);
    if (swapped) (void)hipThreadExchangeStreamCaptureMode(&mode);
    if (e != hipSuccess || ptr == nullptr)
      return fail(RBF_ATTN_ELAUNCH, "hipGetSymbolAddress(scratch) on device %d: %s", dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = static_cast<float*>(ptr);
  }
  *out = g_scratch_ptr[dev];
  return RBF_ATTN_OK;
}

}  // namespace

extern "C" {

uint64_t rbf_attn_decode_workspace_size(const rbf_attn_decode_args* a) {
  DecodeGeom g;
  if (decode_check(a, &g)) return 0;
  return g.ws_bytes;
}

int rbf_attn_decode(const rbf_attn_decode_args* a, void* stream) {
  DecodeGeom g;
  int rc = decode_check(a, &g);
  if (rc) return rc;
  const size_t esz = elem_size(a->dtype);
  if ((rc = check_tensor("q", a->q, esz))) return rc;
  if ((rc = check_tensor("k", a->k, esz))) return rc;
  if ((rc = check_tensor("v", a->v, esz))) return rc;
  if ((rc = check_tensor("o", a->o, esz))) return rc;
  if (a->lse != nullptr && reinterpret_cast<uintptr_t>(a->lse) % 4 != 0)
    return fail(RBF_ATTN_EINVAL_STRIDE, "lse: not 4-byte aligned");
  if (a->lens != nullptr && reinterpret_cast<uintptr_t>(a->lens) % 4 != 0)
    return fail(RBF_ATTN_EINVAL_STRIDE, "lens: not 4-byte aligned");
  if ((long long)a->B * a->H == 0) return RBF_ATTN_OK;
  if (a->workspace == nullptr) return fail(RBF_ATTN_EINVAL_PTR, "workspace: null pointer");
  if (reinterpret_cast<uintptr_t>(a->workspace) % 16 != 0)
    return fail(RBF_ATTN_EINVAL_STRIDE, "workspace: not 16-byte aligned");
  if (a->workspace_bytes < g.ws_bytes)
    return fail(RBF_ATTN_EINVAL_ARGS, "workspace of %llu bytes, %llu needed", (unsigned long long)a->workspace_bytes,
                (unsigned long long)g.ws_bytes);
  rbf::DecodeParams p = {};
  p.q = a->q.ptr;
  p.k = a->k.ptr;
  p.v = a->v.ptr;
  p.o = a->o.ptr;
  copy_strides(p.sq, a->q);
  copy_strides(p.sk, a->k);
  copy_strides(p.sv, a->v);
  copy_strides(p.so, a->o);
  p.lens = a->lens;
  p.lse = a->variant == RBF_ATTN_SOFTMAX ? a->lse : nullptr;
  p.ws = reinterpret_cast<float*>(a->workspace);
  p.B = a->B;
  p.H = a->H;
  p.T = a->T;
  p.D = a->D;
  p.L = a->L;
  p.nsplit = g.nsplit;
  p.tps = g.tps;
  p.W = g.waves;
  p.gamma = a->gamma;
  p.c = (float)(2.0 * (double)a->gamma * 1.4426950408889634);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (a->dtype) {
    case RBF_ATTN_BF16: e = rbf::launch_decode_bf16(p, a->variant, st); break;
    case RBF_ATTN_FP16: e = rbf::launch_decode_fp16(p, a->variant, st); break;
    default: e = rbf::launch_decode_fp32(p, a->variant, st); break;
  }
  return launched(e, "decode");
}


int rbf_attn_abi_version(void) { return RBF_ATTN_ABI_VERSION; }

const char* rbf_attn_last_error(void) { return g_err; }

// Checks a position term for rbf_attn_{fwd,bwd}_pos and stores it in p.
static int set_pos(const rbf_attn_args* a, const rbf_attn_pos_term* pos, rbf::Params& p) {
  int rc;
  if (pos == nullptr) return fail(RBF_ATTN_EINVAL_PTR, "pos: null descriptor");
  if (pos->batch != 1 && pos->batch != a->B)
    return fail(RBF_ATTN_EINVAL_SHAPE, "pos: batch extent %d must be 1 or B=%d", pos->batch, a->B);
  if (pos->batch == 1 && a->B > 1 && pos->t.stride_b != 0)
    return fail(RBF_ATTN_EINVAL_STRIDE,
                "pos: a term shared by the batch (batch=1) must have stride_b = 0 (got %lld): it is read at every b",
                (long long)pos->t.stride_b);
  if ((rc = check_tensor("pos", pos->t, elem_size(a->dtype)))) return rc;
  if (rbf_attn_pos_supported(a) != 1)
    return fail(RBF_ATTN_EUNSUPPORTED, "position term fused only for bf16/fp16, 32 < D <= 64, N <= 576 (D=%d N=%d)", a->D,
                a->N);
  p.pos = pos->t.ptr;
  copy_strides(p.spos, pos->t);
  return RBF_ATTN_OK;
}

int rbf_attn_pos_supported(const rbf_attn_args* a) {
  int rc = check_common(a);
  if (rc) return rc;
  return (a->dtype != RBF_ATTN_FP32 && a->D > 32 && a->D <= 64 && a->N <= 576) ? 1 : 0;
}

static int fwd_impl(const rbf_attn_args* a, const rbf_attn_pos_term* pos, void* stream) {
  int rc = check_common(a);
  if (rc) return rc;
  const size_t esz = elem_size(a->dtype);
  if ((rc = check_tensor("q", a->q, esz))) return rc;
  if ((rc = check_tensor("k", a->k, esz))) return rc;
  if ((rc = check_tensor("v", a->v, esz))) return rc;
  if ((rc = check_tensor("o", a->o, esz))) return rc;
  if (a->variant == RBF_ATTN_SOFTMAX && (rc = check_f32("lse", a->lse))) return rc;
  if ((long long)a->B * a->H * a->N == 0) return RBF_ATTN_OK;
  rbf::Params p = make_params(a);
  if (pos && (rc = set_pos(a, pos, p))) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipError_t e;
  switch (a->dtype) {
    case RBF_ATTN_BF16: e = rbf::launch_fwd_bf16(p, a->variant, st); break;
    case RBF_ATTN_FP16: e = rbf::launch_fwd_fp16(p, a->variant, st); break;
    default: e = rbf::launch_fwd_fp32(p, a->variant, st); break;
  }
  return launched(e, "forward");
}

int rbf_attn_fwd(const rbf_attn_args* a, void* stream) { return fwd_impl(a, nullptr, stream); }
int rbf_attn_fwd_pos(const rbf_attn_args* a, const rbf_attn_pos_term* pos, void* stream) {
  if (pos == nullptr) {
    g_err[0] = '\0';
    return fail(RBF_ATTN_EINVAL_PTR, "pos: null descriptor");
  }
  return fwd_impl(a, pos, stream);
}

// noalloc: the per-query workspace (softmax Delta, non-softmax norm offsets)
// is the library's scratch array instead of args->delta / args->lse.
static int bwd_impl(const rbf_attn_args* a, const rbf_attn_pos_term* pos, void* stream, int stage,
                    bool noalloc = false) {
  int rc = check_common(a);
  if (rc) return rc;
  if (stage < 0 || stage > 2) return fail(RBF_ATTN_EINVAL_ARGS, "unknown backward stage %d", stage);
  const long long rows = (long long)a->B * a->H * a->N;
  if (noalloc && rows > RBF_ATTN_NOALLOC_MAX_ROWS)
    return fail(RBF_ATTN_EINVAL_SHAPE, "B*H*N = %lld rows exceed the no-allocation workspace of %d rows", rows,
                RBF_ATTN_NOALLOC_MAX_ROWS);
  const size_t esz = elem_size(a->dtype);
  const bool softmax = a->variant == RBF_ATTN_SOFTMAX;
  if ((rc = check_tensor("q", a->q, esz))) return rc;
  if ((rc = check_tensor("k", a->k, esz))) return rc;
  if ((rc = check_tensor("v", a->v, esz))) return rc;
  if ((rc = check_tensor("dout", a->dout, esz))) return rc;
  if ((rc = check_tensor("dq", a->dq, esz))) return rc;
  if ((rc = check_tensor("dk", a->dk, esz))) return rc;
  if ((rc = check_tensor("dv", a->dv, esz))) return rc;
  if ((softmax || !noalloc) && (rc = check_f32("lse", a->lse))) return rc;
  if (softmax) {
    if ((rc = check_tensor("o", a->o, esz))) return rc;
    if (!noalloc && (rc = check_f32("delta", a->delta))) return rc;
  }
  if (rows == 0) return RBF_ATTN_OK;
  rbf::Params p = make_params(a);
  if (pos && (rc = set_pos(a, pos, p))) return rc;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (noalloc) {
    float* ws = nullptr;
    if ((rc = scratch_ptr(st, &ws))) return rc;
    if (softmax)
      p.delta = ws;
    else
      p.lse = ws;
  }
  hipError_t e;
  if (stage == 0) {
    switch (a->dtype) {
      case RBF_ATTN_BF16: e = rbf::launch_bwd_bf16(p, a->variant, st); break;
      case RBF_ATTN_FP16: e = rbf::launch_bwd_fp16(p, a->variant, st); break;
      default: e = rbf::launch_bwd_fp32(p, a->variant, st); break;
    }
    return launched(e, "backward");
  }
  if (stage == 1) {
    switch (a->dtype) {
      case RBF_ATTN_BF16: e = rbf::launch_bwd_dq_bf16(p, a->variant, st); break;
      case RBF_ATTN_FP16: e = rbf::launch_bwd_dq_fp16(p, a->variant, st); break;
      default: e = rbf::launch_bwd_dq_fp32(p, a->variant, st); break;
    }
    if ((rc = launched(e, "backward dQ"))) return rc;
  }
  if (stage == 2) {
    switch (a->dtype) {
      case RBF_ATTN_BF16: e = rbf::launch_bwd_dkdv_bf16(p, a->variant, st); break;
      case RBF_ATTN_FP16: e = rbf::launch_bwd_dkdv_fp16(p, a->variant, st); break;
      default: e = rbf::launch_bwd_dkdv_fp32(p, a->variant, st); break;
    }
    if ((rc = launched(e, "backward dK/dV"))) return rc;
  }
  return RBF_ATTN_OK;
}

int rbf_attn_bwd(const rbf_attn_args* a, void* stream) { return bwd_impl(a, nullptr, stream, 0); }

int rbf_attn_bwd_noalloc(const rbf_attn_args* a, void* stream) { return bwd_impl(a, nullptr, stream, 0, true); }

int rbf_attn_bwd_pos(const rbf_attn_args* a, const rbf_attn_pos_term* pos, void* stream) {
  if (pos == nullptr) {
    g_err[0] = '\0';
    return fail(RBF_ATTN_EINVAL_PTR, "pos: null descriptor");
  }
  return bwd_impl(a, pos, stream, 0);
}

int rbf_attn_bwd_kernels(const rbf_attn_args* a, const rbf_attn_pos_term* pos) {
  int rc = check_common(a);
  if (rc) return rc;
  if ((long long)a->B * a->H * a->N == 0) return 0;
  rbf::Params p = make_params(a);
  if (pos && (rc = set_pos(a, pos, p))) return rc;
  switch (a->dtype) {
    case RBF_ATTN_BF16: return rbf::bwd_kernels_bf16(p);
    case RBF_ATTN_FP16: return rbf::bwd_kernels_fp16(p);
    default: return rbf::bwd_kernels_fp32(p);
  }
}

int rbf_attn_bwd_stage(const rbf_attn_args* a, void* stream, int stage) {
  if (stage != 1 && stage != 2) {
    g_err[0] = '\0';
    return fail(RBF_ATTN_EINVAL_ARGS, "unknown backward stage %d", stage);
  }
  return bwd_impl(a, nullptr, stream, stage);
}

}  // extern "C"
