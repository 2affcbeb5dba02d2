// Decode: T new query tokens (1..32) of every (batch, head) against a KV
// cache, split over the key axis (flash-decoding).  No counterpart in the
// reference, which has no decode path.
//
// Query t of batch b sits at cache position len_b - T + t and attends to the
// keys [0, len_b - T + t] (the cache already holds the new tokens' K and V).
//
//   rbf_decode_split_kernel: grid (B*H, nsplit), W waves per work-group.  A
//     work-group streams its split's 32*W-key tiles of V through
//     double-buffered LDS; wave w owns the w-th 32-key block of every tile,
//     loads that block's K rows straight into registers (one tile ahead) and
//     keeps its own partial (m, l, O^T) for the T queries, with the online
//     max of the forward kernel.  Each wave writes its partial to the
//     workspace.
//   rbf_decode_merge_kernel: one wave per (b, h, t) combines the partials:
//     O = sum_p 2^(m_p - M) o_p / sum_p 2^(m_p - M) l_p, L = M + log2(l).
//     Non-softmax partials share m_p = c*0.5||q||^2 and simply add.
#pragma once

#include "rbf_attn_kernels.h"

namespace rbf {

struct DecodeParams {
  const void* q;
  const void* k;
  const void* v;
  void* o;
  int64_t sq[3], sk[3], sv[3], so[3];  // batch, head, token strides (elements)
  const int* lens;                     // per-batch cache lengths or nullptr
  float* lse;                          // (B,H,T) or nullptr
  float* ws;                           // partials
  int B, H, T, D, L;
  int nsplit, tps;  // splits per (b, h), tiles per split
  int W;            // waves per split work-group (partials per split)
  float gamma, c;
};

// Workspace layout (floats): o [B*H][P][T][DP], then m [B*H][P][T], then
// l [B*H][P][T], with P = nsplit * W partials per (b, h).
__host__ __device__ inline int64_t decode_ws_floats(int BH, int P, int T, int DP) {
  return (int64_t)BH * P * T * (DP + 2);
}

template <typename T, int DP, int W, bool SOFTMAX>
__global__ __launch_bounds__(64 * W) void rbf_decode_split_kernel(const DecodeParams p) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  constexpr int BN = 32 * W, NT = 64 * W, KS = DP / 16, ND = DP / 32;
  constexpr int LDT = BN + E::PAD;
  constexpr bool TR = sizeof(T) == 2;
  typedef TileLayout<T, BN, DP> TLy;
  // Only V goes through LDS (it is read transposed); each wave loads the K
  // rows of its own 32-key block straight into MFMA operand registers, one
  // tile ahead, and derives the key norms from them.
  __shared__ __attribute__((aligned(16))) T sVt[2][TR ? TLy::SIZE : DP * LDT];
  __shared__ __attribute__((aligned(16))) float sKn[W][32];

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int bh = blockIdx.x, split = blockIdx.y;
  const int b = bh / p.H, hh = bh - b * p.H;
  const int Tq = p.T, D = p.D;
  const float c = p.c;
  const int len = min(p.lens ? p.lens[b] : p.L, p.L);
  const int ntiles = (len + BN - 1) / BN;
  const int kt0 = split * p.tps, kt1 = min(kt0 + p.tps, ntiles);
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];

  const bool qvalid = n < Tq;
  const int jmax = len - Tq + n;  // last key query n sees
  frag qf[KS];
  float qn2 = 0.f;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    qf[t] = (qvalid && 16 * t + 8 * h < D) ? ld8<T>(Q + (int64_t)n * p.sq[2] + 16 * t + 8 * h) : zero_frag<T>();
    qn2 += sumsq8<T>(qf[t]);
  }
  qn2 = c * 0.5f * xhalf_sum(qn2);
  f32x16_t oacc[ND];
  float lsum = 0.f;  // this lane's share of the row sum (VALU; decode is HBM-bound)
#pragma unroll
  for (int d = 0; d < ND; ++d) oacc[d] = zero16();
  float m_run = SOFTMAX ? -__builtin_inff() : qn2;

  frag kA[KS];
  auto load_k = [&](int kt) {
    const int tok = kt * BN + 32 * wave + n;
    const bool ok = tok < len;
#pragma unroll
    for (int t = 0; t < KS; ++t)
      kA[t] = (ok && 16 * t + 8 * h < D) ? ld8<T>(K + (int64_t)tok * p.sk[2] + 16 * t + 8 * h) : zero_frag<T>();
  };
  TileFor<T, BN, DP, NT> tv;
  if (kt0 < kt1) {
    load_k(kt0);
    tv.load(V, p.sv[2], kt0 * BN, len, D, tid);
  }
  for (int kt = kt0; kt < kt1; ++kt) {
    const int buf = kt & 1;
    if constexpr (TR) TLy::store(tv, sVt[buf], tid);
    else tv.template store_trans<LDT>(sVt[buf], tid);
    __syncthreads();
    if (kt + 1 < kt1) tv.load(V, p.sv[2], (kt + 1) * BN, len, D, tid);
    const int k0 = kt * BN + 32 * wave;
    if (k0 >= len) continue;  // wave-uniform: the block lies past the cache
    // -0.5||k||^2 of this lane's key, transposed to the accumulator's rows
    // through the wave's own LDS slot (-inf past the cache length)
    float kn = 0.f;
#pragma unroll
    for (int t = 0; t < KS; ++t) kn += sumsq8<T>(kA[t]);
    kn = xhalf_sum(kn);
    if (h == 0) sKn[wave][n] = (k0 + n < len) ? -0.5f * kn : -__builtin_inff();
    f32x16_t s = ld_rows16(sKn[wave], h);
#pragma unroll
    for (int t = 0; t < KS; ++t) s = E::mma(kA[t], qf[t], s);
    if (kt + 1 < kt1) load_k(kt + 1);  // kA is free once the S products are issued
    frag vA[ND][2];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if constexpr (TR) vA[d][t] = TLy::tr(sVt[buf], 32 * wave + 16 * t, 32 * d, lane);
        else vA[d][t] = ld8<T>(sVt[buf] + (32 * d + n) * LDT + tchunk<BN>(32 * d + n, 32 * wave + 16 * t + 8 * h));
      }
    if (k0 + 31 > len - Tq) mask_key_rows(s, k0, h, jmax);  // the new tokens' causal corner
    if constexpr (SOFTMAX) {
      const float mt = xhalf_max(tree_max16(s)) * c;
      if (__any(mt > m_run + kTau)) {
        const float mnew = fmaxf(m_run, mt);
        const float alpha = (mnew == -__builtin_inff()) ? 1.f : fast_exp2(m_run - mnew);
#pragma unroll
        for (int d = 0; d < ND; ++d) oacc[d] *= alpha;
        lsum *= alpha;
        m_run = mnew;
      }
    }
    const float moff = (SOFTMAX && m_run == -__builtin_inff()) ? 0.f : m_run;
    frag pf[2];
    float pv[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      pv[i] = fast_exp2(fmaf(s[i], c, -moff));  // the row sum takes P unrounded, as the forward does
      pf[i >> 3][i & 7] = (T)pv[i];
    }
    if constexpr (SOFTMAX) lsum += tree_sum16(pv);
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int d = 0; d < ND; ++d) oacc[d] = E::mma(vA[d][t], pf[t], oacc[d]);
  }

  // partial of this wave
  const int P = p.nsplit * W;
  const int64_t pidx = (int64_t)bh * P + split * W + wave;
  if (!qvalid) return;
  float* wo = p.ws + (pidx * Tq + n) * DP;
#pragma unroll
  for (int d = 0; d < ND; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = 32 * d + 8 * g + 4 * h;
      f32x4_t v4 = {oacc[d][4 * g], oacc[d][4 * g + 1], oacc[d][4 * g + 2], oacc[d][4 * g + 3]};
      *reinterpret_cast<f32x4_t*>(wo + dd) = v4;
    }
  const float l = SOFTMAX ? xhalf_sum(lsum) : 0.f;
  if (h == 0) {
    float* wm = p.ws + (int64_t)p.B * p.H * P * Tq * DP;
    float* wl = wm + (int64_t)p.B * p.H * P * Tq;
    wm[pidx * Tq + n] = m_run;
    wl[pidx * Tq + n] = l;
  }
}

// Max / sum over the 64 lanes of a wave (every lane receives the result).
__device__ inline float wave_max64(float x) {
  x = xhalf_max(x);
#pragma unroll
  for (int o = 16; o >= 1; o >>= 1) x = fmaxf(x, __shfl_xor(x, o));
  return x;
}

template <typename T, int DP, bool SOFTMAX>
__global__ __launch_bounds__(64) void rbf_decode_merge_kernel(const DecodeParams p) {
  const int lane = threadIdx.x;
  const int idx = blockIdx.x;  // (b*H + h) * T + t
  const int Tq = p.T;
  const int bh = idx / Tq, t = idx - bh * Tq;
  const int b = bh / p.H, hh = bh - b * p.H;
  const int P = p.nsplit * p.W;
  const float* wo = p.ws + (int64_t)bh * P * Tq * DP;
  const float* wm = p.ws + (int64_t)p.B * p.H * P * Tq * DP + (int64_t)bh * P * Tq;
  const float* wl = wm + (int64_t)p.B * p.H * P * Tq;
  // M = max_p m_p, the lanes striding over the partials
  float M = -__builtin_inff();
  for (int q = lane; q < P; q += 64) M = fmaxf(M, wm[q * Tq + t]);
  M = wave_max64(M);
  // O and l: partials are read G at a time, so that their loads overlap
  constexpr int PER = (DP + 63) / 64, G = 8;
  float acc[PER] = {};
  float l = 0.f;
  for (int q0 = 0; q0 < P; q0 += G) {
    float w[G], lq[G], ov[G][PER];
#pragma unroll
    for (int j = 0; j < G; ++j) {
      const int q = q0 + j;
      const bool ok = q < P;
      const float mq = ok ? wm[q * Tq + t] : -__builtin_inff();
      if constexpr (SOFTMAX) w[j] = (mq == -__builtin_inff()) ? 0.f : fast_exp2(mq - M);
      else w[j] = ok ? 1.f : 0.f;
      lq[j] = (SOFTMAX && ok) ? wl[q * Tq + t] : 0.f;
#pragma unroll
      for (int e = 0; e < PER; ++e) {
        const int d = lane + 64 * e;
        ov[j][e] = (ok && d < DP) ? wo[((int64_t)q * Tq + t) * DP + d] : 0.f;
      }
    }
#pragma unroll
    for (int j = 0; j < G; ++j) {
      if constexpr (SOFTMAX) l = fmaf(w[j], lq[j], l);
#pragma unroll
      for (int e = 0; e < PER; ++e) acc[e] = fmaf(w[j], ov[j][e], acc[e]);
    }
  }
  const float inv = SOFTMAX ? (l > 0.f ? 1.f / l : 0.f) : 1.f;
  T* orow = reinterpret_cast<T*>(p.o) + b * p.so[0] + hh * p.so[1] + (int64_t)t * p.so[2];
#pragma unroll
  for (int e = 0; e < PER; ++e) {
    const int d = lane + 64 * e;
    if (d < p.D) orow[d] = (T)(acc[e] * inv);
  }
  if (SOFTMAX && p.lse && lane == 0) p.lse[(int64_t)bh * Tq + t] = M + __log2f(l);
}

}  // namespace rbf
