// Head-resident kernels for short sequences (16-bit elements).
//
// When a head's streamed operands fit in LDS (two (N, D) tensors and their
// per-token scalars within ~150 KB: N <= 576 for D <= 64) and there are at
// least as many heads as CUs, one work-group per head loads them once, then
// every wave runs its own 32-token blocks against the resident tiles with no
// further barriers.  Compared with the streaming kernels this removes the
// per-tile barrier and the per-tile global-load latency from every wave's
// chain, and the launch is a single round of equal work-groups.
//
// Waves take their blocks in snake order over the causal weights (heaviest
// first), so each wave -- and each SIMD -- gets a near-equal share of the
// head's 32x32 block pairs.
//
// POS: a position term P (Params::pos) is added to Q and K as they are read
// (q + P and k + P, each sum rounded to the element type, as the separate
// elementwise adds of the model would store them): the SuSiE position
// embedding of the reference model (rbf_attention.py:1666-1688) fused into
// the loads.
#pragma once

#include "rbf_attn_kernels.h"

namespace rbf {

// A position term is added where the value is consumed, not where it is
// loaded: a sum taken right after the loads makes them wait there, which
// turns the prefetch of the next block into a synchronous load.
template <typename T, bool POS>
__device__ inline void add_pos(typename Elem<T>::frag* x, const typename Elem<T>::frag* pos, int n) {
  if constexpr (POS)
    for (int i = 0; i < n; ++i) x[i] = add8<T>(x[i], pos[i]);
}

// Chunk-major index of unit u: 16 consecutive units cover 4 tokens x 4
// chunks, i.e. 64 contiguous bytes of each of 4 rows in global memory.
template <int DP>
__device__ inline void hr_unit(int u, int& row, int& ch) {
  constexpr int CG = DP / 32;  // groups of 4 chunks per row
  const int rest = u >> 4;
  ch = 4 * (rest % CG) + (u & 3);
  row = 4 * (rest / CG) + ((u >> 2) & 3);
}

// Two head tiles in flight: fetch() requests rows [0, rows) -- tokens
// org + row -- of two (N, D) slices into registers (tokens outside [0, N) and
// features >= D read as zero; when ADD, the rows of addA, row stride asa, too),
// put() stores them into chunk-major LDS tiles of ROWS rows, the position term
// added to the first slice.  Every chunk of a thread is requested before the
// first is stored, and between the two calls the loads stay outstanding, so a
// caller can wait at a barrier meanwhile.
template <typename T, int ROWS, int DP, int NT, bool ADD>
struct HrTiles2 {
  typedef typename Elem<T>::frag frag;
  static constexpr int PB = (ROWS * (DP / 8) + NT - 1) / NT;
  frag ra[PB], rb[PB], rp[ADD ? PB : 1];

  __device__ inline void fetch(const T* A, int64_t sa, const T* B, int64_t sb, int rows, int org, int N, int D, int tid,
                               const T* addA, int64_t asa) {
    const int units = rows * (DP / 8);
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      const int u = tid + j * NT;
      int row, ch;
      hr_unit<DP>(u, row, ch);
      const int tok = org + row;
      const bool ok = u < units && tok >= 0 && tok < N && ch * 8 < D;
      ra[j] = ok ? ld8<T>(A + (int64_t)tok * sa + ch * 8) : zero_frag<T>();
      rb[j] = ok ? ld8<T>(B + (int64_t)tok * sb + ch * 8) : zero_frag<T>();
      if constexpr (ADD) rp[j] = ok ? ld8<T>(addA + (int64_t)tok * asa + ch * 8) : zero_frag<T>();
    }
  }

  __device__ inline void put(T* sA, T* sB, int tid) {
    typedef CLayout<ROWS> L;
    add_pos<T, ADD>(ra, rp, PB);
    // Units past the tile store into the padding after chunk column 0
    // instead of branching around the store.
#pragma unroll
    for (int j = 0; j < PB; ++j) {
      const int u = tid + j * NT;
      int row, ch;
      hr_unit<DP>(u, row, ch);
      const int o = u < ROWS * (DP / 8) ? L::off(row, 8 * ch) : L::off(ROWS, 0);
      st8<T>(sA + o, ra[j]);
      st8<T>(sB + o, rb[j]);
    }
  }
};

// fetch() then put(): both tiles of a head loaded into LDS.
template <typename T, int ROWS, int DP, int NT, bool ADD>
__device__ inline void hr_load2(const T* A, int64_t sa, T* sA, const T* B, int64_t sb, T* sB, int rows, int org,
                                int N, int D, int tid, const T* addA, int64_t asa) {
  HrTiles2<T, ROWS, DP, NT, ADD> t;
  t.fetch(A, sa, B, sb, rows, org, N, D, tid, addA, asa);
  t.put(sA, sB, tid);
}

// nrm[row] = -0.5 ||row||^2 of a resident chunk-major tile (fp32, from the
// element-type values), -inf for padding rows (tokens outside [0, N)).
template <typename T, int ROWS, int DP, int NT>
__device__ inline void hr_neg_halfnorms(const T* sA, float* nrm, int rows, int org, int N, int tid) {
  typedef CLayout<ROWS> L;
  for (int r = tid; r < rows; r += NT) {
    float s = 0.f;
#pragma unroll
    for (int ch = 0; ch < DP / 8; ++ch) s += sumsq8<T>(ld8<T>(sA + L::off(r, 8 * ch)));
    const int tok = org + r;
    nrm[r] = (tok >= 0 && tok < N) ? -0.5f * s : -__builtin_inff();
  }
}

// Stores one token's 32 features of an accumulator tile (C layout: lane
// (n, h) holds features fbase + 8(i/4) + 4h + i%4, i = 0..15, of token n) as
// whole 16-byte chunks: lanes n and n + 32 trade halves of their 4-feature
// groups (v_permlane32_swap), after which lane half h writes chunks 2j + h.
// Every lane must call it (the swap reads the partner lane); `on` predicates
// only the stores.  8-byte stores of the same data measured 2.3x the
// compulsory HBM write bytes for the dK/dV tiles of the head-resident kernel.
template <typename T>
__device__ inline void store_tile_chunks(T* row, const float* v, int fbase, int h, int D, bool on) {
  uint32_t w[8];
#pragma unroll
  for (int g = 0; g < 4; ++g)
#pragma unroll
    for (int m = 0; m < 2; ++m) w[2 * g + m] = bits16<T>((T)v[4 * g + 2 * m]) | (bits16<T>((T)v[4 * g + 2 * m + 1]) << 16);
#pragma unroll
  for (int q = 0; q < 4; q += 2) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const auto r = __builtin_amdgcn_permlane32_swap(w[2 * q + m], w[2 * q + 2 + m], false, false);
      w[2 * q + m] = r[0];
      w[2 * q + 2 + m] = r[1];
    }
    const int f = fbase + 8 * (q + h);
    if (on && f < D) {
      const u32x4_t c = {w[2 * q], w[2 * q + 1], w[2 * q + 2], w[2 * q + 3]};
      *reinterpret_cast<u32x4_t*>(row + f) = c;
    }
  }
}

// The lane's token features in the accumulator layout of a 32x32 tile whose
// rows are features (lane (n, h) of tile d holds features 32d + 8g + 4h + e,
// g, e = 0..3), taken from B-operand fragments of the same token (f[t] of
// lane (n, h) = features 16t + 8h .. 16t + 8h + 7).  Lane halves trade
// dwords with v_permlane32_swap: out[d][g][e] for features 32d + 8g + 4h + e.
// Every lane must call it.
template <typename T, int KS>
__device__ inline void frag_cfeat(const typename Elem<T>::frag* f, float (*out)[4][4]) {
  typedef typename Elem<T>::raw raw;
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    const raw w = __builtin_bit_cast(raw, f[t]);
    // (w0, w2) -> features 4h + {0, 1} of groups g = 2(t%2) and 2(t%2) + 1;
    // (w1, w3) -> features 4h + {2, 3}
    const auto a = __builtin_amdgcn_permlane32_swap(w[0], w[2], false, false);
    const auto b = __builtin_amdgcn_permlane32_swap(w[1], w[3], false, false);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float* o = out[t >> 1][2 * (t & 1) + s];
      const uint32_t lo = a[s], hi = b[s];
      o[0] = (float)__builtin_bit_cast(T, (uint16_t)(lo & 0xffffu));
      o[1] = (float)__builtin_bit_cast(T, (uint16_t)(lo >> 16));
      o[2] = (float)__builtin_bit_cast(T, (uint16_t)(hi & 0xffffu));
      o[3] = (float)__builtin_bit_cast(T, (uint16_t)(hi >> 16));
    }
  }
}

// Block index of the k-th block (k = 0, 1, ...) of `wave` out of W, or -1:
// blocks ranked heaviest first (rank 0 = block nblk-1 when `reverse`, i.e.
// when the weight rises with the block index), dealt in snake order.
__device__ inline int hr_block(int k, int wave, int W, int nblk, bool reverse) {
  const int rank = k * W + ((k & 1) ? W - 1 - wave : wave);
  if (rank >= nblk) return -1;
  return reverse ? nblk - 1 - rank : rank;
}

// ---------------------------------------------------------------------------
// Forward, head-resident.  The work-group loads the head's K and V (and
// -0.5||k||^2) into LDS once; wave w then computes the output of its query
// blocks as rbf_fwd_group does per block (static softmax bound; O normalised
// by the rounded P's fp32 sum, L from the unrounded P's; online max for fp16,
// or as a per-block rerun when a row's sum leaves [2^-60, 2^100]), reading K
// rows and transposed V from the resident tiles.
//
// With up to 12 waves and no running max (the static softmax bound,
// non-softmax) the key loop is software pipelined: iteration kb issues the S
// MFMAs of block kb+1 (K fragments and norms read one block earlier) next to
// the exponentials of block kb, so the MFMA and VALU work of one wave overlap.
// Only the causal diagonal block needs a mask; it is peeled off the loop.  The
// softmax forward without a position term runs 16 waves (4 per SIMD) with the
// plain loop instead: its registers fit 128 per lane only without the
// pipeline's second S accumulator and norm rows, and the other waves on the
// SIMD do the overlapping (C2 forward 22.9 -> 22.4 us against 12 pipelined
// waves; fp16 24.1 -> 23.5).
// ---------------------------------------------------------------------------
template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS = false>
__global__ __launch_bounds__(64 * W) void rbf_fwd_hr_kernel(const Params p) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  static_assert(sizeof(T) == 2, "head-resident tiles are chunk-major 16-bit tiles");
  constexpr int ROWS = 32 * NB, NT = 64 * W, KS = DP / 16, ND = DP / 32;
  typedef CLayout<ROWS> L;
  __shared__ __attribute__((aligned(16))) T sK[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) T sV[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) float sKn[ROWS];

  if (p.nblk > NB) return;  // the host launches this kernel only for heads that fit
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const int bh = blockIdx.x;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* Pos = POS ? reinterpret_cast<const T*>(p.pos) + b * p.spos[0] + hh * p.spos[1] : nullptr;
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  T* O = reinterpret_cast<T*>(const_cast<void*>(p.o)) + b * p.so[0] + hh * p.so[1];

  // Q fragments of a query block (and the position term's, summed with
  // them where they are consumed)
  auto load_q = [&](int qb, frag* qf, frag* pf) {
    const int qtok = org + 32 * qb + n;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool ok = qb >= 0 && qtok >= 0 && 16 * t + 8 * h < D;
      qf[t] = ok ? ld8<T>(Q + (int64_t)qtok * p.sq[2] + 16 * t + 8 * h) : zero_frag<T>();
      if constexpr (POS) pf[t] = ok ? ld8<T>(Pos + (int64_t)qtok * p.spos[2] + 16 * t + 8 * h) : zero_frag<T>();
    }
  };
  // The first query block's Q fragments are requested before the K/V load.
  frag qf[KS], pq[POS ? KS : 1];
  int qb = hr_block(0, wave, W, nblk, causal);
  load_q(qb, qf, pq);

  hr_load2<T, ROWS, DP, NT, POS>(K, p.sk[2], sK, V, p.sv[2], sV, 32 * nblk, org, N, D, tid, Pos, p.spos[2]);
  __syncthreads();
  hr_neg_halfnorms<T, ROWS, DP, NT>(sK, sKn, 32 * nblk, org, N, tid);
  __syncthreads();
  add_pos<T, POS>(qf, pq, KS);

  auto load_k = [&](int kb, frag* kA) {
#pragma unroll
    for (int t = 0; t < KS; ++t) kA[t] = ld8<T>(sK + L::off(32 * kb + n, 16 * t + 8 * h));
  };
  auto load_vt = [&](int kb, frag (*vA)[2]) {
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int t = 0; t < 2; ++t) vA[d][t] = ld_trc<T, ROWS>(sV, 32 * kb + 16 * t, 32 * d, lane);
  };
  auto s_mma = [&](const frag* kA, f32x16_t s) {
#pragma unroll
    for (int t = 0; t < KS; ++t) s = E::mma(kA[t], qf[t], s);
    return s;
  };

  const frag ones = ones_frag<T>();
  for (int k = 0; qb >= 0; ++k) {
    // the next block's Q fragments are requested before this block's work
    const int qb_next = hr_block(k + 1, wave, W, nblk, causal);
    frag qf_next[KS], pq_next[POS ? KS : 1];
    load_q(qb_next, qf_next, pq_next);
    const int q0 = org + 32 * qb, qtok = q0 + n;
    const bool qvalid = qtok >= 0;
    const int jmax = last_key(qtok, N, causal, npre);
    float qn2 = 0.f;
#pragma unroll
    for (int t = 0; t < KS; ++t) qn2 += sumsq8<T>(qf[t]);
    qn2 = c * 0.5f * xhalf_sum(qn2);
    // key blocks [0, kend) hold every key some query of the block sees
    const int kend = causal ? min(nblk, ((max(q0 + 31, npre - 1) - org) >> 5) + 1) : nblk;

    f32x16_t oacc[ND];
    // this lane's share (16 of each block's 32 keys) of the sums of the
    // rounded P (normalises O) and of the unrounded P (gives L)
    float lrnd, lrow;
    float m_run;
    // P = exp2(c S - m) for one block, then O^T += V^T P^T and l_r += sum P
    // (P rounded to the element type) and l += sum P (fp32, unrounded)
    auto pv = [&](const f32x16_t& s, float moff, frag (*vA)[2]) {
      frag pf[2];
      float pe[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        pe[i] = fast_exp2(fmaf(s[i], c, -moff));
        pf[i >> 3][i & 7] = (T)pe[i];
      }
      if constexpr (SOFTMAX) {
        lrow += tree_sum16(pe);
        lrnd += dot8<T>(pf[0], ones) + dot8<T>(pf[1], ones);
      }
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int d = 0; d < ND; ++d) oacc[d] = E::mma(vA[d][t], pf[t], oacc[d]);
    };
    auto init = [&](float m0) {
#pragma unroll
      for (int d = 0; d < ND; ++d) oacc[d] = zero16();
      lrnd = 0.f;
      lrow = 0.f;
      m_run = m0;
    };

    // Online max with lazy rescaling (fp16 softmax, or the rerun of a block
    // whose row sums left the static bound's range).
    auto run_safe = [&]() {
      init(SOFTMAX ? -__builtin_inff() : qn2);
      for (int kb = 0; kb < kend; ++kb) {
        const int k0 = org + 32 * kb;
        frag kA[KS], vA[ND][2];
        load_k(kb, kA);
        f32x16_t s = s_mma(kA, ld_rows16(sKn + 32 * kb, h));
        load_vt(kb, vA);
        if (!blk_nomask(q0, k0, causal, npre)) mask_key_rows(s, k0, h, jmax);
        if constexpr (SOFTMAX) {
          const float mt = xhalf_max(tree_max16(s)) * c;
          if (__any(mt > m_run + kTau)) {
            const float mnew = fmaxf(m_run, mt);
            const float alpha = (mnew == -__builtin_inff()) ? 1.f : fast_exp2(m_run - mnew);
#pragma unroll
            for (int d = 0; d < ND; ++d) oacc[d] *= alpha;
            lrnd *= alpha;
            lrow *= alpha;
            m_run = mnew;
          }
        }
        pv(s, m_run == -__builtin_inff() ? 0.f : m_run, vA);
      }
    };

    // Fixed offset (static bound or non-softmax), software pipelined.  With
    // num_prefix == 0 the blocks before the last need no mask (causal: the
    // last block is the diagonal one; not causal: padding keys are -inf
    // through their norms).
    auto run_fixed = [&]() {
      init(SOFTMAX ? qn2 - kBoundMargin : qn2);
      const float moff = m_run;
      const int last = kend - 1;
      frag kA[KS], vA[ND][2];
      load_k(0, kA);
      f32x16_t s = s_mma(kA, ld_rows16(sKn, h));
      load_k(min(1, last), kA);
      f32x16_t nrm = ld_rows16(sKn + 32 * min(1, last), h);
      for (int kb = 0; kb < last; ++kb) {
        load_vt(kb, vA);
        const f32x16_t sn = s_mma(kA, nrm);  // S of block kb + 1
        const int k2 = min(kb + 2, last);
        load_k(k2, kA);
        nrm = ld_rows16(sKn + 32 * k2, h);
        pv(s, moff, vA);
        s = sn;
      }
      load_vt(last, vA);
      if (causal) mask_key_rows(s, org + 32 * last, h, jmax);
      pv(s, moff, vA);
    };

    constexpr bool STATIC = SOFTMAX && !std::is_same<T, _Float16>::value;
    constexpr bool PIPE = W <= 12;  // registers for the pipelined key loop
    if (PIPE && !(SOFTMAX && !STATIC) && npre == 0) {
      run_fixed();
    } else if constexpr (SOFTMAX && !STATIC) {
      run_safe();
    } else {
      // fixed offset with a num_prefix mask, or 16 waves: the plain loop at
      // the fixed offset
      init(SOFTMAX ? qn2 - kBoundMargin : qn2);
      for (int kb = 0; kb < kend; ++kb) {
        const int k0 = org + 32 * kb;
        frag kA[KS], vA[ND][2];
        load_k(kb, kA);
        f32x16_t s = s_mma(kA, ld_rows16(sKn + 32 * kb, h));
        load_vt(kb, vA);
        if (!blk_nomask(q0, k0, causal, npre)) mask_key_rows(s, k0, h, jmax);
        pv(s, m_run, vA);
      }
    }
    if constexpr (STATIC) {
      const float l = xhalf_sum(lrow);
      const bool bad = qvalid && !(l >= kSumLow && l <= kSumHigh);
      if (__any(bad)) run_safe();
    }

    const float lsum = SOFTMAX ? xhalf_sum(lrow) : 1.f;
    const float inv = SOFTMAX ? 1.f / xhalf_sum(lrnd) : 1.f;
    if (qvalid) {
      T* orow = O + (int64_t)qtok * p.so[2];
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dd = 32 * d + 8 * g + 4 * h;
          if (dd < D) {
            float v4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = oacc[d][4 * g + e] * inv;
            st4f<T>(orow + dd, v4);
          }
        }
      if (SOFTMAX && h == 0) p.lse[(int64_t)bh * N + qtok] = m_run + __log2f(lsum);
    }
    qb = qb_next;
#pragma unroll
    for (int t = 0; t < KS; ++t) qf[t] = qf_next[t];
    add_pos<T, POS>(qf, pq_next, KS);
  }
}

// ---------------------------------------------------------------------------
// dK / dV, head-resident.  The work-group holds the head's Q and dO
// (chunk-major) and the per-query offsets -L/c (non-softmax: -0.5||q||^2)
// and -Delta in LDS; wave w takes key blocks in snake order over the causal
// weights (key block j is seen by the query blocks from j on, so block 0 is
// the heaviest) and, per key block, runs the query blocks that see it exactly
// as rbf_bwd_dkdv_group does per 32x32 block:
//   S = Q K^T (init -L/c), P = exp2(c S - c 0.5||k||^2), dP = dO V^T (init
//   -Delta), dS = P dP, dV^T += dO^T P, dK^T += Q^T dS, colsum += dS,
// with K and V in registers and no barrier after the load.
// ---------------------------------------------------------------------------
// XFER: runs after a dQ pass of the same head in the same LDS.  That pass
// left the per-query term it forms (softmax: sDel = -Delta; non-softmax:
// sOff = -off / c) in LDS, so it is neither read from global memory nor
// staged here, and the tiles are stored only after a barrier.
template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS, bool XFER = false>
__device__ __forceinline__ void bwd_dkdv_hr_body(const Params& p, T* sQ, T* sD, float* sOff, float* sDel) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  static_assert(sizeof(T) == 2, "head-resident tiles are chunk-major 16-bit tiles");
  constexpr int ROWS = 32 * NB, NT = 64 * W, KS = DP / 16, ND = DP / 32;
  typedef CLayout<ROWS> L;

  if (p.nblk > NB) return;  // the host launches this kernel only for heads that fit
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const float inv_c = 1.f / c;
  const int bh = blockIdx.x;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* Pos = POS ? reinterpret_cast<const T*>(p.pos) + b * p.spos[0] + hh * p.spos[1] : nullptr;
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  const T* dO = reinterpret_cast<const T*>(p.dout) + b * p.sdo[0] + hh * p.sdo[1];
  T* dK = reinterpret_cast<T*>(p.dk) + b * p.sdk[0] + hh * p.sdk[1];
  T* dV = reinterpret_cast<T*>(p.dv) + b * p.sdv[0] + hh * p.sdv[1];
  const float* offg = p.lse + (int64_t)bh * N;
  const float* delg = SOFTMAX ? p.delta + (int64_t)bh * N : nullptr;

  // K and V of one key block, straight to registers (their norm is taken
  // where the block is first used, so the loads stay in flight until then).
  frag kf[KS], vf[KS], pk[POS ? KS : 1];
  auto load_kv = [&](int kb) {
    const int ktok = org + 32 * kb + n;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool ok = kb >= 0 && ktok >= 0 && 16 * t + 8 * h < D;
      kf[t] = ok ? ld8<T>(K + (int64_t)ktok * p.sk[2] + 16 * t + 8 * h) : zero_frag<T>();
      vf[t] = ok ? ld8<T>(V + (int64_t)ktok * p.sv[2] + 16 * t + 8 * h) : zero_frag<T>();
      if constexpr (POS) pk[t] = ok ? ld8<T>(Pos + (int64_t)ktok * p.spos[2] + 16 * t + 8 * h) : zero_frag<T>();
    }
  };
  int kb = hr_block(0, wave, W, nblk, false);
  if constexpr (XFER && !POS) {
    // After a dQ pass, sQ / sD still hold the head's K and V (tokens outside
    // [0, N) and features past D as zeros) until the barrier below: the first
    // key block comes from there instead of from global memory (C2 backward
    // 56.15 -> 55.4 us).  With a position term that pass's K tile holds k + P,
    // so the block is loaded as raw K here.
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      kf[t] = kb >= 0 ? ld8<T>(sQ + L::off(32 * kb + n, 16 * t + 8 * h)) : zero_frag<T>();
      vf[t] = kb >= 0 ? ld8<T>(sD + L::off(32 * kb + n, 16 * t + 8 * h)) : zero_frag<T>();
    }
  } else {
    load_kv(kb);
  }

  // L and Delta of the rows this thread stages are requested with the Q / dO
  // rows, so the load phase waits for one round trip.
  constexpr int RPT = (ROWS + NT - 1) / NT;
  float offv[RPT], delv[RPT];
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = tid + j * NT, tok = org + r;
    const bool ok = r < 32 * nblk && tok >= 0 && tok < N;
    offv[j] = (ok && !(XFER && !SOFTMAX)) ? offg[tok] : 0.f;
    delv[j] = (SOFTMAX && !XFER && ok) ? delg[tok] : 0.f;
  }
  {
    HrTiles2<T, ROWS, DP, NT, POS> tiles;
    tiles.fetch(Q, p.sq[2], dO, p.sdo[2], 32 * nblk, org, N, D, tid, Pos, p.spos[2]);
    // After a dQ pass in the same LDS: wait until every wave is done with its
    // tiles (the loads above stay in flight meanwhile).
    if constexpr (XFER) __syncthreads();
    tiles.put(sQ, sD, tid);
  }
#pragma unroll
  for (int j = 0; j < RPT; ++j) {
    const int r = tid + j * NT, tok = org + r;
    const bool ok = tok >= 0 && tok < N;
    if (r < 32 * nblk) {
      if (!(XFER && !SOFTMAX)) sOff[r] = ok ? -offv[j] * inv_c : -__builtin_inff();  // padding queries: P = 0
      if (!(XFER && SOFTMAX)) sDel[r] = ok ? -delv[j] : 0.f;
    }
  }
  __syncthreads();

  const float g2 = 2.f * p.gamma;
  for (int k = 0; kb >= 0; ++k) {
    const int k0 = org + 32 * kb, ktok = k0 + n;
    add_pos<T, POS>(kf, pk, KS);
    float nckn;  // -c 0.5 ||k||^2
    {
      float ss = 0.f;
#pragma unroll
      for (int t = 0; t < KS; ++t) ss += sumsq8<T>(kf[t]);
      nckn = -c * 0.5f * xhalf_sum(ss);
    }
    const int ilo = first_query(ktok, causal, npre);
    // query blocks [qb0, nblk) hold every query that sees some key of the block
    const int qlo = causal ? (max(k0, 0) < npre ? 0 : max(k0, 0)) : 0;
    const int qb0 = max(0, (qlo - org) >> 5);

    f32x16_t dkacc[ND], dvacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      dkacc[d] = zero16();
      dvacc[d] = zero16();
    }
    float csum = 0.f;
    // Q and dO row fragments of the next query block are read while this
    // block's products and exponentials run.
    frag qA[KS], dA[KS];
    auto load_rows = [&](int qb) {
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        qA[t] = ld8<T>(sQ + L::off(32 * qb + n, 16 * t + 8 * h));
        dA[t] = ld8<T>(sD + L::off(32 * qb + n, 16 * t + 8 * h));
      }
    };
    load_rows(qb0);
    for (int qb = qb0; qb < nblk; ++qb) {
      const int q0 = org + 32 * qb;
      f32x16_t s = ld_rows16(sOff + 32 * qb, h);
      f32x16_t dp = SOFTMAX ? ld_rows16(sDel + 32 * qb, h) : zero16();
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        s = E::mma(qA[t], kf[t], s);
        dp = E::mma(dA[t], vf[t], dp);
      }
      load_rows(min(qb + 1, nblk - 1));
      // dO^T and Q^T fragments are read while the S / dP MFMAs run.
      frag dtA[ND][2], qtA[ND][2];
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          dtA[d][t] = ld_trc<T, ROWS>(sD, 32 * qb + 16 * t, 32 * d, lane);
          qtA[d][t] = ld_trc<T, ROWS>(sQ, 32 * qb + 16 * t, 32 * d, lane);
        }
      if (!blk_nomask(q0, k0, causal, npre)) mask_query_rows(s, q0, h, ilo);
      frag pf[2], sf[2];
      float ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const float pv = fast_exp2(fmaf(s[i], c, nckn));
        ds[i] = pv * dp[i];
        pf[i >> 3][i & 7] = (T)pv;
        sf[i >> 3][i & 7] = (T)ds[i];
      }
      csum += tree_sum16(ds);
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          dvacc[d] = E::mma(dtA[d][t], pf[t], dvacc[d]);
          dkacc[d] = E::mma(qtA[d][t], sf[t], dkacc[d]);
        }
    }

    const float cs = xhalf_sum(csum);
    // The block's K (with the position term) in the dK accumulator layout,
    // for the key-norm term; then the next block's K and V are requested
    // before this block's results are written.
    float kc[ND][4][4];
    frag_cfeat<T, KS>(kf, kc);
    kb = hr_block(k + 1, wave, W, nblk, false);
    if (kb >= 0) load_kv(kb);
    const bool on = ktok >= 0;
    T* dkrow = dK + (int64_t)ktok * p.sdk[2];
    T* dvrow = dV + (int64_t)ktok * p.sdv[2];
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      float a[16];
#pragma unroll
      for (int g = 0; g < 4; ++g)
#pragma unroll
        for (int e = 0; e < 4; ++e) a[4 * g + e] = g2 * (dkacc[d][4 * g + e] - cs * kc[d][g][e]);
      float bv[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) bv[i] = dvacc[d][i];
      store_tile_chunks<T>(dkrow, a, 32 * d, h, D, on);
      store_tile_chunks<T>(dvrow, bv, 32 * d, h, D, on);
    }
  }
}

// ---------------------------------------------------------------------------
// dQ (and Delta), head-resident.  The work-group holds the head's K, V and
// -0.5||k||^2 in LDS; wave w takes query blocks in snake order over the
// causal weights and, per query block, computes Delta = rowsum(O dO) (or the
// non-softmax norm offset) as rbf_bwd_dq_group does, then runs the key
// blocks the block sees:
//   S^T = K Q^T (init -0.5||k||^2), P = exp2(c S^T - L), dP^T = V dO^T
//   (init -Delta), dS = P dP^T, dQ^T += K^T dS^T,
// with the next key block's K and V rows read one block ahead and no
// barrier after the load.
// ---------------------------------------------------------------------------
// sX (optional): the per-query term the dK/dV pass needs is also stored there,
// in that pass's LDS form (softmax: -Delta; non-softmax: -off / c, -inf for
// padding queries).
template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS>
__device__ __forceinline__ void bwd_dq_hr_body(const Params& p, T* sK, T* sV, float* sKn, float* sX = nullptr) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  static_assert(sizeof(T) == 2, "head-resident tiles are chunk-major 16-bit tiles");
  constexpr int ROWS = 32 * NB, NT = 64 * W, KS = DP / 16, ND = DP / 32;
  typedef CLayout<ROWS> L;

  if (p.nblk > NB) return;  // the host launches this kernel only for heads that fit
  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const int bh = blockIdx.x;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* Pos = POS ? reinterpret_cast<const T*>(p.pos) + b * p.spos[0] + hh * p.spos[1] : nullptr;
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  const T* Og = reinterpret_cast<const T*>(p.o) + b * p.so[0] + hh * p.so[1];
  const T* dO = reinterpret_cast<const T*>(p.dout) + b * p.sdo[0] + hh * p.sdo[1];
  T* dQ = reinterpret_cast<T*>(p.dq) + b * p.sdq[0] + hh * p.sdq[1];

  // Q and dO fragments of one query block, straight to registers; the next
  // block's are requested before this block's dQ is written.  (The block's O
  // rows and L are read where Delta is formed: requested together with Q and
  // dO they cost registers and measured 1.5 us slower at C2.)
  frag qf[KS], df[KS], pq[POS ? KS : 1];
  auto load_qd = [&](int qb) {
    const int qtok = org + 32 * qb + n;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool ok = qb >= 0 && qtok >= 0 && 16 * t + 8 * h < D;
      qf[t] = ok ? ld8<T>(Q + (int64_t)qtok * p.sq[2] + 16 * t + 8 * h) : zero_frag<T>();
      df[t] = ok ? ld8<T>(dO + (int64_t)qtok * p.sdo[2] + 16 * t + 8 * h) : zero_frag<T>();
      if constexpr (POS) pq[t] = ok ? ld8<T>(Pos + (int64_t)qtok * p.spos[2] + 16 * t + 8 * h) : zero_frag<T>();
    }
  };
  int qb = hr_block(0, wave, W, nblk, causal);
  load_qd(qb);

  hr_load2<T, ROWS, DP, NT, POS>(K, p.sk[2], sK, V, p.sv[2], sV, 32 * nblk, org, N, D, tid, Pos, p.spos[2]);
  __syncthreads();
  hr_neg_halfnorms<T, ROWS, DP, NT>(sK, sKn, 32 * nblk, org, N, tid);
  __syncthreads();

  const float g2 = 2.f * p.gamma;
  for (int k = 0; qb >= 0; ++k) {
    add_pos<T, POS>(qf, pq, KS);
    const int q0 = org + 32 * qb, qtok = q0 + n;
    const bool qvalid = qtok >= 0;
    const int jmax = last_key(qtok, N, causal, npre);
    float off, dlt = 0.f;
    if constexpr (SOFTMAX) {
      float sdot = 0.f;
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const bool ok = qvalid && 16 * t + 8 * h < D;
        const frag o1 = ok ? ld8<T>(Og + (int64_t)qtok * p.so[2] + 16 * t + 8 * h) : zero_frag<T>();
        sdot += dot8<T>(o1, df[t]);
      }
      dlt = xhalf_sum(sdot);
      off = qvalid ? p.lse[(int64_t)bh * N + qtok] : 0.f;
      if (qvalid && h == 0) p.delta[(int64_t)bh * N + qtok] = dlt;
    } else {
      float ss = 0.f;
#pragma unroll
      for (int t = 0; t < KS; ++t) ss += sumsq8<T>(qf[t]);
      off = c * 0.5f * xhalf_sum(ss);
      if (qvalid && h == 0) p.lse[(int64_t)bh * N + qtok] = off;
    }
    if (sX != nullptr && h == 0)
      sX[32 * qb + n] = SOFTMAX ? -dlt : (qvalid ? -off * (1.f / c) : -__builtin_inff());
    const f32x16_t ndel = SOFTMAX ? splat16(-dlt) : zero16();  // +0: the MFMA's inline constant
    // key blocks [0, kend) hold every key some query of the block sees
    const int kend = causal ? min(nblk, ((max(q0 + 31, npre - 1) - org) >> 5) + 1) : nblk;

    f32x16_t dqacc[ND];
#pragma unroll
    for (int d = 0; d < ND; ++d) dqacc[d] = zero16();
    float rsum = 0.f;
    frag kA[KS], vA[KS];
    auto load_rows = [&](int kb) {
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        kA[t] = ld8<T>(sK + L::off(32 * kb + n, 16 * t + 8 * h));
        vA[t] = ld8<T>(sV + L::off(32 * kb + n, 16 * t + 8 * h));
      }
    };
    load_rows(0);
    for (int kb = 0; kb < kend; ++kb) {
      const int k0 = org + 32 * kb;
      f32x16_t s = ld_rows16(sKn + 32 * kb, h);
      f32x16_t dp = ndel;
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        s = E::mma(kA[t], qf[t], s);
        dp = E::mma(vA[t], df[t], dp);
      }
      load_rows(min(kb + 1, kend - 1));
      // K^T fragments are read while the S / dP MFMAs and the softmax run.
      frag ktA[ND][2];
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) ktA[d][t] = ld_trc<T, ROWS>(sK, 32 * kb + 16 * t, 32 * d, lane);
      if (!blk_nomask(q0, k0, causal, npre)) mask_key_rows(s, k0, h, jmax);
      frag sf[2];
      float ds[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        ds[i] = fast_exp2(fmaf(s[i], c, -off)) * dp[i];
        sf[i >> 3][i & 7] = (T)ds[i];
      }
      if constexpr (!SOFTMAX) rsum += tree_sum16(ds);
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t) dqacc[d] = E::mma(ktA[d][t], sf[t], dqacc[d]);
    }

    float rs = 0.f;
    if constexpr (!SOFTMAX) rs = xhalf_sum(rsum);
    // Non-softmax: the block's Q (with the position term) in the dQ
    // accumulator layout, for the norm term.  Then the next block's operands
    // are requested before this block's dQ is written.
    float qc[SOFTMAX ? 1 : ND][4][4];
    if constexpr (!SOFTMAX) frag_cfeat<T, KS>(qf, qc);
    qb = hr_block(k + 1, wave, W, nblk, causal);
    if (qb >= 0) load_qd(qb);
    if (qvalid) {
      T* drow = dQ + (int64_t)qtok * p.sdq[2];
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int dd = 32 * d + 8 * g + 4 * h;
          if (dd < D) {
            float v4[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              if constexpr (SOFTMAX) v4[e] = g2 * dqacc[d][4 * g + e];
              else v4[e] = g2 * (dqacc[d][4 * g + e] - rs * qc[d][g][e]);
            }
            st4f<T>(drow + dd, v4);
          }
        }
    }
  }
}

template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS = false>
__global__ __launch_bounds__(64 * W) void rbf_bwd_dkdv_hr_kernel(const Params p) {
  typedef CLayout<32 * NB> L;
  __shared__ __attribute__((aligned(16))) T sQ[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) T sD[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) float sOff[32 * NB];
  __shared__ __attribute__((aligned(16))) float sDel[32 * NB];
  bwd_dkdv_hr_body<T, DP, W, NB, SOFTMAX, POS>(p, sQ, sD, sOff, sDel);
}

template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS = false>
__global__ __launch_bounds__(64 * W) void rbf_bwd_dq_hr_kernel(const Params p) {
  typedef CLayout<32 * NB> L;
  __shared__ __attribute__((aligned(16))) T sK[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) T sV[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) float sKn[32 * NB];
  bwd_dq_hr_body<T, DP, W, NB, SOFTMAX, POS>(p, sK, sV, sKn);
}

// ---------------------------------------------------------------------------
// The whole backward of a head in one launch: the dQ pass (K, V resident;
// writes Delta) then, after a barrier, the dK/dV pass (Q, dO resident; reads
// that Delta) in the same LDS.  One kernel boundary fewer than two launches,
// and a CU that finishes its dQ pass starts its dK/dV load while others still
// compute.
// ---------------------------------------------------------------------------
template <typename T, int DP, int W, int NB, bool SOFTMAX, bool POS = false>
__global__ __launch_bounds__(64 * W) void rbf_bwd_hr_kernel(const Params p) {
  typedef CLayout<32 * NB> L;
  __shared__ __attribute__((aligned(16))) T sA[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) T sB[L::template size<DP>()];
  __shared__ __attribute__((aligned(16))) float s1[32 * NB];
  __shared__ __attribute__((aligned(16))) float s2[32 * NB];
  // The per-query term passes from one pass to the other through s2 (the
  // global copy is written too, as the two-launch form writes it, but not
  // read back).  The dK/dV pass requests its first loads before the barrier
  // that ends the dQ pass.
  bwd_dq_hr_body<T, DP, W, NB, SOFTMAX, POS>(p, sA, sB, s1, s2);
  if constexpr (SOFTMAX)
    bwd_dkdv_hr_body<T, DP, W, NB, SOFTMAX, POS, true>(p, sA, sB, s1, s2);
  else
    bwd_dkdv_hr_body<T, DP, W, NB, SOFTMAX, POS, true>(p, sA, sB, s2, s1);
}

}  // namespace rbf
