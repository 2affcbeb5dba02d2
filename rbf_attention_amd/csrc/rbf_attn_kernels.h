// Fused RBF attention kernels for MI355X (gfx950, CDNA4).
//
// Math (reference: rbf_attention.py:65-219, 279-642, 861-1352):
//   acc_ij = q_i.k_j - 0.5*||k_j||^2               (MFMA, fp32 accumulate)
//   softmax:     P_ij = exp2(c*acc_ij - L_i),  c = 2*gamma*log2(e)
//                L_i  = base-2 log-sum-exp of c*acc_i.  (rbf_attention.py:219)
//   non-softmax: P_ij = exp2(c*acc_ij - c*0.5*||q_i||^2) = exp(-gamma||q_i-k_j||^2)
//   bwd: dP = dO.V^T; dS = P*(dP - Delta) (softmax) or P*dP (non-softmax)
//        dV = P^T dO; dQ = 2g(dS.K - rowsum(dS) q) [rowsum term non-softmax only]
//        dK = 2g(dS^T.Q - colsum(dS) k)
//
// Layout choices (all MFMA are v_mfma_f32_32x32x16_{bf16,f16}, or eight
// v_mfma_f32_32x32x2f32 for fp32):
//  * A 32x32 MFMA accumulator holds, in lane l = 32h + n, column n and the 16
//    rows crow(i, h) = 8(i/4) + 4h + (i%4).  Every product is oriented so that
//    the column index is the token the wave "owns" (the query in fwd/dQ, the
//    key in dK/dV): softmax statistics, L, Delta, the key norm and the
//    row/column sums are then per-lane scalars.
//  * An operand fragment is 8 elements per lane: lane (n, h), k-step t holds
//    contraction indices 16t + 8h + s (s = 0..7).  Both operands of one MFMA
//    use the same convention, so any hardware K-order is consistent.
//  * An accumulator reused as an operand (P, dS) contributes contraction index
//    crow(8t + s, h) = 16t + 8(s/4) + 4h + s%4 at slot s of k-step t.  The
//    other operand is read from a "transposed" LDS tile whose token axis is
//    stored in permuted order swap23(r) (bits 2 and 3 of the token index
//    swapped), which turns that index set back into 8 contiguous elements.
//  * Token axis is cut into 32-token blocks aligned to the END of the
//    sequence: block b covers [org + 32b, org + 32b + 32), org = -(-N mod 32).
//    The ragged part (e.g. 4 register tokens of N = 516) is the head of
//    block 0, which causal attention touches least.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

namespace rbf {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x8_t __attribute__((ext_vector_type(8)));

constexpr float kLog2e = 1.4426950408889634f;
// Lazy rescale threshold (base-2 units): the running max is only raised when a
// new tile exceeds it by more than this, so P <= 2^kTau before normalising.
constexpr float kTau = 8.0f;

// Kernel parameters, shared by all kernels (passed by value).
struct Params {
  const void* q;
  const void* k;
  const void* v;
  const void* o;     // fwd: output (written); bwd softmax: read for Delta
  const void* dout;
  void* dq;
  void* dk;
  void* dv;
  float* lse;        // (B,H,N) fp32
  float* delta;      // (B,H,N) fp32
  int64_t sq[3], sk[3], sv[3], so[3], sdo[3], sdq[3], sdk[3], sdv[3];
  int B, H, N, D;
  int causal, num_prefix;
  float gamma;       // RBF bandwidth
  float c;           // 2 * gamma * log2(e)
  int org;           // first token of block 0 (<= 0)
  int nblk;          // number of 32-token blocks
  int hchunk;        // heads per heaviest-first chunk on one XCD (>= 1)
  int nbin;          // work-groups per head (set per launch; each runs a bin of groups)
  const void* pos;   // position term added to Q and K as they are read (null: none;
                     // only the head-resident kernels read it)
  int64_t spos[3];   // its (b, h, n) strides; b may be 0 (shared by the batch)
};

// ---------------------------------------------------------------------------
// Element traits: fragment type, MFMA, LDS padding.
// ---------------------------------------------------------------------------
template <typename T>
struct Elem;

template <>
struct Elem<__bf16> {
  typedef bf16x8_t frag;
  typedef bf16x4_t quad;
  typedef u32x4_t raw;
  static constexpr int PAD = 8;  // 16 bytes
  __device__ static inline f32x16_t mma(frag a, frag b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<_Float16> {
  typedef f16x8_t frag;
  typedef f16x4_t quad;
  typedef u32x4_t raw;
  static constexpr int PAD = 8;
  __device__ static inline f32x16_t mma(frag a, frag b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

template <>
struct Elem<float> {
  typedef f32x8_t frag;
  typedef f32x4_t quad;
  typedef u32x8_t raw;
  static constexpr int PAD = 4;  // 16 bytes
  __device__ static inline f32x16_t mma(frag a, frag b, f32x16_t c) {
#pragma unroll
    for (int s = 0; s < 8; ++s) c = __builtin_amdgcn_mfma_f32_32x32x2f32(a[s], b[s], c, 0, 0, 0);
    return c;
  }
};

template <typename T>
__device__ inline typename Elem<T>::frag zero_frag() {
  typedef typename Elem<T>::raw raw;
  raw z = {};
  return __builtin_bit_cast(typename Elem<T>::frag, z);
}

// 8 consecutive elements; p is 16-byte aligned.
template <typename T>
__device__ inline typename Elem<T>::frag ld8(const T* p) {
  typedef typename Elem<T>::raw raw;
  typedef raw raw16 __attribute__((aligned(16)));
  return __builtin_bit_cast(typename Elem<T>::frag, *reinterpret_cast<const raw16*>(p));
}

template <typename T>
__device__ inline void st8(T* p, typename Elem<T>::frag f) {
  typedef typename Elem<T>::raw raw;
  typedef raw raw16 __attribute__((aligned(16)));
  *reinterpret_cast<raw16*>(p) = __builtin_bit_cast(raw, f);
}

// a + b in fp32, rounded to the element type: what an elementwise add of two
// element-type tensors stores.
template <typename T>
__device__ inline typename Elem<T>::frag add8(typename Elem<T>::frag a, typename Elem<T>::frag b) {
  typename Elem<T>::frag r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (T)((float)a[e] + (float)b[e]);
  return r;
}

// 8 elements at p, plus the 8 at pp when pp is not null (the position term
// of a Q or K row).
template <typename T>
__device__ inline typename Elem<T>::frag ld8p(const T* p, const T* pp) {
  const typename Elem<T>::frag x = ld8<T>(p);
  return pp ? add8<T>(x, ld8<T>(pp)) : x;
}

// ld8 of p, plus the 8 elements at pp (rounded as add8) when ADD: a position
// term fused into a Q or K read, chosen at compile time so that the loads
// carry no null-pointer branches (with them every load waited on the
// previous one).
template <typename T, bool ADD>
__device__ inline typename Elem<T>::frag ld8a(const T* p, const T* pp) {
  if constexpr (ADD) return add8<T>(ld8<T>(p), ld8<T>(pp));
  else return ld8<T>(p);
}

// 4 consecutive elements (8-byte aligned for 16-bit types, 16 for fp32).
template <typename T>
__device__ inline void ld4f(const T* p, float out[4]) {
  typedef typename Elem<T>::quad quad;
  typedef quad quadA __attribute__((aligned(sizeof(T) * 4)));
  quad v = *reinterpret_cast<const quadA*>(p);
#pragma unroll
  for (int e = 0; e < 4; ++e) out[e] = (float)v[e];
}

// ld4f of p, plus pp (rounded to the element type, as add8) when not null.
template <typename T>
__device__ inline void ld4fp(const T* p, const T* pp, float out[4]) {
  ld4f<T>(p, out);
  if (pp) {
    float a[4];
    ld4f<T>(pp, a);
#pragma unroll
    for (int e = 0; e < 4; ++e) out[e] = (float)(T)(out[e] + a[e]);
  }
}

template <typename T>
__device__ inline void st4f(T* p, const float in[4]) {
  typedef typename Elem<T>::quad quad;
  typedef quad quadA __attribute__((aligned(sizeof(T) * 4)));
  quad v;
#pragma unroll
  for (int e = 0; e < 4; ++e) v[e] = (T)in[e];
  *reinterpret_cast<quadA*>(p) = v;
}

__device__ inline int swap23(int r) { return (r & ~12) | ((r & 4) << 1) | ((r & 8) >> 1); }
// Row of accumulator element i held by lane half h (32x32 MFMA C layout).
__device__ inline int crow(int i, int h) { return 8 * (i >> 2) + 4 * h + (i & 3); }

// gfx950 ds_read_b64_tr_b16: within each 16-lane group, lane g addresses
// token row R0 + g/4 at feature column n0 + 4(g%4) and receives
// X[R0 + e][n0 + g] for e = 0..3.  Two such reads give lane (m = lane % 32,
// h = lane / 32) feature fbase + m of the 8 tokens tbase + 8(s/4) + 4h + s%4,
// s = 0..7 -- the contraction order of a P / dS accumulator reused as the
// other MFMA operand (crow(8t + s, h) with tbase = 16t).  See ld_trc.
typedef short s16x4_t __attribute__((ext_vector_type(4)));

// Transposing read from a padded row-major tile (row stride LD elements).
template <typename T, int LD>
__device__ inline typename Elem<T>::frag ld_tr8(const T* tile, int tbase, int fbase, int lane) {
  static_assert(sizeof(T) == 2, "transposing LDS reads are for 16-bit elements");
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const int g = lane & 15;
  const int row = tbase + 4 * (lane >> 5) + (g >> 2);
  const int col = fbase + 16 * ((lane >> 4) & 1) + 4 * (g & 3);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + row * LD + col));
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(tile + (row + 8) * LD + col));
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
  const s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Elem<T>::frag, v);
}

// Offset of the 8-token chunk starting at tile-local token position p8
// (a multiple of 8) in feature row `feat` of a transposed tile with ROWS
// tokens (see Tile::store_trans).
template <int ROWS>
__device__ inline int tchunk(int feat, int p8) {
  return (((p8 >> 3) ^ ((feat >> 3) & (ROWS / 8 - 1))) << 3);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Combine a lane's value with the one of lane l ^ 32 (v_permlane32_swap: a
// VALU op, no LDS round trip).  Both halves receive the same result.
__device__ inline float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Sum over lanes l and l ^ 16 (v_permlane16_swap).
__device__ inline float xrow_sum(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Sum over aligned groups of G consecutive lanes (G in {1, 2, 4, 8, 16, 32})
// with DPP lane moves (and one permlane16 swap for 32); every lane of a group
// receives the group sum.
template <int G>
__device__ inline float group_sum(float x) {
  if constexpr (G >= 2) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0xB1, 0xF, 0xF, false));
  if constexpr (G >= 4) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x4E, 0xF, 0xF, false));
  if constexpr (G >= 8) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x141, 0xF, 0xF, false));
  if constexpr (G >= 16) x += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), 0x140, 0xF, 0xF, false));
  if constexpr (G >= 32) x = xrow_sum(x);
  static_assert(G <= 32, "group_sum supports groups of at most 32 lanes");
  return x;
}

// Pairwise (tree) reductions of the 16 accumulator values of a lane.
__device__ inline float tree_sum16(const float v[16]) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = v[i] + v[i + 8];
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] += a[i + 4];
  return (a[0] + a[2]) + (a[1] + a[3]);
}
__device__ inline float tree_max16(const f32x16_t& v) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = fmaxf(v[i], v[i + 8]);
#pragma unroll
  for (int i = 0; i < 4; ++i) a[i] = fmaxf(a[i], a[i + 4]);
  return fmaxf(fmaxf(a[0], a[2]), fmaxf(a[1], a[3]));
}

__device__ inline f32x16_t zero16() {
  f32x16_t z = {};
  return z;
}

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

// sum_e a[e] * b[e] over 8 elements in fp32 (v_dot2_f32_{bf16,f16} for the
// 16-bit types: products exact, fp32 accumulation).
template <typename T>
__device__ inline float dot8(typename Elem<T>::frag a, typename Elem<T>::frag b) {
  float s = 0.f;
  if constexpr (sizeof(T) == 2) {
    typedef typename std::conditional<std::is_same<T, __bf16>::value, bf16x2_t, f16x2_t>::type pair;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const pair x = {a[e], a[e + 1]}, y = {b[e], b[e + 1]};
      if constexpr (std::is_same<T, __bf16>::value) s = __builtin_amdgcn_fdot2_f32_bf16(x, y, s, false);
      else s = __builtin_amdgcn_fdot2(x, y, s, false);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) s = fmaf((float)a[e], (float)b[e], s);
  }
  return s;
}

template <typename T>
__device__ inline float sumsq8(typename Elem<T>::frag f) {
  return dot8<T>(f, f);
}

template <typename T>
__device__ inline uint32_t bits16(T x) {
  return (uint32_t)__builtin_bit_cast(uint16_t, x);
}

// ---------------------------------------------------------------------------
// Cooperative tile of ROWS tokens x DP features, staged global -> registers
// -> LDS.  Work unit = two adjacent rows x 8 features.  Consecutive threads
// take consecutive 8-feature chunks of a row pair, so each load instruction
// reads whole rows.
// ---------------------------------------------------------------------------
template <typename T, int ROWS, int DP, int NT>
struct Tile {
  typedef typename Elem<T>::frag frag;
  static constexpr int CPR = DP / 8;
  static constexpr int UNITS = (ROWS / 2) * CPR;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static_assert(NT % CPR == 0, "a row pair must not straddle threads unevenly");
  frag r[PER][2];
  int tok0_, n_;  // token of row 0 and sequence length of the loaded tile

  __device__ inline void load(const T* base, int64_t sn, int tok0, int N, int D, int tid) {
    tok0_ = tok0;
    n_ = N;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      const int rp = u / CPR, dc = u % CPR;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int tok = tok0 + 2 * rp + e;
        if (u < UNITS && tok >= 0 && tok < N && dc * 8 < D)
          r[j][e] = ld8<T>(base + (int64_t)tok * sn + dc * 8);
        else
          r[j][e] = zero_frag<T>();
      }
    }
  }

  // lds[row * LD + feature]
  template <int LD>
  __device__ inline void store_rows(T* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      if (UNITS % NT != 0 && u >= UNITS) continue;
      const int rp = u / CPR, dc = u % CPR;
#pragma unroll
      for (int e = 0; e < 2; ++e) st8<T>(lds + (2 * rp + e) * LD + dc * 8, r[j][e]);
    }
  }

  // lds[feature * LDT + tpos(feature, row)]: the token axis is stored in
  // swap23 order and its 8-element chunks are XOR-swizzled by feature/8, so
  // that the 8 feature rows one store instruction touches fall in different
  // LDS banks while an 8-token chunk stays contiguous for the MFMA reads.
  template <int LDT>
  __device__ inline void store_trans(T* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      if (UNITS % NT != 0 && u >= UNITS) continue;
      const int rp = u / CPR, dc = u % CPR;
      const int pos = swap23(2 * rp);  // even; row 2rp+1 lands at pos+1
      // every feature row 8dc + c shares the swizzle value dc
      const int spos = (((pos >> 3) ^ (dc & (ROWS / 8 - 1))) << 3) | (pos & 7);
      if constexpr (sizeof(T) == 2) {
        const u32x4_t a = __builtin_bit_cast(u32x4_t, r[j][0]);  // row 2rp: elements (2m, 2m+1) in dword m
        const u32x4_t b = __builtin_bit_cast(u32x4_t, r[j][1]);  // row 2rp+1
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          // (row0[2m], row1[2m]) and (row0[2m+1], row1[2m+1]) as 16-bit pairs
          *reinterpret_cast<uint32_t*>(lds + (dc * 8 + 2 * m) * LDT + spos) = __builtin_amdgcn_perm(b[m], a[m], 0x05040100u);
          *reinterpret_cast<uint32_t*>(lds + (dc * 8 + 2 * m + 1) * LDT + spos) = __builtin_amdgcn_perm(b[m], a[m], 0x07060302u);
        }
      } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          lds[(dc * 8 + c) * LDT + spos] = r[j][0][c];
          lds[(dc * 8 + c) * LDT + spos + 1] = r[j][1][c];
        }
      }
    }
  }

  // nrm[row] = -0.5 * ||row||^2 in fp32 (from the input-dtype values), and
  // -inf for padding rows (tokens outside [0, N)): used as the initial value
  // of an S accumulator, it makes every logit against a padding key -inf, so
  // padding needs no element mask.
  __device__ inline void store_neg_halfnorm(float* nrm, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      const int rp = u / CPR, dc = u % CPR;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const float s = group_sum<CPR>(sumsq8<T>(r[j][e]));
        const int tok = tok0_ + 2 * rp + e;
        if (dc == 0 && u < UNITS) nrm[2 * rp + e] = (tok >= 0 && tok < n_) ? -0.5f * s : -__builtin_inff();
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Chunk-major LDS tile for 16-bit elements (ROWS tokens x DP features).  A
// chunk is 8 consecutive features of one token (16 bytes).  The tile is
// DP/8 chunk columns; column c holds chunk c of the ROWS tokens back to back
// and is followed by 64 bytes of padding, so consecutive columns start 64
// bytes apart modulo the 256 bytes that the 64 LDS banks cover.  Every access
// pattern of the kernels is then free of bank conflicts:
//   * row reads (ld8): 16 lanes read one chunk of 16 consecutive tokens --
//     256 contiguous bytes;
//   * transposing reads (ld_trc): 32 lanes read 4 chunks x 4 tokens -- four
//     64-byte runs in four different bank quarters;
//   * tile stores (CTile::store): 16 lanes write 4 chunks x 4 tokens, same.
// Addresses are a per-lane base plus compile-time offsets.
// ---------------------------------------------------------------------------
template <int ROWS>
struct CLayout {
  static_assert(ROWS % 16 == 0, "chunk columns must span a multiple of 256 bytes");
  static constexpr int CS = ROWS * 8 + 32;  // elements per chunk column
  template <int DP>
  static constexpr int size() { return DP / 8 * CS; }
  __device__ static inline int off(int row, int col) { return (col >> 3) * CS + row * 8 + (col & 7); }
};

// Transposing read from a chunk-major tile: 8 consecutive tokens (in the
// P / dS contraction order tbase + 8(s/4) + 4h + s%4) of feature fbase + n.
template <typename T, int ROWS>
__device__ inline typename Elem<T>::frag ld_trc(const T* tile, int tbase, int fbase, int lane) {
  static_assert(sizeof(T) == 2, "transposing LDS reads are for 16-bit elements");
  typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
  const int g = lane & 15;
  const int row = tbase + 4 * (lane >> 5) + (g >> 2);
  const int col = fbase + 16 * ((lane >> 4) & 1) + 4 * (g & 3);
  const T* a = tile + CLayout<ROWS>::off(row, col);
  const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)a);
  const s16x4_t hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(a + 64));  // row + 8
  typedef short s16x8_t __attribute__((ext_vector_type(8)));
  const s16x8_t v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(typename Elem<T>::frag, v);
}

// Cooperative chunk-major tile, staged global -> registers -> LDS.  Work
// unit = one chunk.  Unit u maps to chunk 4*(u/16 mod DP/32) + u%4 of token
// 4*(u/16 div DP/32) + (u/4)%4: 16 consecutive units cover 4 tokens x 4
// chunks (64 contiguous bytes of each token in global memory).
template <typename T, int ROWS, int DP, int NT>
struct CTile {
  typedef typename Elem<T>::frag frag;
  typedef CLayout<ROWS> L;
  static constexpr int CPR = DP / 8;
  static constexpr int CG = CPR / 4;  // groups of 4 chunks per token
  static constexpr int UNITS = ROWS * CPR;
  static constexpr int PER = (UNITS + NT - 1) / NT;
  static_assert(CPR % 4 == 0 && CG <= 4, "DP must be 32, 64 or 128");
  frag r[PER];
  int tok0_, n_;

  __device__ static inline void unit(int u, int& row, int& ch) {
    const int rest = u >> 4;
    ch = 4 * (rest % CG) + (u & 3);
    row = 4 * (rest / CG) + ((u >> 2) & 3);
  }

  __device__ inline void load(const T* base, int64_t sn, int tok0, int N, int D, int tid) {
    tok0_ = tok0;
    n_ = N;
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      int row, ch;
      unit(u, row, ch);
      const int tok = tok0 + row;
      r[j] = (u < UNITS && tok >= 0 && tok < N && ch * 8 < D) ? ld8<T>(base + (int64_t)tok * sn + ch * 8) : zero_frag<T>();
    }
  }

  __device__ inline void store(T* lds, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      if (UNITS % NT != 0 && u >= UNITS) continue;
      int row, ch;
      unit(u, row, ch);
      st8<T>(lds + L::off(row, 8 * ch), r[j]);
    }
  }

  // nrm[row] = -0.5 * ||row||^2 in fp32 (from the input-dtype values), and
  // -inf for padding rows (tokens outside [0, N)): used as the initial value
  // of an S accumulator, it makes every logit against a padding key -inf, so
  // padding needs no element mask.  A token's chunks sit in lanes that differ
  // in lane bits 0-1 and, for DP > 32, 4-5.
  __device__ inline void store_neg_halfnorm(float* nrm, int tid) const {
#pragma unroll
    for (int j = 0; j < PER; ++j) {
      const int u = tid + j * NT;
      int row, ch;
      unit(u, row, ch);
      float s = group_sum<4>(sumsq8<T>(r[j]));
      if constexpr (CG >= 2) s = xrow_sum(s);
      if constexpr (CG >= 4) s = xhalf_sum(s);
      const int tok = tok0_ + row;
      if (ch == 0 && u < UNITS) nrm[row] = (tok >= 0 && tok < n_) ? -0.5f * s : -__builtin_inff();
    }
  }
};

// LDS tile layout of the kernels.  16-bit tiles with 128 features are
// chunk-major (CLayout); narrower 16-bit tiles and fp32 tiles are row-major
// with a 16-byte row pad, which measured faster for them (their row reads
// and transposing reads are already nearly conflict-free).
template <typename T, int DP>
constexpr bool kChunkMajor = sizeof(T) == 2 && DP == 128;

template <typename T, int ROWS, int DP, int NT>
using TileFor = std::conditional_t<kChunkMajor<T, DP>, CTile<T, ROWS, DP, NT>, Tile<T, ROWS, DP, NT>>;

// CMF: chunk-major whatever the default for (T, DP) (the LDS-DMA kernels,
// whose DMA writes 64-row chunk columns).
template <typename T, int ROWS, int DP, bool CMF = kChunkMajor<T, DP>>
struct TileLayout {
  static constexpr bool CM = CMF;
  static constexpr int LDR = DP + Elem<T>::PAD;
  static constexpr int SIZE = CM ? CLayout<ROWS>::template size<DP>() : ROWS * LDR;
  __device__ static inline int off(int row, int col) {
    if constexpr (CM) return CLayout<ROWS>::off(row, col);
    else return row * LDR + col;
  }
  template <typename TT>
  __device__ static inline void store(const TT& tile, T* lds, int tid) {
    if constexpr (CM) tile.store(lds, tid);
    else tile.template store_rows<LDR>(lds, tid);
  }
  // V^T / K^T / Q^T / dO^T fragment (16-bit types)
  __device__ static inline typename Elem<T>::frag tr(const T* tile, int tbase, int fbase, int lane) {
    if constexpr (CM) return ld_trc<T, ROWS>(tile, tbase, fbase, lane);
    else return ld_tr8<T, LDR>(tile, tbase, fbase, lane);
  }
};

// ---------------------------------------------------------------------------
// LDS-DMA staging of chunk-major tiles (16-bit elements, 64 or 128 features).
//
// global_load_lds_dwordx4 writes each lane's 16 bytes to consecutive 16-byte
// LDS slots (M0 base + 16 * lane), i.e. 1 KB per instruction: in a CLayout
// tile, 64 consecutive rows of one chunk column.  So one instruction stages
// rows r0 .. r0 + 63 of chunk ch, lane l reading row r0 + l, and no register
// ever holds the tile.  Rows outside [0, N) read zeros (the buffer range
// check of buffer_rsrc): the kernels mask such keys and queries by their -inf
// norm or offset, never by their values, which only have to be finite.
//
// A pipeline of three tiles (dma_pipeline) runs the compute of tile t while
// tile t + 1 is landed in LDS (its per-row terms formed from LDS) and tile
// t + 2 is in flight.  One barrier per tile: before it every wave waits for
// its own DMA of tile t + 1 (issued a whole tile earlier); after it tile
// t + 1 and the per-row terms of tile t (formed during tile t - 1) are
// visible to every wave.
//
// The DMA instruction is issued from inline assembly, so the compiler neither
// tracks it nor waits for it: every wait for it is the explicit one before
// the barrier.  (The compiler's own waits for its loads stay correct, since
// vector-memory operations retire in order; at worst they also wait for a
// DMA issued earlier.  Through the compiler builtin, the DMA made every read
// of the tiles wait for the DMA in flight unless the three buffers were
// separate arrays in an unrolled loop, which cost the kernels spills.)
// ---------------------------------------------------------------------------
// s_waitcnt vmcnt(0): this wave's vector-memory loads (LDS-DMA included) done.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Work-group barrier for LDS data only: this wave's LDS operations complete,
// then s_barrier; the compiler moves no memory access across it.
// __syncthreads() also waits for every outstanding vector-memory load (its
// fence), which would make a mid-tile barrier wait for the DMA in flight.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource over `bytes` bytes from `base` (stride 0, gfx9 data
// format word): a load at byte offset >= bytes -- a negative offset included,
// read as unsigned -- returns zeros.
__device__ __forceinline__ i32x4_t buffer_rsrc(const void* base, uint32_t bytes) {
  const uint64_t a = (uint64_t)base;
  i32x4_t r;
  r.x = __builtin_amdgcn_readfirstlane((int)(uint32_t)a);
  r.y = __builtin_amdgcn_readfirstlane((int)((uint32_t)(a >> 32) & 0xffffu));
  r.z = __builtin_amdgcn_readfirstlane((int)bytes);
  r.w = 0x00020000;
  return r;
}

// buffer_load_dwordx4 ... lds: 16 bytes per lane from byte offset voff of
// the buffer to LDS byte address lds + 16 * lane (lds wave-uniform).  M0
// carries the LDS address; nothing else in these kernels uses M0.
#pragma clang diagnostic push
#pragma clang diagnostic ignored "-Winline-asm"
__device__ __forceinline__ void dma16(uint32_t voff, i32x4_t rsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dwordx4 %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
// The same with 4 bytes per lane (LDS address lds + 4 * lane).
__device__ __forceinline__ void dma4(uint32_t voff, i32x4_t rsrc, uint32_t lds) {
  asm volatile("s_mov_b32 m0, %2\n\tbuffer_load_dword %0, %1, 0 offen lds" : : "v"(voff), "s"(rsrc), "s"(lds)
               : "memory", "m0");
}
#pragma clang diagnostic pop

// LDS byte address of a __shared__ element.
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(const T* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) T*)p;
}

// The DMA of two (ROWS x DP) chunk-major tiles -- tokens tok0 .. tok0 +
// ROWS - 1 of slices A and B, each (N, DP) with row stride sa / sb -- by W
// waves: 2 * (ROWS / 64) * (DP / 8) instructions of 64 rows x one chunk, dealt
// round-robin to the waves.  A wave's lane offsets (relative to the tile's
// first row) and LDS offsets are fixed, so a tile costs one add per
// instruction.  Tokens outside [0, N) read zeros (buffer range check; the
// host keeps N * stride * sizeof(T) below 2^31).
template <typename T, int ROWS, int DP, int W>
struct DmaPair {
  static_assert(sizeof(T) == 2 && ROWS % 64 == 0, "DMA tiles: 16-bit, whole 64-row groups");
  static constexpr int CPR = DP / 8, PER = (ROWS / 64) * CPR, NI = 2 * PER, NIW = (NI + W - 1) / W;
  i32x4_t ra, rb;
  uint32_t voff[NIW];  // lane byte offset of instruction j, tile row 0 at offset 0
  int loff[NIW];       // element offset of instruction j's 1 KB in its tile
  int rowa, rowb;      // row strides in bytes
  int wave;

  __device__ inline void init(const T* A, int64_t sa, const T* B, int64_t sb, int N, int wave_, int lane) {
    wave = wave_;
    rowa = (int)(sa * (int64_t)sizeof(T));
    rowb = (int)(sb * (int64_t)sizeof(T));
    ra = buffer_rsrc(A, (uint32_t)N * (uint32_t)rowa);
    rb = buffer_rsrc(B, (uint32_t)N * (uint32_t)rowb);
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      const int i = min(wave + j * W, NI - 1), k = i % PER, rg = k / CPR, ch = k % CPR;
      const int row = i < PER ? rowa : rowb;
      voff[j] = (uint32_t)((64 * rg + lane) * row + 16 * ch);
      loff[j] = CLayout<ROWS>::off(64 * rg, 8 * ch);
    }
  }

  __device__ inline void issue(int tok0, T* tA, T* tB) const {
    const uint32_t la = lds_addr(tA), lb = lds_addr(tB);
#pragma unroll
    for (int j = 0; j < NIW; ++j) {
      // instruction wave + j * W (if below NI) reads slice A when below PER
      // (both known per j when W divides PER)
      if (NI % W != 0 && wave + j * W >= NI) continue;
      const bool isa = PER % W == 0 ? j < PER / W : wave + j * W < PER;
      if (isa) dma16(voff[j] + (uint32_t)(tok0 * rowa), ra, la + 2u * (uint32_t)loff[j]);
      else dma16(voff[j] + (uint32_t)(tok0 * rowb), rb, lb + 2u * (uint32_t)loff[j]);
    }
  }
};

// nrm[row] = -0.5 ||row||^2 (fp32, from the element-type values) of a landed
// (ROWS x DP) chunk-major tile, -inf for tokens outside [0, N).  TPR
// consecutive threads share a row (the largest power of two <= NT / ROWS,
// at most DP / 8); threads past ROWS * TPR have no row.
template <typename T, int ROWS, int DP, int NT>
__device__ __forceinline__ void tile_neg_halfnorms(const T* tile, float* nrm, int tok0, int N, int tid) {
  constexpr int Q = NT / ROWS, CPR = DP / 8;
  constexpr int TQ = Q >= 16 ? 16 : Q >= 8 ? 8 : Q >= 4 ? 4 : Q >= 2 ? 2 : 1;
  constexpr int TPR = TQ < CPR ? TQ : CPR, CPT = CPR / TPR;
  static_assert(Q >= 1, "at least one thread per row");
  if (ROWS * TPR < NT && tid >= ROWS * TPR) return;
  const int row = tid / TPR, part = tid % TPR;
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < CPT; ++j) s += sumsq8<T>(ld8<T>(tile + CLayout<ROWS>::off(row, 8 * (part * CPT + j))));
  s = group_sum<TPR>(s);
  const int tok = tok0 + row;
  if (part == 0) nrm[row] = (tok >= 0 && tok < N) ? -0.5f * s : -__builtin_inff();
}

// The three-tile pipeline.  issue(t, b) requests tile t into buffer b,
// land(t, b) forms tile t's per-row terms from buffer b (after its data is
// visible), compute(t, b) runs tile t from buffer b (b = t mod 3).
template <typename Issue, typename Land, typename Compute>
__device__ __forceinline__ void dma_pipeline(int nt, Issue&& issue, Land&& land, Compute&& compute) {
  if (nt <= 0) return;
  issue(0, 0);
  if (nt > 1) issue(1, 1);
  wait_vmem();
  __syncthreads();
  land(0, 0);
  int b0 = 0, b1 = 1, b2 = 2;  // buffers of tiles t, t + 1, t + 2
  for (int t = 0; t < nt; ++t) {
    wait_vmem();
    lds_barrier();
    if (t + 2 < nt) issue(t + 2, b2);
    // tile t + 1's terms after tile t's compute (they are used only after
    // the next barrier): waves that finish their blocks early do this work
    // while the others still compute.
    compute(t, b0);
    if (t + 1 < nt) land(t + 1, b1);
    const int b = b0;
    b0 = b1;
    b1 = b2;
    b2 = b;
  }
}

// Work-group -> (b*H + h, bin).  The hardware deals work-groups round-robin
// over the 8 XCDs (block id mod 8) and each XCD starts its share in block-id
// order.  When B*H is a multiple of 8, XCD x owns whole heads
// [x*BH/8, (x+1)*BH/8), so the work-groups of a head share K/V (or Q/dO) in
// that XCD's L2.  The XCD's heads are taken in chunks of `hchunk` heads -- as
// many as the host expects to fit in L2 together -- and inside a chunk bin 0
// of every head runs first, then every head's bin 1, and so on.
__device__ inline void decode_wg(int nbin, int hchunk, int& bh, int& bin) {
  const int total = gridDim.x;
  const int bid = blockIdx.x;
  const int BH = total / nbin;
  if ((BH & 7) == 0) {
    const int per_xcd = BH >> 3;
    const int local = bid >> 3;
    const int chunk = local / (hchunk * nbin);
    const int h0 = chunk * hchunk;
    const int nh = min(hchunk, per_xcd - h0);
    const int r = local - h0 * nbin;
    bin = r / nh;
    bh = (bid & 7) * per_xcd + h0 + (r - bin * nh);
  } else {
    bh = bid / nbin;
    bin = bid - bh * nbin;
  }
}

// Runs f(bh, group) for every group of this work-group's bin.  A head's
// `ngrp` groups are ranked by causal weight, heaviest first (the weight
// rises with the group index when `reverse` is true -- causal forward and dQ
// -- and falls with it otherwise -- dK/dV, whose early keys see the most
// queries), and dealt to the head's `p.nbin` bins in boustrophedon order:
// ranks 0..R-1 to bins 0..R-1, ranks R..2R-1 to bins R-1..0, and so on.  With
// R = ngrp every bin holds one group (heaviest bins first in launch order);
// with fewer bins the host picks R so that all work-groups run at once and
// the snake order gives them near-equal causal work.  The bin's groups run
// back to back, separated by a barrier (they reuse the LDS tiles).
// BIN = false compiles the one-group-per-work-group form only (no loop
// around the body: the loop costs the long-sequence kernels registers and
// speed).
template <bool BIN, typename F>
__device__ __forceinline__ void for_each_group(const Params& p, int ngrp, bool reverse, F&& f) {
  if constexpr (!BIN) {
    int bh, rank;
    decode_wg(ngrp, p.hchunk, bh, rank);
    f(bh, reverse ? ngrp - 1 - rank : rank);
    return;
  }
  const int nbin = (p.nbin > 0 && p.nbin < ngrp) ? p.nbin : ngrp;
  int bh, bin;
  decode_wg(nbin, p.hchunk, bh, bin);
  for (int k = 0;; ++k) {
    const int rank = k * nbin + ((k & 1) ? nbin - 1 - bin : bin);
    if (rank >= ngrp) break;
    if (k) __syncthreads();
    f(bh, reverse ? ngrp - 1 - rank : rank);
  }
}

// Visibility of a 32x32 (query block, key block) pair: `any` if at least one
// pair (i, j) is visible, `full` if every pair is (no element mask needed).
// Block starts below 0 hold padding tokens, which are never visible.
__device__ inline bool blk_any(int q0, int k0, bool causal, int npre) {
  return q0 + 31 >= 0 && k0 + 31 >= 0 && (!causal || k0 <= q0 + 31 || k0 < npre);
}
__device__ inline bool blk_full(int q0, int k0, bool causal, int npre) {
  return q0 >= 0 && k0 >= 0 && (!causal || k0 + 31 <= q0 || k0 + 31 < npre);
}
// Like blk_full, but padding tokens (block 0 when N % 32 != 0) count as
// visible: their logits are already -inf through the accumulator's initial
// value (padding keys, and padding queries in the dK/dV kernel) or their rows
// are never stored (padding queries in the forward and dQ kernels).
__device__ inline bool blk_nomask(int q0, int k0, bool causal, int npre) {
  return !causal || k0 + 31 <= q0 || k0 + 31 < npre;
}
__device__ inline bool elem_vis(int i, int j, bool causal, int npre) {
  return i >= 0 && j >= 0 && (!causal || j <= i || j < npre);
}

// Row offset of accumulator element i without the lane-half term:
// crow(i, h) = crow0(i) + 4h.
__device__ inline constexpr int crow0(int i) { return 8 * (i >> 2) + (i & 3); }

// The keys visible to query i form one range [0, last_key(i)]: j <= i, or a
// prefix (register) key j < npre, or every key when not causal.
__device__ inline int last_key(int i, int N, bool causal, int npre) {
  if (i < 0) return -1;
  return causal ? max(i, npre - 1) : N - 1;
}
// The queries that see key j form one range [first_query(j), N).
__device__ inline int first_query(int j, bool causal, int npre) {
  if (j < 0) return 1 << 30;
  return (!causal || j < npre) ? 0 : j;
}

// Keys along the accumulator rows (fwd, dQ: lane = query): element i holds key
// k0 + crow(i, h); keep it iff 0 <= key <= jmax.  Callers apply the masks
// only to the blocks that need one; the empty volatile asm keeps the compiler
// from turning that branch into compares and selects run on every block.
__device__ inline void mask_key_rows(f32x16_t& s, int k0, int h, int jmax) {
  asm volatile("");
  const int lo = -k0 - 4 * h, hi = jmax - k0 - 4 * h;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (crow0(i) < lo || crow0(i) > hi) s[i] = -__builtin_inff();
}
// Queries along the accumulator rows (dK/dV: lane = key): element i holds
// query q0 + crow(i, h); keep it iff query >= ilo (queries never exceed N-1).
__device__ inline void mask_query_rows(f32x16_t& s, int q0, int h, int ilo) {
  asm volatile("");
  const int lo = ilo - q0 - 4 * h;
#pragma unroll
  for (int i = 0; i < 16; ++i)
    if (crow0(i) < lo) s[i] = -__builtin_inff();
}

// Per-slot values of a 32-entry fp32 LDS vector for the C layout rows of lane
// half h: out[i] = v[crow(i, h)] (four 16-byte reads).
__device__ inline f32x16_t ld_rows16(const float* v, int h) {
  f32x16_t r;
#pragma unroll
  for (int g = 0; g < 4; ++g) {
    const f32x4_t x = *reinterpret_cast<const f32x4_t*>(v + 8 * g + 4 * h);
#pragma unroll
    for (int e = 0; e < 4; ++e) r[4 * g + e] = x[e];
  }
  return r;
}

__device__ inline f32x16_t splat16(float x) {
  f32x16_t r;
#pragma unroll
  for (int i = 0; i < 16; ++i) r[i] = x;
  return r;
}

// ---------------------------------------------------------------------------
// Forward.  A wave owns one 32-query block, a work-group W waves; BN-key
// tiles of K (row-major), V and -0.5||k||^2 stream through double-buffered
// LDS.  Per 32-key block:
//   S^T = K Q^T (accumulator initialised with -0.5||k||^2),
//   P   = exp2(c S^T - m),
//   O^T += V^T P^T with P rounded to the element type (as the reference
//   rounds it before its P V product, rbf_attention.py:201),
//   l_r += the rounded P's sum, in fp32 (v_dot2 against ones on the VALU, 2
//   MFMAs per block fewer than a ones-row product, C3 forward 1140 ->
//   1128 us; the head-resident forward does the same): O is normalised by
//   the sum of exactly the rounded P its numerator uses, so a row that sees
//   one key returns that key's v exactly;
//   l += sum_j P in fp32 from the unrounded P, for L (the reference sums the
//   unrounded P, 196-198).  L taken from l_r was off by up to 2^-9 relative
//   per row, a scale every P of the backward then carried (dV's error at
//   N = 32 was 1.2x that of the reference's own rounding); O normalised by
//   the unrounded l was off by the rounding of the dominant P (the static
//   offset below does not make it 1), e.g. O = v (1 + 2^-9) for one key.
// Softmax offset m: every RBF logit obeys c(q.k - 0.5||k||^2) <= c 0.5||q||^2,
// so m = c 0.5||q||^2 - 60 bounds P by 2^60 without any running max.  If some
// row's keys all lie so far away that its sum falls below 2^-60 (or the sum is
// not finite), the work-group reruns with an online, lazily raised max.  fp16
// cannot hold P up to 2^60 and always takes the online max.
// ---------------------------------------------------------------------------
template <typename T>
__device__ inline typename Elem<T>::frag ones_frag() {
  typename Elem<T>::frag f;
#pragma unroll
  for (int s = 0; s < 8; ++s) f[s] = (T)1.f;
  return f;
}

constexpr float kBoundMargin = 60.f;  // P <= 2^60 under the static bound
constexpr float kSumLow = 0x1p-60f, kSumHigh = 0x1p100f;

// DMA: K and V tiles staged by LDS-DMA (dma_pipeline; 16-bit, D = 64 or 128)
// instead of through registers.
template <typename T, int DP, int W, int BN, bool SOFTMAX, bool DMA = false>
__device__ __forceinline__ void rbf_fwd_group(const Params& p, int bh, int grp) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  constexpr int NT = 64 * W, KB = BN / 32, KS = DP / 16, ND = DP / 32;
  constexpr int LDR = DP + E::PAD, LDT = BN + E::PAD;
  // 16-bit types keep K and V in chunk-major tiles and read V^T with
  // transposing LDS reads; fp32 uses padded row-major K and a transposed copy
  // of V.
  constexpr bool TR = sizeof(T) == 2;
  typedef TileLayout<T, BN, DP, DMA || kChunkMajor<T, DP>> TLy;
  static_assert(!DMA || TR, "LDS-DMA staging is for 16-bit tiles");
  constexpr int TSZ = TLy::SIZE;
  // register staging: two buffers each (a single element when DMA)
  constexpr int NB2 = DMA ? 1 : 2;
  __shared__ __attribute__((aligned(16))) T sK[NB2][DMA ? 8 : TSZ];
  __shared__ __attribute__((aligned(16))) T sVt[NB2][DMA ? 8 : (TR ? TSZ : DP * LDT)];
  auto roff = [](int row, int col) { return TLy::off(row, col); };
  __shared__ __attribute__((aligned(16))) float sKn[NB2][DMA ? 1 : BN];
  // LDS-DMA staging: three buffers each (a single element without DMA)
  constexpr int NB3 = DMA ? 3 : 1;
  __shared__ __attribute__((aligned(16))) T dK[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) T dV[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) float dN[NB3][DMA ? BN : 1];

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const int ngrp = (nblk + W - 1) / W;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  T* O = reinterpret_cast<T*>(const_cast<void*>(p.o)) + b * p.so[0] + hh * p.so[1];

  const int blk0 = nblk - (ngrp - grp) * W;
  const int qblk = blk0 + wave;
  const bool wave_on = qblk >= 0;  // the wave's block holds real queries
  const int q0 = org + 32 * qblk;
  const int qtok = q0 + n;
  const bool qvalid = wave_on && qtok >= 0;
  const int jmax = last_key(qtok, N, causal, npre);
  const int wg_qlast = org + 32 * (blk0 + W) - 1;
  int hi = causal ? max(wg_qlast + 1, npre) : N;
  hi = min(hi, N);
  const int nkt_all = (nblk + KB - 1) / KB;
  const int kshift = nkt_all * KB - nblk;
  const int last_blk = (hi - 1 - org) >> 5;
  const int nkt = (last_blk + kshift) / KB + 1;

  frag qf[KS];
  float qn2 = 0.f;  // c * 0.5 ||q||^2
#pragma unroll
  for (int t = 0; t < KS; ++t) {
    qf[t] = (qvalid && 16 * t + 8 * h < D) ? ld8<T>(Q + (int64_t)qtok * p.sq[2] + 16 * t + 8 * h) : zero_frag<T>();
    qn2 += sumsq8<T>(qf[t]);
  }
  qn2 = c * 0.5f * xhalf_sum(qn2);
  frag ones;
#pragma unroll
  for (int e = 0; e < 8; ++e) ones[e] = (T)1.f;

  f32x16_t oacc[ND];
  // this lane's share (16 of a block's 32 keys) of the sums of the rounded P
  // (normalises O) and of the unrounded P (gives L)
  float lrnd, lrow;
  float m_run;

  typedef TileFor<T, BN, DP, NT> TileT;
  TileT tk, tv;
  auto load_kv = [&](int kt) {
    const int tok0 = org + 32 * (kt * KB - kshift);
    tk.load(K, p.sk[2], tok0, N, D, tid);
    tv.load(V, p.sv[2], tok0, N, D, tid);
  };

  // One pass over the key tiles.  SAFE = online max with lazy rescaling.
  auto run = [&](auto safe_tag) {
    constexpr bool SAFE = decltype(safe_tag)::value;
#pragma unroll
    for (int d = 0; d < ND; ++d) oacc[d] = zero16();
    lrnd = 0.f;
    lrow = 0.f;
    m_run = !SOFTMAX ? qn2 : (SAFE ? -__builtin_inff() : qn2 - kBoundMargin);
    // The blocks of key tile kt against this wave's queries, from tiles kbuf
    // (K), vbuf (V, or V^T for fp32) and norms nbuf.
    auto tile = [&](int kt, const T* kbuf, const T* vbuf, const float* nbuf) {
      if (!wave_on) return;
      const int kblk0 = kt * KB - kshift;
#pragma unroll
      for (int kb = 0; kb < KB; ++kb) {
        const int k0 = org + 32 * (kblk0 + kb);
        if (!blk_any(q0, k0, causal, npre)) continue;
        frag kA[KS];
#pragma unroll
        for (int t = 0; t < KS; ++t) kA[t] = ld8<T>(kbuf + roff(32 * kb + n, 16 * t + 8 * h));
        f32x16_t s = ld_rows16(nbuf + 32 * kb, h);
#pragma unroll
        for (int t = 0; t < KS; ++t) s = E::mma(kA[t], qf[t], s);
        // V^T fragments are read while the S MFMAs and the softmax run.
        frag vA[ND][2];
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if constexpr (TR) vA[d][t] = TLy::tr(vbuf, 32 * kb + 16 * t, 32 * d, lane);
            else vA[d][t] = ld8<T>(vbuf + (32 * d + n) * LDT + tchunk<BN>(32 * d + n, 32 * kb + 16 * t + 8 * h));
          }
        if (!blk_nomask(q0, k0, causal, npre)) mask_key_rows(s, k0, h, jmax);
        if constexpr (SOFTMAX && SAFE) {
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
        const float moff = (SAFE && m_run == -__builtin_inff()) ? 0.f : m_run;
        frag pf[2];
        float pe[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          pe[i] = fast_exp2(fmaf(s[i], c, -moff));
          pf[i >> 3][i & 7] = (T)pe[i];
        }
        if constexpr (SOFTMAX) lrow += tree_sum16(pe);
        // With 128 features the wave issues its P V MFMAs at a raised
        // priority, ahead of the other wave's S chain and exponentials on the
        // SIMD: C3 forward 1172 -> 1151 us (D = 64, C4: within +0.4 %, off).
        if constexpr (DP == 128) __builtin_amdgcn_s_setprio(1);
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
          for (int d = 0; d < ND; ++d) oacc[d] = E::mma(vA[d][t], pf[t], oacc[d]);
        }
        if constexpr (SOFTMAX) lrnd += dot8<T>(pf[0], ones) + dot8<T>(pf[1], ones);
        if constexpr (DP == 128) __builtin_amdgcn_s_setprio(0);
      }
    };
    if constexpr (DMA) {
      auto tok0_of = [&](int kt) { return org + 32 * (kt * KB - kshift); };
      DmaPair<T, BN, DP, W> dma;
      dma.init(K, p.sk[2], V, p.sv[2], N, wave, lane);
      dma_pipeline(
          nkt, [&](int kt, int b) { dma.issue(tok0_of(kt), dK[b], dV[b]); },
          [&](int kt, int b) { tile_neg_halfnorms<T, BN, DP, NT>(dK[b], dN[b], tok0_of(kt), N, tid); },
          [&](int kt, int b) { tile(kt, dK[b], dV[b], dN[b]); });
    } else {
      load_kv(0);
      for (int kt = 0; kt < nkt; ++kt) {
        const int buf = kt & 1;
        if constexpr (TR) {
          TLy::store(tk, sK[buf], tid);
          TLy::store(tv, sVt[buf], tid);
        } else {
          tk.template store_rows<LDR>(sK[buf], tid);
          tv.template store_trans<LDT>(sVt[buf], tid);
        }
        tk.store_neg_halfnorm(sKn[buf], tid);
        __syncthreads();
        if (kt + 1 < nkt) load_kv(kt + 1);
        tile(kt, sK[buf], sVt[buf], sKn[buf]);
      }
    }
  };

  constexpr bool STATIC = SOFTMAX && !std::is_same<T, _Float16>::value;
  if constexpr (SOFTMAX && !STATIC) {
    run(std::true_type{});
  } else {
    run(std::false_type{});
  }
  if constexpr (STATIC) {
    const float l = xhalf_sum(lrow);
    const bool bad = qvalid && !(l >= kSumLow && l <= kSumHigh);
    if (__syncthreads_or(bad)) {
      __syncthreads();  // every wave is done reading the last tile
      run(std::true_type{});
    }
  }

  if (!wave_on) return;
  const float inv = SOFTMAX ? 1.f / xhalf_sum(lrnd) : 1.f;
  const float lsum = SOFTMAX ? xhalf_sum(lrow) : 1.f;
  if (qtok < 0) return;
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

// WPE asks the compiler for at least WPE waves per SIMD (register budget
// 512 / WPE): the binned 16-bit D <= 64 forward keeps three, as it has
// without the bin loop around its body.
template <typename T, int DP, int W, int BN, bool SOFTMAX, bool BIN = false,
          int WPE = (BIN && sizeof(T) == 2 && DP <= 64) ? 3 : 1, bool DMA = false>
__global__ __launch_bounds__(64 * W) __attribute__((amdgpu_waves_per_eu(WPE))) void rbf_fwd_kernel(const Params p) {
  for_each_group<BIN>(p, (p.nblk + W - 1) / W, p.causal != 0,
                 [&](int bh, int grp) { rbf_fwd_group<T, DP, W, BN, SOFTMAX, DMA>(p, bh, grp); });
}

// ---------------------------------------------------------------------------
// Backward, query-stationary: dQ.  A wave owns QPW query blocks.  Also
// produces, per query, Delta = rowsum(O*dO) (softmax) or the norm offset
// c*0.5*||q||^2 (non-softmax, written to the lse workspace), both consumed by
// the dK/dV kernel launched next.  K (row-major and transposed), V
// (row-major) and -0.5||k||^2 stream through LDS.
//   S^T = K Q^T (init -0.5||k||^2), P = exp2(c S^T - L),
//   dP^T = V dO^T (init -Delta), dS = P dP^T, dQ^T += K^T dS^T.
// ---------------------------------------------------------------------------
// DMA: K and V tiles staged by LDS-DMA (dma_pipeline; 16-bit, D = 64 or 128)
// instead of through registers.
template <typename T, int DP, int W, int QPW, int BN, bool SOFTMAX, bool EARLY = true, bool DMA = false>
__device__ __forceinline__ void rbf_bwd_dq_group(const Params& p, int bh, int grp) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  constexpr int NT = 64 * W, KB = BN / 32, KS = DP / 16, ND = DP / 32, GB = W * QPW;
  constexpr int LDR = DP + E::PAD, LDT = BN + E::PAD;
  // 16-bit types read K^T from the row-major K tile with transposing LDS
  // reads; fp32 stages a transposed copy.
  constexpr bool TR = sizeof(T) == 2;
  typedef TileLayout<T, BN, DP, DMA || kChunkMajor<T, DP>> TLy;
  static_assert(!DMA || TR, "LDS-DMA staging is for 16-bit tiles");
  constexpr int TSZ = TLy::SIZE;
  // register staging: two buffers each (a single element when DMA).  fp32
  // tiles of 256 features (K, K^T, V: 104 KB per buffer) fit LDS only once:
  // SB single-buffers them, with a barrier before each tile's stores.
  constexpr bool SB = !TR && DP > 128;
  constexpr int NB2 = (DMA || SB) ? 1 : 2;
  __shared__ __attribute__((aligned(16))) T sK[NB2][DMA ? 8 : TSZ];
  __shared__ __attribute__((aligned(16))) T sKt[TR ? 1 : NB2][TR ? 8 : DP * LDT];
  __shared__ __attribute__((aligned(16))) T sV[NB2][DMA ? 8 : TSZ];
  auto roff = [](int row, int col) { return TLy::off(row, col); };
  __shared__ __attribute__((aligned(16))) float sKn[NB2][DMA ? 1 : BN];
  // LDS-DMA staging: three buffers each (a single element without DMA)
  constexpr int NB3 = DMA ? 3 : 1;
  __shared__ __attribute__((aligned(16))) T dK[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) T dV[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) float dN[NB3][DMA ? BN : 1];

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const int ngrp = (nblk + GB - 1) / GB;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  const T* Og = reinterpret_cast<const T*>(p.o) + b * p.so[0] + hh * p.so[1];
  const T* dO = reinterpret_cast<const T*>(p.dout) + b * p.sdo[0] + hh * p.sdo[1];
  T* dQ = reinterpret_cast<T*>(p.dq) + b * p.sdq[0] + hh * p.sdq[1];

  const int blk0 = nblk - (ngrp - grp) * GB;
  const int qblk0 = blk0 + wave * QPW;
  const bool wave_on = qblk0 + QPW - 1 >= 0;
  const int wg_qlast = org + 32 * (blk0 + GB) - 1;
  int hi = causal ? max(wg_qlast + 1, npre) : N;
  hi = min(hi, N);
  const int nkt_all = (nblk + KB - 1) / KB;
  const int kshift = nkt_all * KB - nblk;
  const int last_blk = (hi - 1 - org) >> 5;
  const int nkt = (last_blk + kshift) / KB + 1;

  int q0[QPW], qtok[QPW], jmax[QPW];
  frag qf[QPW][KS], df[QPW][KS];
  float off[QPW];
  f32x16_t ndel[QPW];  // -Delta broadcast: the dP accumulator's initial value
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    q0[j] = org + 32 * (qblk0 + j);
    qtok[j] = q0[j] + n;
    jmax[j] = last_key(qtok[j], N, causal, npre);
    const bool qvalid = wave_on && qtok[j] >= 0;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool ok = qvalid && 16 * t + 8 * h < D;
      qf[j][t] = ok ? ld8<T>(Q + (int64_t)qtok[j] * p.sq[2] + 16 * t + 8 * h) : zero_frag<T>();
      df[j][t] = ok ? ld8<T>(dO + (int64_t)qtok[j] * p.sdo[2] + 16 * t + 8 * h) : zero_frag<T>();
    }
    float dlt = 0.f;
    if constexpr (SOFTMAX) {
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        const bool ok = qvalid && 16 * t + 8 * h < D;
        const frag of = ok ? ld8<T>(Og + (int64_t)qtok[j] * p.so[2] + 16 * t + 8 * h) : zero_frag<T>();
        s += dot8<T>(of, df[j][t]);
      }
      s = xhalf_sum(s);
      dlt = s;
      off[j] = qvalid ? p.lse[(int64_t)bh * N + qtok[j]] : 0.f;
      if (qvalid && h == 0) p.delta[(int64_t)bh * N + qtok[j]] = dlt;
    } else {
      float s = 0.f;
#pragma unroll
      for (int t = 0; t < KS; ++t) s += sumsq8<T>(qf[j][t]);
      s = xhalf_sum(s);
      off[j] = c * 0.5f * s;
      if (qvalid && h == 0) p.lse[(int64_t)bh * N + qtok[j]] = off[j];
    }
    ndel[j] = SOFTMAX ? splat16(-dlt) : zero16();  // +0: the MFMA's inline constant, no copies
  }

  f32x16_t dqacc[QPW][ND];
  float rsum[QPW];
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
#pragma unroll
    for (int d = 0; d < ND; ++d) dqacc[j][d] = zero16();
    rsum[j] = 0.f;
  }

  // The blocks of key tile kt against this wave's queries, from tiles kbuf
  // (K), ktbuf (K^T, fp32 only), vbuf (V) and norms nbuf.
  auto tile = [&](int kt, const T* kbuf, const T* ktbuf, const T* vbuf, const float* nbuf) {
    if (!wave_on) return;
    const int kblk0 = kt * KB - kshift;
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
      const int k0 = org + 32 * (kblk0 + kb);
      bool act[QPW];
      bool any = false;
#pragma unroll
      for (int j = 0; j < QPW; ++j) {
        act[j] = blk_any(q0[j], k0, causal, npre);
        any = any || act[j];
      }
      if (!any) continue;
      frag kA[KS], vA[KS];
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        kA[t] = ld8<T>(kbuf + roff(32 * kb + n, 16 * t + 8 * h));
        vA[t] = ld8<T>(vbuf + roff(32 * kb + n, 16 * t + 8 * h));
      }
      const f32x16_t kinit = ld_rows16(nbuf + 32 * kb, h);
      f32x16_t sacc[QPW], dpacc[QPW];
#pragma unroll
      for (int j = 0; j < QPW; ++j) {
        if (!act[j]) continue;
        sacc[j] = kinit;
        dpacc[j] = ndel[j];
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          sacc[j] = E::mma(kA[t], qf[j][t], sacc[j]);
          dpacc[j] = E::mma(vA[t], df[j][t], dpacc[j]);
        }
      }
      // K^T fragments are read while the S / dP MFMAs and the softmax run
      // (EARLY), or next to the dQ MFMAs.
      frag ktA[ND][2];
      auto read_kt = [&]() {
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if constexpr (TR) ktA[d][t] = TLy::tr(kbuf, 32 * kb + 16 * t, 32 * d, lane);
            else ktA[d][t] = ld8<T>(ktbuf + (32 * d + n) * LDT + tchunk<BN>(32 * d + n, 32 * kb + 16 * t + 8 * h));
          }
      };
      if constexpr (EARLY) read_kt();
      frag sf[QPW][2];
#pragma unroll
      for (int j = 0; j < QPW; ++j) {
        if (!act[j]) continue;
        f32x16_t s = sacc[j];
        const f32x16_t dp = dpacc[j];
        if (!blk_nomask(q0[j], k0, causal, npre)) mask_key_rows(s, k0, h, jmax[j]);
        float ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          ds[i] = fast_exp2(fmaf(s[i], c, -off[j])) * dp[i];
          sf[j][i >> 3][i & 7] = (T)ds[i];
        }
        if constexpr (!SOFTMAX) rsum[j] += tree_sum16(ds);
      }
      if constexpr (!EARLY) read_kt();
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int j = 0; j < QPW; ++j)
            if (act[j]) dqacc[j][d] = E::mma(ktA[d][t], sf[j][t], dqacc[j][d]);
    }
  };

  auto tok0_of = [&](int kt) { return org + 32 * (kt * KB - kshift); };
  if constexpr (DMA) {
    DmaPair<T, BN, DP, W> dma;
    dma.init(K, p.sk[2], V, p.sv[2], N, wave, lane);
    dma_pipeline(
        nkt, [&](int kt, int b) { dma.issue(tok0_of(kt), dK[b], dV[b]); },
        [&](int kt, int b) { tile_neg_halfnorms<T, BN, DP, NT>(dK[b], dN[b], tok0_of(kt), N, tid); },
        [&](int kt, int b) { tile(kt, dK[b], nullptr, dV[b], dN[b]); });
  } else {
    TileFor<T, BN, DP, NT> tk, tv;
    tk.load(K, p.sk[2], tok0_of(0), N, D, tid);
    tv.load(V, p.sv[2], tok0_of(0), N, D, tid);
    for (int kt = 0; kt < nkt; ++kt) {
      const int buf = SB ? 0 : (kt & 1);
      if (SB && kt > 0) __syncthreads();  // every wave is done with tile kt - 1
      if constexpr (TR) {
        TLy::store(tk, sK[buf], tid);
        TLy::store(tv, sV[buf], tid);
      } else {
        tk.template store_rows<LDR>(sK[buf], tid);
        tk.template store_trans<LDT>(sKt[buf], tid);
        tv.template store_rows<LDR>(sV[buf], tid);
      }
      tk.store_neg_halfnorm(sKn[buf], tid);
      __syncthreads();
      if (kt + 1 < nkt) {
        tk.load(K, p.sk[2], tok0_of(kt + 1), N, D, tid);
        tv.load(V, p.sv[2], tok0_of(kt + 1), N, D, tid);
      }
      tile(kt, sK[buf], sKt[TR ? 0 : buf], sV[buf], sKn[buf]);
    }
  }

  if (!wave_on) return;
  const float g2 = 2.f * p.gamma;
#pragma unroll
  for (int j = 0; j < QPW; ++j) {
    float rs = 0.f;
    if constexpr (!SOFTMAX) rs = xhalf_sum(rsum[j]);
    if (qtok[j] < 0) continue;
    T* drow = dQ + (int64_t)qtok[j] * p.sdq[2];
    const T* qrow = Q + (int64_t)qtok[j] * p.sq[2];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = 32 * d + 8 * g + 4 * h;
        if (dd < D) {
          float v4[4];
          if constexpr (SOFTMAX) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = g2 * dqacc[j][d][4 * g + e];
          } else {
            float q4[4];
            ld4f<T>(qrow + dd, q4);
#pragma unroll
            for (int e = 0; e < 4; ++e) v4[e] = g2 * (dqacc[j][d][4 * g + e] - rs * q4[e]);
          }
          st4f<T>(drow + dd, v4);
        }
      }
  }
}

template <typename T, int DP, int W, int QPW, int BN, bool SOFTMAX, bool EARLY = true, bool BIN = false,
          bool DMA = false>
__global__ __launch_bounds__(64 * W) void rbf_bwd_dq_kernel(const Params p) {
  for_each_group<BIN>(p, (p.nblk + W * QPW - 1) / (W * QPW), p.causal != 0,
                 [&](int bh, int grp) { rbf_bwd_dq_group<T, DP, W, QPW, BN, SOFTMAX, EARLY, DMA>(p, bh, grp); });
}

// ---------------------------------------------------------------------------
// Backward, key-stationary: dK and dV.  A wave owns KPW key blocks (K and V
// fragments in registers); BM-query tiles of Q and dO (row-major and
// transposed), the per-query offset -L/c (or -0.5||q||^2) and -Delta stream
// through LDS.  Per 32-query block the wave reads the Q, dO fragments and the
// offsets once and reuses them for its KPW key blocks:
//   S = Q K^T (init -L/c), P = exp2(c S - c*0.5||k||^2),
//   dP = dO V^T (init -Delta), dS = P dP,
//   dV^T += dO^T P, dK^T += Q^T dS, colsum += sum_i dS.
// ---------------------------------------------------------------------------
// DMA: Q and dO tiles, and the raw L and Delta rows, staged by LDS-DMA
// (dma_pipeline; 16-bit, D = DP only).
template <typename T, int DP, int W, int KPW, int BM, bool SOFTMAX, bool EARLY = true, bool PIPE = false,
          bool PRIO = false, bool DMA = false>
__device__ __forceinline__ void rbf_bwd_dkdv_group(const Params& p, int bh, int grp) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  constexpr int NT = 64 * W, QB = BM / 32, KS = DP / 16, ND = DP / 32, GB = W * KPW;
  constexpr int LDR = DP + E::PAD, LDT = BM + E::PAD;
  // 16-bit types read Q^T and dO^T from the row-major tiles with transposing
  // LDS reads; fp32 stages transposed copies.
  constexpr bool TR = sizeof(T) == 2;
  typedef TileLayout<T, BM, DP, DMA || kChunkMajor<T, DP>> TLy;
  static_assert(!DMA || (TR && BM % 64 == 0), "LDS-DMA staging: 16-bit tiles of whole 64-row groups");
  constexpr int TSZ = TLy::SIZE;
  // register staging: two buffers each; LDS-DMA staging: three (the other
  // form's arrays shrink to a single element).  fp32 tiles of 256 features
  // (Q, Q^T, dO, dO^T: 140 KB per buffer) fit LDS only once: SB
  // single-buffers them, with a barrier before each tile's stores.
  constexpr bool SB = !TR && DP > 128;
  constexpr int NB2 = (DMA || SB) ? 1 : 2, NB3 = DMA ? 3 : 1;
  __shared__ __attribute__((aligned(16))) T sQ[NB2][DMA ? 8 : TSZ];
  __shared__ __attribute__((aligned(16))) T sQt[TR ? 1 : NB2][TR ? 8 : DP * LDT];
  __shared__ __attribute__((aligned(16))) T sD[NB2][DMA ? 8 : TSZ];
  auto roff = [](int row, int col) { return TLy::off(row, col); };
  __shared__ __attribute__((aligned(16))) T sDt[TR ? 1 : NB2][TR ? 8 : DP * LDT];
  __shared__ __attribute__((aligned(16))) float sOff[NB2][DMA ? 1 : BM];
  __shared__ __attribute__((aligned(16))) float sDel[NB2][DMA ? 1 : BM];
  __shared__ __attribute__((aligned(16))) T dQt[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) T dDt[NB3][DMA ? TSZ : 8];
  __shared__ __attribute__((aligned(16))) float dOff[NB3][DMA ? BM : 1];
  __shared__ __attribute__((aligned(16))) float dDel[NB3][DMA ? BM : 1];
  __shared__ __attribute__((aligned(16))) float dRaw[NB3][2][DMA ? BM : 1];  // L, Delta as loaded

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const float inv_c = 1.f / c;
  const int ngrp = (nblk + GB - 1) / GB;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  const T* dO = reinterpret_cast<const T*>(p.dout) + b * p.sdo[0] + hh * p.sdo[1];
  T* dK = reinterpret_cast<T*>(p.dk) + b * p.sdk[0] + hh * p.sdk[1];
  T* dV = reinterpret_cast<T*>(p.dv) + b * p.sdv[0] + hh * p.sdv[1];
  const float* offg = p.lse + (int64_t)bh * N;
  const float* delg = SOFTMAX ? p.delta + (int64_t)bh * N : nullptr;

  // Key groups are aligned to the start of the sequence (group g holds blocks
  // [g GB, g GB + GB)): the heaviest causal group is then a full one, and the
  // one group that may hold fewer real blocks is the lightest (aligned to the
  // end, it was the heaviest, with most of its waves idle).
  const int blk0 = grp * GB;
  const int kblk0 = blk0 + wave * KPW;
  const bool wave_on = kblk0 < nblk;

  int k0[KPW], ktok[KPW], ilo[KPW];
  frag kf[KPW][KS], vf[KPW][KS];
  float nckn[KPW];  // -c * 0.5||k||^2
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    k0[j] = org + 32 * (kblk0 + j);
    ktok[j] = k0[j] + n;
    ilo[j] = first_query(ktok[j], causal, npre);
    const bool kvalid = wave_on && ktok[j] >= 0 && ktok[j] < N;
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const bool ok = kvalid && 16 * t + 8 * h < D;
      kf[j][t] = ok ? ld8<T>(K + (int64_t)ktok[j] * p.sk[2] + 16 * t + 8 * h) : zero_frag<T>();
      vf[j][t] = ok ? ld8<T>(V + (int64_t)ktok[j] * p.sv[2] + 16 * t + 8 * h) : zero_frag<T>();
      s += sumsq8<T>(kf[j][t]);
    }
    s = xhalf_sum(s);
    nckn[j] = -c * 0.5f * s;
  }

  f32x16_t dkacc[KPW][ND], dvacc[KPW][ND];
  float csum[KPW];
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
#pragma unroll
    for (int d = 0; d < ND; ++d) {
      dkacc[j][d] = zero16();
      dvacc[j][d] = zero16();
    }
    csum[j] = 0.f;
  }

  // Query range: causal keys are seen by queries at or after them, except
  // prefix (register) keys, which every query sees.
  const int wg_kfirst = max(org + 32 * max(blk0, 0), 0);
  const int qlo = causal ? (wg_kfirst < npre ? 0 : wg_kfirst) : 0;
  const int nqt_all = (nblk + QB - 1) / QB;
  const int qshift = nqt_all * QB - nblk;
  const int qt_lo = (((qlo - org) >> 5) + qshift) / QB;

  TileFor<T, BM, DP, NT> tq, td;
  float offr = 0.f, delr = 0.f;
  auto load_tile = [&](int qt) {
    const int tok0 = org + 32 * (qt * QB - qshift);
    tq.load(Q, p.sq[2], tok0, N, D, tid);
    td.load(dO, p.sdo[2], tok0, N, D, tid);
    if (tid < BM) {
      const int tok = tok0 + tid;
      const bool ok = tok >= 0 && tok < N;
      offr = ok ? -offg[tok] * inv_c : -__builtin_inff();  // padding queries: P = 0
      if constexpr (SOFTMAX) delr = ok ? -delg[tok] : 0.f;
    }
  };
  // Query tile qt against this wave's key blocks, from tiles sQb (Q), sDb
  // (dO), sQtb / sDtb (their transposes, fp32 only) and per-query terms offb
  // (-L/c), delb (-Delta).
  auto tile = [&](int qt, const T* sQb, const T* sDb, const T* sQtb, const T* sDtb, const float* offb,
                  const float* delb) {
    if (!wave_on) return;
    const int qblk0 = qt * QB - qshift;
    if constexpr (PIPE && KPW == 1) {
      // Fast path for tiles whose every (query block, key block) pair is fully
      // visible to this wave (the interior of the causal triangle): no
      // branches, and software-pipelined -- the S and dP MFMAs of all QB
      // blocks are issued first, so block qb's elementwise work overlaps the
      // MFMAs of block qb+1 and the dV/dK MFMAs of block qb-1.
      bool fast = true;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        const int q0 = org + 32 * (qblk0 + qb);
        fast = fast && blk_any(q0, k0[0], causal, npre) && blk_nomask(q0, k0[0], causal, npre);
      }
      if (fast) {
        f32x16_t sacc[QB], dpacc[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          sacc[qb] = ld_rows16(offb + 32 * qb, h);
          if constexpr (SOFTMAX) dpacc[qb] = ld_rows16(delb + 32 * qb, h);
          else dpacc[qb] = zero16();
#pragma unroll
          for (int t = 0; t < KS; ++t) {
            const frag qA = ld8<T>(sQb + roff(32 * qb + n, 16 * t + 8 * h));
            const frag dA = ld8<T>(sDb + roff(32 * qb + n, 16 * t + 8 * h));
            sacc[qb] = E::mma(qA, kf[0][t], sacc[qb]);
            dpacc[qb] = E::mma(dA, vf[0][t], dpacc[qb]);
          }
        }
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          frag pf[2], sf[2];
          float ds[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float pv = fast_exp2(fmaf(sacc[qb][i], c, nckn[0]));
            ds[i] = pv * dpacc[qb][i];
            pf[i >> 3][i & 7] = (T)pv;
            sf[i >> 3][i & 7] = (T)ds[i];
          }
          csum[0] += tree_sum16(ds);
#pragma unroll
          for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int t = 0; t < 2; ++t) {
              frag dtA, qtA;
              if constexpr (TR) {
                dtA = TLy::tr(sDb, 32 * qb + 16 * t, 32 * d, lane);
                qtA = TLy::tr(sQb, 32 * qb + 16 * t, 32 * d, lane);
              } else {
                const int o = (32 * d + n) * LDT + tchunk<BM>(32 * d + n, 32 * qb + 16 * t + 8 * h);
                dtA = ld8<T>(sDtb + o);
                qtA = ld8<T>(sQtb + o);
              }
              dvacc[0][d] = E::mma(dtA, pf[t], dvacc[0][d]);
              dkacc[0][d] = E::mma(qtA, sf[t], dkacc[0][d]);
            }
        }
        return;
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      const int q0 = org + 32 * (qblk0 + qb);
      bool act[KPW];
      bool any = false;
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        act[j] = blk_any(q0, k0[j], causal, npre);
        any = any || act[j];
      }
      if (!any) continue;
      frag qA[KS], dA[KS];
#pragma unroll
      for (int t = 0; t < KS; ++t) {
        qA[t] = ld8<T>(sQb + roff(32 * qb + n, 16 * t + 8 * h));
        dA[t] = ld8<T>(sDb + roff(32 * qb + n, 16 * t + 8 * h));
      }
      const f32x16_t oinit = ld_rows16(offb + 32 * qb, h);
      f32x16_t dinit;
      if constexpr (SOFTMAX) dinit = ld_rows16(delb + 32 * qb, h);
      else dinit = zero16();
      f32x16_t sacc[KPW], dpacc[KPW];
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        if (!act[j]) continue;
        sacc[j] = oinit;
        dpacc[j] = dinit;
#pragma unroll
        for (int t = 0; t < KS; ++t) {
          sacc[j] = E::mma(qA[t], kf[j][t], sacc[j]);
          dpacc[j] = E::mma(dA[t], vf[j][t], dpacc[j]);
        }
      }
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
      // dO^T and Q^T fragments are read while the S / dP MFMAs and the
      // elementwise work run.
      frag dtA[ND][2], qtA[ND][2];
      auto read_t = [&]() {
#pragma unroll
        for (int d = 0; d < ND; ++d)
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if constexpr (TR) {
              dtA[d][t] = TLy::tr(sDb, 32 * qb + 16 * t, 32 * d, lane);
              qtA[d][t] = TLy::tr(sQb, 32 * qb + 16 * t, 32 * d, lane);
            } else {
              const int o = (32 * d + n) * LDT + tchunk<BM>(32 * d + n, 32 * qb + 16 * t + 8 * h);
              dtA[d][t] = ld8<T>(sDtb + o);
              qtA[d][t] = ld8<T>(sQtb + o);
            }
          }
      };
      if constexpr (EARLY) read_t();
      frag pf[KPW][2], sf[KPW][2];
#pragma unroll
      for (int j = 0; j < KPW; ++j) {
        if (!act[j]) continue;
        f32x16_t s = sacc[j];
        const f32x16_t dp = dpacc[j];
        if (!blk_nomask(q0, k0[j], causal, npre)) mask_query_rows(s, q0, h, ilo[j]);
        float ds[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const float pv = fast_exp2(fmaf(s[i], c, nckn[j]));
          ds[i] = pv * dp[i];
          pf[j][i >> 3][i & 7] = (T)pv;
          sf[j][i >> 3][i & 7] = (T)ds[i];
        }
        csum[j] += tree_sum16(ds);
      }
      if constexpr (!EARLY) read_t();
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int d = 0; d < ND; ++d)
#pragma unroll
        for (int t = 0; t < 2; ++t)
#pragma unroll
          for (int j = 0; j < KPW; ++j)
            if (act[j]) {
              dvacc[j][d] = E::mma(dtA[d][t], pf[j][t], dvacc[j][d]);
              dkacc[j][d] = E::mma(qtA[d][t], sf[j][t], dkacc[j][d]);
            }
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    }
  };
  if constexpr (DMA) {
    // The tile's raw L and Delta are DMA'd with it (the last wave issues
    // them) and turned into -L/c and -Delta by the first waves once landed.
    DmaPair<T, BM, DP, W> dma;
    dma.init(Q, p.sq[2], dO, p.sdo[2], N, wave, lane);
    const i32x4_t roffr = buffer_rsrc(offg, 4u * (uint32_t)N);
    const i32x4_t rdelr = buffer_rsrc(SOFTMAX ? delg : offg, 4u * (uint32_t)N);
    auto tok0_of = [&](int qt) { return org + 32 * (qt * QB - qshift); };
    dma_pipeline(
        nqt_all - qt_lo,
        [&](int t, int b) {
          const int tok0 = tok0_of(qt_lo + t);
          dma.issue(tok0, dQt[b], dDt[b]);
          if (wave == W - 1) {
#pragma unroll
            for (int r = 0; r < BM / 64; ++r) {
              const uint32_t vo = 4u * (uint32_t)(tok0 + 64 * r + lane);  // negative tokens: out of range
              dma4(vo, roffr, lds_addr(&dRaw[b][0][64 * r]));
              if constexpr (SOFTMAX) dma4(vo, rdelr, lds_addr(&dRaw[b][1][64 * r]));
            }
          }
        },
        [&](int t, int b) {
          if (tid < BM) {
            const int tok = tok0_of(qt_lo + t) + tid;
            const bool ok = tok >= 0 && tok < N;
            dOff[b][tid] = ok ? -dRaw[b][0][tid] * inv_c : -__builtin_inff();  // padding queries: P = 0
            dDel[b][tid] = (SOFTMAX && ok) ? -dRaw[b][1][tid] : 0.f;
          }
        },
        [&](int t, int b) { tile(qt_lo + t, dQt[b], dDt[b], nullptr, nullptr, dOff[b], dDel[b]); });
  } else {
    load_tile(qt_lo);
    for (int qt = qt_lo; qt < nqt_all; ++qt) {
      const int buf = SB ? 0 : (qt & 1);
      if (SB && qt > qt_lo) __syncthreads();  // every wave is done with tile qt - 1
      if constexpr (TR) {
        TLy::store(tq, sQ[buf], tid);
        TLy::store(td, sD[buf], tid);
      } else {
        tq.template store_rows<LDR>(sQ[buf], tid);
        td.template store_rows<LDR>(sD[buf], tid);
        tq.template store_trans<LDT>(sQt[buf], tid);
        td.template store_trans<LDT>(sDt[buf], tid);
      }
      if (tid < BM) {
        sOff[buf][tid] = offr;
        sDel[buf][tid] = delr;
      }
      __syncthreads();
      if (qt + 1 < nqt_all) load_tile(qt + 1);
      tile(qt, sQ[buf], sD[buf], sQt[TR ? 0 : buf], sDt[TR ? 0 : buf], sOff[buf], sDel[buf]);
    }
  }

  if (!wave_on) return;
  const float g2 = 2.f * p.gamma;
#pragma unroll
  for (int j = 0; j < KPW; ++j) {
    const float cs = xhalf_sum(csum[j]);
    if (ktok[j] < 0 || ktok[j] >= N) continue;
    T* dkrow = dK + (int64_t)ktok[j] * p.sdk[2];
    T* dvrow = dV + (int64_t)ktok[j] * p.sdv[2];
    const T* krow = K + (int64_t)ktok[j] * p.sk[2];
#pragma unroll
    for (int d = 0; d < ND; ++d)
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int dd = 32 * d + 8 * g + 4 * h;
        if (dd < D) {
          float k4[4], a4[4], b4[4];
          ld4f<T>(krow + dd, k4);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            a4[e] = g2 * (dkacc[j][d][4 * g + e] - cs * k4[e]);
            b4[e] = dvacc[j][d][4 * g + e];
          }
          st4f<T>(dkrow + dd, a4);
          st4f<T>(dvrow + dd, b4);
        }
      }
  }
}

template <typename T, int DP, int W, int KPW, int BM, bool SOFTMAX, bool EARLY = true, bool PIPE = false,
          bool PRIO = false, bool BIN = false, bool DMA = false>
__global__ __launch_bounds__(64 * W) void rbf_bwd_dkdv_kernel(const Params p) {
  for_each_group<BIN>(p, (p.nblk + W * KPW - 1) / (W * KPW), false,
                 [&](int bh, int grp) { rbf_bwd_dkdv_group<T, DP, W, KPW, BM, SOFTMAX, EARLY, PIPE, PRIO, DMA>(p, bh, grp); });
}

// ---------------------------------------------------------------------------
// Backward, key-stationary, two waves per key block (16-bit types).  A
// work-group holds NP key blocks and 2*NP waves: wave j (< NP) is the P-wave
// of key block j, wave NP + j its dS-wave, and the hardware places the two on
// the same SIMD.  Each holds half of the key block's state (K and dV, or V and
// dK), which halves the registers per wave and lets the exponential work of
// one wave overlap the MFMAs of the other.  Per BM-query tile:
//   phase 1  P-wave:  S = Q K^T (init -L/c), P = exp2(c S - c*0.5||k||^2),
//                     P -> LDS
//            dS-wave: dP = dO V^T (init -Delta)
//   barrier
//   phase 2  P-wave:  dV^T += dO^T P
//            dS-wave: dS = P dP with P from LDS, dK^T += Q^T dS, colsum += dS
// P reaches the dS-wave in fp32 (four float4 planes of 64 lanes each, so
// every 16-byte LDS access of a wave is contiguous), as the one-wave kernels
// form dS: dS and its column sum then carry no rounding of P, which only the
// dV product sees (rounded to the element type, as in the reference).  With P
// handed over in the element type instead, dK's relative L2 error at C3 was
// 1.25x that of the reference's own rounding.  SGB: every 32-query block
// issues its LDS operand reads ahead of its MFMAs (sched_group_barrier: all
// of them before the S / dP products, in two halves before the dV / dK
// products), trading registers for hidden LDS latency.
// ---------------------------------------------------------------------------
// DMA: Q and dO tiles staged by LDS-DMA (dma_pipeline; the launcher uses it at D = 128), the
// per-query offsets through two registers of the first wave.
template <typename T, int DP, int NP, int BM, bool SOFTMAX, bool SGB = false, bool DMA = false>
__device__ __forceinline__ void rbf_bwd_dkdv_pair_group(const Params& p, int bh, int grp) {
  typedef Elem<T> E;
  typedef typename E::frag frag;
  static_assert(sizeof(T) == 2, "the paired kernel reads transposed operands with ds_read_b64_tr_b16");
  constexpr int W = 2 * NP, NT = 64 * W, QB = BM / 32, KS = DP / 16, ND = DP / 32;
  typedef TileLayout<T, BM, DP> TLy;
  static_assert(!DMA || TLy::CM, "LDS-DMA staging is for chunk-major tiles");
  // register staging: two buffers each; LDS-DMA staging: three (the other
  // form's arrays shrink to a single element)
  constexpr int NB2 = DMA ? 1 : 2, NB3 = DMA ? 3 : 1;
  __shared__ __attribute__((aligned(16))) T sQ[NB2][DMA ? 8 : TLy::SIZE];
  __shared__ __attribute__((aligned(16))) T sD[NB2][DMA ? 8 : TLy::SIZE];
  __shared__ __attribute__((aligned(16))) float sOff[NB2][DMA ? 1 : BM];
  __shared__ __attribute__((aligned(16))) float sDel[NB2][DMA ? 1 : BM];
  __shared__ __attribute__((aligned(16))) T dQt[NB3][DMA ? TLy::SIZE : 8];
  __shared__ __attribute__((aligned(16))) T dDt[NB3][DMA ? TLy::SIZE : 8];
  __shared__ __attribute__((aligned(16))) float dOff[NB3][DMA ? BM : 1];
  __shared__ __attribute__((aligned(16))) float dDel[NB3][DMA ? BM : 1];
  __shared__ __attribute__((aligned(16))) float dRaw[NB3][2][DMA ? BM : 1];  // L, Delta as loaded
  __shared__ __attribute__((aligned(16))) f32x4_t sP[NP][QB][4][64];

  const int tid = threadIdx.x, lane = tid & 63, n = lane & 31, h = lane >> 5;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bool pwave = wave < NP;
  const int j = pwave ? wave : wave - NP;
  const int N = p.N, D = p.D, org = p.org, nblk = p.nblk;
  const bool causal = p.causal != 0;
  const int npre = p.num_prefix;
  const float c = p.c;
  const float inv_c = 1.f / c;
  const int ngrp = (nblk + NP - 1) / NP;
  const int b = bh / p.H, hh = bh - b * p.H;
  const T* Q = reinterpret_cast<const T*>(p.q) + b * p.sq[0] + hh * p.sq[1];
  const T* K = reinterpret_cast<const T*>(p.k) + b * p.sk[0] + hh * p.sk[1];
  const T* V = reinterpret_cast<const T*>(p.v) + b * p.sv[0] + hh * p.sv[1];
  const T* dO = reinterpret_cast<const T*>(p.dout) + b * p.sdo[0] + hh * p.sdo[1];
  const float* offg = p.lse + (int64_t)bh * N;
  const float* delg = SOFTMAX ? p.delta + (int64_t)bh * N : nullptr;

  // start-aligned key groups, as in rbf_bwd_dkdv_group
  const int blk0 = grp * NP;
  const int kblk = blk0 + j;
  const bool wave_on = kblk < nblk;
  const int k0 = org + 32 * kblk;
  const int ktok = k0 + n;
  const bool kvalid = wave_on && ktok >= 0;
  const int ilo = first_query(ktok, causal, npre);

  // P-wave: K fragments and -c*0.5||k||^2; dS-wave: V fragments.
  frag kv[KS];
  float nckn = 0.f;
  {
    const T* src = pwave ? K + (int64_t)ktok * p.sk[2] : V + (int64_t)ktok * p.sv[2];
    float s = 0.f;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      kv[t] = (kvalid && 16 * t + 8 * h < D) ? ld8<T>(src + 16 * t + 8 * h) : zero_frag<T>();
      s += sumsq8<T>(kv[t]);
    }
    nckn = -c * 0.5f * xhalf_sum(s);
  }

  f32x16_t acc[ND];  // dV^T (P-wave) or dK^T (dS-wave)
#pragma unroll
  for (int d = 0; d < ND; ++d) acc[d] = zero16();
  float csum = 0.f;

  const int wg_kfirst = max(org + 32 * max(blk0, 0), 0);
  const int qlo = causal ? (wg_kfirst < npre ? 0 : wg_kfirst) : 0;
  const int nqt_all = (nblk + QB - 1) / QB;
  const int qshift = nqt_all * QB - nblk;
  const int qt_lo = (((qlo - org) >> 5) + qshift) / QB;

  TileFor<T, BM, DP, NT> tq, td;
  float offr = 0.f, delr = 0.f;
  auto load_tile = [&](int qt) {
    const int tok0 = org + 32 * (qt * QB - qshift);
    tq.load(Q, p.sq[2], tok0, N, D, tid);
    td.load(dO, p.sdo[2], tok0, N, D, tid);
    if (tid < BM) {
      const int tok = tok0 + tid;
      const bool ok = tok >= 0 && tok < N;
      offr = ok ? -offg[tok] * inv_c : -__builtin_inff();  // padding queries: P = 0
      if constexpr (SOFTMAX) delr = ok ? -delg[tok] : 0.f;
    }
  };
  // The two roles run separate copies of the tile loop (same trip count, same
  // two barriers per tile), so that the compiler allocates registers for each
  // role on its own.
  auto tile_loop = [&](auto role) {
    constexpr bool PW = decltype(role)::value;
    // Query tile qt from tiles sQb (Q), sDb (dO) and per-query terms offb
    // (-L/c), delb (-Delta); the mid-tile barrier hands P to the dS-waves.
    auto compute = [&](int qt, const T* sQb, const T* sDb, const float* offb, const float* delb) {
      const int qblk0 = qt * QB - qshift;
      bool act[QB];
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) act[qb] = wave_on && blk_any(org + 32 * (qblk0 + qb), k0, causal, npre);
      // Each role runs at a raised issue priority in the phase where its path
      // is the longer one (the P-wave's S chain, exponentials and P stores;
      // the dS-wave's P read, dS and dK), so that the other wave's MFMAs fill
      // its gaps rather than delay it: C3 dK/dV 2277 -> 2254 us.
      if constexpr (PW) {
        // phase 1: S, P -> registers and LDS
        __builtin_amdgcn_s_setprio(2);
        frag pf[QB][2];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (!act[qb]) continue;
          const int q0 = org + 32 * (qblk0 + qb);
          f32x16_t s = ld_rows16(offb + 32 * qb, h);
#pragma unroll
          for (int t = 0; t < KS; ++t) s = E::mma(ld8<T>(sQb + TLy::off(32 * qb + n, 16 * t + 8 * h)), kv[t], s);
          if constexpr (SGB) {
            __builtin_amdgcn_sched_group_barrier(0x100, KS + 4, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);
          }
          if (!blk_nomask(q0, k0, causal, npre)) mask_query_rows(s, q0, h, ilo);
          f32x4_t pv[4];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const float e = fast_exp2(fmaf(s[i], c, nckn));
            pv[i >> 2][i & 3] = e;
            pf[qb][i >> 3][i & 7] = (T)e;
          }
#pragma unroll
          for (int u = 0; u < 4; ++u) sP[j][qb][u][lane] = pv[u];
        }
        __builtin_amdgcn_s_setprio(0);
        if constexpr (DMA) lds_barrier();
        else __syncthreads();
        // phase 2: dV^T += dO^T P
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (!act[qb]) continue;
#pragma unroll
          for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[d] = E::mma(TLy::tr(sDb, 32 * qb + 16 * t, 32 * d, lane), pf[qb][t], acc[d]);
          if constexpr (SGB) {
            // in two halves: C3 dK/dV -2.0 % against all reads before all
            // MFMAs (quarters: -0.4 %, two reads per MFMA: +0.1 %)
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
          }
        }
      } else {
        // phase 1: dP
        f32x16_t dpacc[QB];
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (!act[qb]) continue;
          f32x16_t dp;
          if constexpr (SOFTMAX) dp = ld_rows16(delb + 32 * qb, h);
          else dp = zero16();
#pragma unroll
          for (int t = 0; t < KS; ++t) dp = E::mma(ld8<T>(sDb + TLy::off(32 * qb + n, 16 * t + 8 * h)), kv[t], dp);
          dpacc[qb] = dp;
          if constexpr (SGB) {
            __builtin_amdgcn_sched_group_barrier(0x100, KS + (SOFTMAX ? 4 : 0), 0);
            __builtin_amdgcn_sched_group_barrier(0x008, KS, 0);
          }
        }
        if constexpr (DMA) lds_barrier();
        else __syncthreads();
        __builtin_amdgcn_s_setprio(2);
        // phase 2: dS = P dP, dK^T += Q^T dS
#pragma unroll
        for (int qb = 0; qb < QB; ++qb) {
          if (!act[qb]) continue;
          f32x4_t pv[4];
#pragma unroll
          for (int u = 0; u < 4; ++u) pv[u] = sP[j][qb][u][lane];
          frag sf[2];
          float ds[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            ds[i] = pv[i >> 2][i & 3] * dpacc[qb][i];
            sf[i >> 3][i & 7] = (T)ds[i];
          }
          csum += tree_sum16(ds);
#pragma unroll
          for (int d = 0; d < ND; ++d)
#pragma unroll
            for (int t = 0; t < 2; ++t)
              acc[d] = E::mma(TLy::tr(sQb, 32 * qb + 16 * t, 32 * d, lane), sf[t], acc[d]);
          if constexpr (SGB) {
            // in two halves: C3 dK/dV -2.0 % against all reads before all
            // MFMAs (quarters: -0.4 %, two reads per MFMA: +0.1 %)
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x100, 2 * ND, 0);
            __builtin_amdgcn_sched_group_barrier(0x008, ND, 0);
          }
        }
        __builtin_amdgcn_s_setprio(0);
      }
    };
    if constexpr (DMA) {
      static_assert(!DMA || BM == 64, "one 64-lane DMA per per-query term");
      // The tile's raw L and Delta are DMA'd with it (the last wave issues
      // them) and turned into -L/c and -Delta by the first wave once landed.
      DmaPair<T, BM, DP, W> dma;
      dma.init(Q, p.sq[2], dO, p.sdo[2], N, wave, lane);
      const i32x4_t roff = buffer_rsrc(offg, 4u * (uint32_t)N);
      const i32x4_t rdel = buffer_rsrc(SOFTMAX ? delg : offg, 4u * (uint32_t)N);
      auto tok0_of = [&](int qt) { return org + 32 * (qt * QB - qshift); };
      dma_pipeline(
          nqt_all - qt_lo,
          [&](int t, int b) {
            const int tok0 = tok0_of(qt_lo + t);
            dma.issue(tok0, dQt[b], dDt[b]);
            if (wave == W - 1) {
              const uint32_t vo = 4u * (uint32_t)(tok0 + lane);  // negative tokens: out of range
              dma4(vo, roff, lds_addr(dRaw[b][0]));
              if constexpr (SOFTMAX) dma4(vo, rdel, lds_addr(dRaw[b][1]));
            }
          },
          [&](int t, int b) {
            if (tid < BM) {
              const int tok = tok0_of(qt_lo + t) + tid;
              const bool ok = tok >= 0 && tok < N;
              dOff[b][tid] = ok ? -dRaw[b][0][tid] * inv_c : -__builtin_inff();  // padding queries: P = 0
              dDel[b][tid] = (SOFTMAX && ok) ? -dRaw[b][1][tid] : 0.f;
            }
          },
          [&](int t, int b) { compute(qt_lo + t, dQt[b], dDt[b], dOff[b], dDel[b]); });
    } else {
      load_tile(qt_lo);
      for (int qt = qt_lo; qt < nqt_all; ++qt) {
        const int buf = qt & 1;
        TLy::store(tq, sQ[buf], tid);
        TLy::store(td, sD[buf], tid);
        if (tid < BM) {
          sOff[buf][tid] = offr;
          sDel[buf][tid] = delr;
        }
        __syncthreads();
        if (qt + 1 < nqt_all) load_tile(qt + 1);
        compute(qt, sQ[buf], sD[buf], sOff[buf], sDel[buf]);
      }
    }
  };
  if (pwave) tile_loop(std::true_type{});
  else tile_loop(std::false_type{});

  if (!wave_on) return;
  const float g2 = 2.f * p.gamma;
  const float cs = xhalf_sum(csum);
  if (ktok < 0) return;
  T* orow = pwave ? reinterpret_cast<T*>(p.dv) + b * p.sdv[0] + hh * p.sdv[1] + (int64_t)ktok * p.sdv[2]
                  : reinterpret_cast<T*>(p.dk) + b * p.sdk[0] + hh * p.sdk[1] + (int64_t)ktok * p.sdk[2];
  const T* krow = K + (int64_t)ktok * p.sk[2];
#pragma unroll
  for (int d = 0; d < ND; ++d)
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int dd = 32 * d + 8 * g + 4 * h;
      if (dd < D) {
        float a4[4];
        if (pwave) {
#pragma unroll
          for (int e = 0; e < 4; ++e) a4[e] = acc[d][4 * g + e];
        } else {
          float k4[4];
          ld4f<T>(krow + dd, k4);
#pragma unroll
          for (int e = 0; e < 4; ++e) a4[e] = g2 * (acc[d][4 * g + e] - cs * k4[e]);
        }
        st4f<T>(orow + dd, a4);
      }
    }
}

template <typename T, int DP, int NP, int BM, bool SOFTMAX, bool SGB = false, bool BIN = false, bool DMA = false>
__global__ __launch_bounds__(128 * NP) void rbf_bwd_dkdv_pair_kernel(const Params p) {
  for_each_group<BIN>(p, (p.nblk + NP - 1) / NP, false,
                 [&](int bh, int grp) { rbf_bwd_dkdv_pair_group<T, DP, NP, BM, SOFTMAX, SGB, DMA>(p, bh, grp); });
}

}  // namespace rbf
