/*
 * rbf_attn.h - C ABI of the MI355X (gfx950) fused RBF attention library
 * (librbfattn.so).
 *
 * RBF attention scores a query/key pair by -gamma * ||q_i - k_j||^2.
 * Softmax variant:   O = softmax_j(2*gamma*q.k - gamma*||k||^2) V, and the
 *                    row log-sum-exp L is kept in base 2 (log2 of the
 *                    normaliser of exp2(log2(e) * logits)).
 * Non-softmax:       O_i = sum_j exp(-gamma*||q_i - k_j||^2) v_j
 *                    (no max, no normaliser, no L).
 *
 * Every entry point below replaces one piece of the reference's launch code
 * in rbf_attention.py (4rtemi5/rbf_attention); the host side is the
 * torch.library custom-op layer in rbf_attention_amd/ops.py, which keeps the
 * reference op names and schemas.
 *
 * Conventions
 *  - Tensors are (B, H, N, D) with arbitrary strides on B, H and N (in
 *    elements) and unit stride on D.  Base pointers must be 16-byte aligned
 *    and every stride a multiple of 16 bytes; violations return
 *    RBF_ATTN_EINVAL_STRIDE and launch nothing.
 *  - lse and delta are fp32, contiguous (B, H, N).
 *  - The library never allocates device memory: outputs and the fp32
 *    workspaces are owned by the caller.
 *  - All kernels are enqueued on the caller's stream (hipStream_t passed as
 *    void*; NULL = legacy default stream).  Calls never synchronise.
 *  - Calls are re-entrant (they keep no state between calls), except
 *    rbf_attn_bwd_noalloc, whose calls share one workspace per GPU: two of
 *    them overlapping on one GPU race (see its comment).  The last error
 *    message is thread-local.
 *  - Return value 0 = success, negative = error code below.
 */
#ifndef RBF_ATTN_H_
#define RBF_ATTN_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RBF_ATTN_ABI_VERSION 2

/* variant */
#define RBF_ATTN_SOFTMAX 0
#define RBF_ATTN_NON_SOFTMAX 1

/* dtype */
#define RBF_ATTN_BF16 0
#define RBF_ATTN_FP16 1
#define RBF_ATTN_FP32 2

/* error codes */
#define RBF_ATTN_OK 0
#define RBF_ATTN_EINVAL_ARGS -1    /* null args, bad abi version, bad enum  */
#define RBF_ATTN_EINVAL_DTYPE -2   /* unknown dtype                         */
#define RBF_ATTN_EINVAL_STRIDE -3  /* misaligned pointer or stride          */
#define RBF_ATTN_EINVAL_HEADDIM -4 /* D outside [8, 256] or D % 8 != 0      */
#define RBF_ATTN_EINVAL_SHAPE -5   /* negative sizes, grid too large        */
#define RBF_ATTN_EINVAL_PTR -6     /* a required pointer is NULL            */
#define RBF_ATTN_ELAUNCH -7        /* the HIP runtime rejected a launch     */
#define RBF_ATTN_EUNSUPPORTED -8   /* valid, but outside a fused path's set */

/* One (B, H, N, D) operand: base pointer and element strides of dims 0-2. */
typedef struct rbf_attn_tensor {
  void* ptr;
  int64_t stride_b;
  int64_t stride_h;
  int64_t stride_n;
} rbf_attn_tensor;

typedef struct rbf_attn_args {
  int32_t abi_version; /* must be RBF_ATTN_ABI_VERSION                       */
  int32_t variant;     /* RBF_ATTN_SOFTMAX | RBF_ATTN_NON_SOFTMAX            */
  int32_t dtype;       /* element type shared by q,k,v,o,dout,dq,dk,dv       */
  int32_t B, H, N, D;
  int32_t causal;      /* 1: key j visible to query i iff j <= i             */
  int32_t num_prefix;  /* keys j < num_prefix are visible to every query
                          (register tokens); 0 = plain causal mask          */
  float gamma;         /* RBF bandwidth; the reference's sm_scale = 1/sqrt(D) */
  rbf_attn_tensor q, k, v;
  rbf_attn_tensor o;    /* fwd: written; bwd (softmax): read for Delta      */
  rbf_attn_tensor dout; /* bwd: read                                          */
  rbf_attn_tensor dq, dk, dv; /* bwd: written                               */
  float* lse;   /* softmax fwd: written (base-2 LSE); softmax bwd: read.
                   non-softmax bwd: fp32 (B,H,N) workspace, overwritten.    */
  float* delta; /* softmax bwd: fp32 (B,H,N) workspace, overwritten with
                   rowsum(O*dO).  Unused (may be NULL) for non-softmax.     */
} rbf_attn_args;

/*
 * Forward pass: writes o (and lse for the softmax variant).
 * Replaces the Triton launches of
 *   rbf_scaled_fwd       rbf_attention.py:651-690 (_rbf_attn_fwd_kernel,
 *                        rbf_attention.py:65-219), and
 *   rbf_non_softmax_fwd  rbf_attention.py:1355-1391
 *                        (_rbf_non_softmax_fwd_kernel, rbf_attention.py:861-997).
 * Two kernels' worth of launch code collapse into one call: variant selects.
 */
int rbf_attn_fwd(const rbf_attn_args* args, void* stream);

/*
 * Backward pass: writes dq, dk, dv (and the lse/delta workspaces as noted).
 * Replaces the Triton launches of
 *   rbf_scaled_bwd       rbf_attention.py:702-810 (_bwd_preprocess 222-276,
 *                        _rbf_attn_bwd_dk_dv_kernel 279-477,
 *                        _rbf_attn_bwd_dq_kernel 480-642), and
 *   rbf_non_softmax_bwd  rbf_attention.py:1399-1480
 *                        (_rbf_non_softmax_bwd_dk_dv_kernel 1000-1184,
 *                        _rbf_non_softmax_bwd_dq_kernel 1187-1352).
 * Two launches on the stream: the dQ kernel (which also produces Delta, or
 * for the non-softmax variant the per-query norm offsets) and then the
 * dK/dV kernel that consumes them -- or, for heads that fit one work-group's
 * LDS (bf16/fp16, 32 < D <= 64, N <= 576, at least one head per CU), one
 * launch that runs both passes of each head back to back
 * (rbf_attn_bwd_kernels says which).  Same results either way.
 */
int rbf_attn_bwd(const rbf_attn_args* args, void* stream);

/*
 * One stage of rbf_attn_bwd: stage 1 = the dQ kernel (also writes Delta, or
 * the non-softmax norm offsets, into the workspaces), stage 2 = the dK/dV
 * kernel (reads them).  rbf_attn_bwd == stage 1 then stage 2 on one stream.
 * No reference counterpart: it exists so callers can time or schedule the
 * two kernels separately.  Same validation and error codes as rbf_attn_bwd;
 * any other stage value returns RBF_ATTN_EINVAL_ARGS.
 */
int rbf_attn_bwd_stage(const rbf_attn_args* args, void* stream, int stage);

/*
 * Backward pass that allocates nothing and needs no caller workspace.
 * No counterpart in the reference: it is for callers that cannot allocate
 * device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid allocation).  Same kernels and results as rbf_attn_bwd, but the fp32
 * per-query workspace (softmax: Delta, in place of args->delta; non-softmax:
 * the norm offsets, in place of args->lse) lives in a static device array of
 * the library, one per GPU, held until the process ends.  args->delta is
 * ignored; args->lse is read (the forward's L) for the softmax variant and
 * ignored for the non-softmax one.  Limit: B * H * N <=
 * RBF_ATTN_NOALLOC_MAX_ROWS (4 MiB of fp32 per GPU); larger problems return
 * RBF_ATTN_EINVAL_SHAPE before any launch.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (e.g. on two streams) race.
 * The array needs no clearing: each call writes every entry it reads.  The
 * first call on a device looks the array's address up (in relaxed stream-
 * capture mode on the calling thread), so that call may itself be captured.
 */
#define RBF_ATTN_NOALLOC_MAX_ROWS (1 << 20)
int rbf_attn_bwd_noalloc(const rbf_attn_args* args, void* stream);

/*
 * A position term for rbf_attn_fwd_pos / rbf_attn_bwd_pos: a
 * (batch, H, N, D) operand, with batch = B (one term per batch entry) or
 * batch = 1 (one term shared by every batch entry, which the kernels read at
 * every b: t.stride_b must then be 0).  Any other batch returns
 * RBF_ATTN_EINVAL_SHAPE, and batch = 1 with t.stride_b != 0 returns
 * RBF_ATTN_EINVAL_STRIDE, both before any launch: the kernels index the term
 * with b * t.stride_b for every b < B, so a batch-1 term passed with its own
 * nonzero batch stride would be read past its end.
 */
typedef struct rbf_attn_pos_term {
  rbf_attn_tensor t;
  int32_t batch;
} rbf_attn_pos_term;

/*
 * Forward / backward with a position term fused into the Q and K reads:
 * the kernels use q + pos and k + pos (each sum rounded to the element type,
 * as two separate elementwise adds of the tensors would store it) wherever
 * the plain entry points use q and k.  The gradients dq, dk are those of the
 * shifted inputs, which equal the gradients of q, k; the term's own gradient
 * is sum_b (dq + dk) (batch = 1) or dq + dk (batch = B) and is left to the
 * caller.  No reference counterpart: it fuses the SuSiE position embedding
 * of the reference model (rbf_attention.py:1666-1688,
 * `q, k = q + pos_emb, k + pos_emb`) into the attention kernels.  Supported
 * for bf16/fp16, 32 < D <= 64, N <= 576 (the head-resident kernels);
 * otherwise RBF_ATTN_EUNSUPPORTED before any launch.
 */
int rbf_attn_fwd_pos(const rbf_attn_args* args, const rbf_attn_pos_term* pos, void* stream);
int rbf_attn_bwd_pos(const rbf_attn_args* args, const rbf_attn_pos_term* pos, void* stream);

/* Number of kernels rbf_attn_bwd (pos == NULL) or rbf_attn_bwd_pos enqueues
 * for args: 1 (both passes of a head in one head-resident kernel), 2 (a dQ
 * kernel, then a dK/dV kernel), 0 for an empty problem, or a negative error
 * code for invalid args.  Launches nothing.  No reference counterpart: for
 * callers that time or profile the backward per kernel. */
int rbf_attn_bwd_kernels(const rbf_attn_args* args, const rbf_attn_pos_term* pos);

/* 1 if rbf_attn_fwd_pos / rbf_attn_bwd_pos support args (shape, dtype), 0 if
 * not, or a negative error code for invalid args.  No reference counterpart. */
int rbf_attn_pos_supported(const rbf_attn_args* args);

/*
 * Decode against a KV cache: T new query tokens per (batch, head) attend to
 * the cached keys and values.  No reference counterpart -- the reference has
 * no decode path (its README lists one as future work); this is the
 * "KV-cache decode" next step of the build.  Query t of batch b sits at
 * cache position len_b - T + t and sees keys [0, len_b - T + t]: the cache
 * already holds the new tokens' K and V.  The key axis is split over
 * work-groups; partial results go to a caller-provided fp32 workspace and a
 * second kernel merges them (softmax: log-sum-exp weights; non-softmax: sum).
 */
typedef struct rbf_attn_decode_args {
  int32_t abi_version; /* must be RBF_ATTN_ABI_VERSION                       */
  int32_t variant;     /* RBF_ATTN_SOFTMAX | RBF_ATTN_NON_SOFTMAX            */
  int32_t dtype;       /* element type of q, k, v, o                         */
  int32_t B, H;
  int32_t T;           /* new query tokens per (b, h): 1 <= T <= 32          */
  int32_t D;           /* 8 <= D <= 256, D % 8 == 0                          */
  int32_t L;           /* cache length (maximum over the batch), L >= T      */
  float gamma;         /* RBF bandwidth                                      */
  rbf_attn_tensor q;   /* (B, H, T, D)                                        */
  rbf_attn_tensor k, v; /* (B, H, >= L, D) caches                             */
  rbf_attn_tensor o;   /* (B, H, T, D), written                              */
  const int32_t* lens; /* optional device int32[B]: per-batch cache lengths,
                          each in [T, L]; NULL = every batch entry has L     */
  float* lse;          /* optional (softmax): fp32 contiguous (B, H, T) base-2
                          log-sum-exp, written; NULL = not written           */
  void* workspace;     /* fp32 scratch, rbf_attn_decode_workspace_size bytes,
                          16-byte aligned, overwritten                       */
  uint64_t workspace_bytes;
} rbf_attn_decode_args;

/* Bytes of workspace rbf_attn_decode needs for these sizes (0 on invalid
 * sizes; the reason is in rbf_attn_last_error). */
uint64_t rbf_attn_decode_workspace_size(const rbf_attn_decode_args* args);

/* Decode: writes o (and lse when given).  Two launches on the stream. */
int rbf_attn_decode(const rbf_attn_decode_args* args, void* stream);

/* Message describing the last failed call on this thread ("" if none).
 * No reference counterpart: the reference surfaces Triton exceptions. */
const char* rbf_attn_last_error(void);

/* RBF_ATTN_ABI_VERSION of the loaded library. No reference counterpart. */
int rbf_attn_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* RBF_ATTN_H_ */
