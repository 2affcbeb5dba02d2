"""CPU oracle for RBF attention -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use
this module, and only as the checker or the timed CPU baseline.  The product
path (rbf_attention_amd) never imports it.

It restates, in numpy float64, the reference's PyTorch math paths:

* logits      -gamma * ||q_i - k_j||^2                rbf_attention.py:1547-1553
              (compute_rbf_logits, with 1/sqrt(D) generalised to gamma)
* softmax     causal-masked softmax(logits) @ V       rbf_attention.py:1738-1744
              ("rbf_slow"), rbf_math_test.py:33-41
* L           base-2 log-sum-exp of 2*gamma*q.k - gamma*||k||^2, i.e. of the
              logits without the per-query -gamma*||q||^2 constant, as the
              fused kernel stores it                  rbf_attention.py:191-219
* non-softmax exp(masked logits) @ V                  rbf_attention.py:1747-1753
              ("rbf_non_softmax_slow")
* decode      the last T query rows of the causal forward over a KV cache
              (no reference counterpart; pinned to softmax_forward /
              non_softmax_forward)
* rounding    rounded_model: the same math with P and dS rounded to the
              element type where the reference kernels round them
              (rbf_attention.py:201, 422, 432, 621) and outputs rounded; an
              error-size reference for bf16/fp16 parity, not a target
* augmented   q' = [q, 1, 0...], k' = [k, -||k||^2/2, 0...] padded to a
              multiple of 8, SDPA with scale 2*gamma  test_equivalence.py:9-33,
              rbf_math_test.py:46-64, rbf_attention.py:1718-1735
* gradients   closed forms of the autograd the reference relies on
              (rbf_attention.py:222-276, 279-477, 480-642 for softmax;
              1000-1184, 1187-1352 for non-softmax):
                dP = dO V^T, dS = P*(dP - Delta) | P*dP,  Delta_i = sum_j P_ij dP_ij
                dV = P^T dO
                dQ = 2 gamma (dS K - rowsum(dS) q)
                dK = 2 gamma (dS^T Q - colsum(dS) k)
  The rowsum(dS) term is identically zero for softmax (sum_j dS_ij = 0) and is
  kept here because the direct-distance logits contain -gamma*||q||^2.

Masking: key j is visible to query i iff (not causal) or j <= i or
j < num_prefix.  num_prefix = 0 is the reference's is_causal=True mask
(rbf_attention.py:186-187, 1556-1565); num_prefix = R makes R register tokens
visible to every query (the benchmark configurations' "registers visible to all").

How this oracle is pinned (tests/test_oracle.py): the two independent
restatements (direct distance, augmented SDPA) agree; the augmented one also
agrees with torch's own float64 scaled_dot_product_attention (a library
routine); the closed-form gradients agree with torch autograd on the direct
form and with central finite differences; pure-Python brute-force loops agree
on tiny inputs; invariants (row 0 sees only key 0, equal-norm keys reduce to
textbook SDPA with scale 2*gamma, L*ln2 = logsumexp, rowsum(dS) = 0, single-key
non-softmax with q = k returns v) hold; and deliberately broken copies of the
oracle fail those checks.
"""
from __future__ import annotations

import math

import numpy as np

LOG2E = 1.0 / math.log(2.0)


def _f64(x) -> np.ndarray:
    return np.asarray(x, dtype=np.float64)


def visibility(n: int, causal: bool = True, num_prefix: int = 0) -> np.ndarray:
    """(n, n) bool: True where key j (column) is visible to query i (row)."""
    if not causal:
        return np.ones((n, n), dtype=bool)
    i = np.arange(n)[:, None]
    j = np.arange(n)[None, :]
    return (j <= i) | (j < num_prefix)


def rbf_logits(q: np.ndarray, k: np.ndarray, gamma: float) -> np.ndarray:
    """-gamma * ||q_i - k_j||^2 via the expansion of rbf_attention.py:1547-1553."""
    q = _f64(q)
    k = _f64(k)
    qq = np.einsum("...nd,...nd->...n", q, q)[..., :, None]
    kk = np.einsum("...nd,...nd->...n", k, k)[..., None, :]
    return -gamma * (qq + kk - 2.0 * q @ np.swapaxes(k, -1, -2))


def _slices(*arrays):
    """Iterate (b, h) slices of (B, H, N, D) arrays."""
    B, H = arrays[0].shape[:2]
    for b in range(B):
        for h in range(H):
            yield b, h, [a[b, h] for a in arrays]


def _softmax_probs(q, k, gamma, mask):
    s = rbf_logits(q, k, gamma)
    s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    e = np.exp(s - m)
    l = e.sum(axis=-1, keepdims=True)
    return e / l, m[..., 0], l[..., 0]


def softmax_forward(q, k, v, gamma: float, causal: bool = True, num_prefix: int = 0):
    """Returns (O, L) in float64; O is (B,H,N,D), L is (B,H,N) base-2."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, N, D = q.shape
    mask = visibility(N, causal, num_prefix)
    O = np.empty_like(v)
    L = np.empty((B, H, N))
    for b, h, (qs, ks, vs) in _slices(q, k, v):
        P, m, l = _softmax_probs(qs, ks, gamma, mask)
        O[b, h] = P @ vs
        # natural-log LSE of -gamma||q-k||^2, then add back gamma||q||^2 and
        # convert to base 2 (rbf_attention.py:219 stores m + log2(l)).
        L[b, h] = (m + np.log(l) + gamma * np.einsum("nd,nd->n", qs, qs)) * LOG2E
    return O, L


def softmax_backward(q, k, v, dO, gamma: float, causal: bool = True, num_prefix: int = 0):
    """Returns (dQ, dK, dV) in float64."""
    q, k, v, dO = _f64(q), _f64(k), _f64(v), _f64(dO)
    N = q.shape[2]
    mask = visibility(N, causal, num_prefix)
    dQ, dK, dV = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    for b, h, (qs, ks, vs, dos) in _slices(q, k, v, dO):
        P, _, _ = _softmax_probs(qs, ks, gamma, mask)
        dP = dos @ vs.T
        delta = (P * dP).sum(axis=-1, keepdims=True)
        dS = P * (dP - delta)
        dV[b, h] = P.T @ dos
        dQ[b, h] = 2.0 * gamma * (dS @ ks - dS.sum(axis=1)[:, None] * qs)
        dK[b, h] = 2.0 * gamma * (dS.T @ qs - dS.sum(axis=0)[:, None] * ks)
    return dQ, dK, dV


def non_softmax_forward(q, k, v, gamma: float, causal: bool = True, num_prefix: int = 0):
    q, k, v = _f64(q), _f64(k), _f64(v)
    N = q.shape[2]
    mask = visibility(N, causal, num_prefix)
    O = np.empty_like(v)
    for b, h, (qs, ks, vs) in _slices(q, k, v):
        P = np.where(mask, np.exp(rbf_logits(qs, ks, gamma)), 0.0)
        O[b, h] = P @ vs
    return O


def non_softmax_backward(q, k, v, dO, gamma: float, causal: bool = True, num_prefix: int = 0):
    q, k, v, dO = _f64(q), _f64(k), _f64(v), _f64(dO)
    N = q.shape[2]
    mask = visibility(N, causal, num_prefix)
    dQ, dK, dV = np.empty_like(q), np.empty_like(k), np.empty_like(v)
    for b, h, (qs, ks, vs, dos) in _slices(q, k, v, dO):
        P = np.where(mask, np.exp(rbf_logits(qs, ks, gamma)), 0.0)
        dS = P * (dos @ vs.T)
        dV[b, h] = P.T @ dos
        dQ[b, h] = 2.0 * gamma * (dS @ ks - dS.sum(axis=1)[:, None] * qs)
        dK[b, h] = 2.0 * gamma * (dS.T @ qs - dS.sum(axis=0)[:, None] * ks)
    return dQ, dK, dV


# ---------------------------------------------------------------------------
# Rounding model of the reference kernels (error-size reference for bf16/fp16)
# ---------------------------------------------------------------------------
def round_bf16(x) -> np.ndarray:
    """float64 -> nearest bfloat16 (ties to even, via float32) -> float64."""
    x32 = np.ascontiguousarray(_f64(x), dtype=np.float32)
    b = x32.view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def round_fp16(x) -> np.ndarray:
    return _f64(x).astype(np.float16).astype(np.float64)


def rounder(dtype: str):
    """Rounding to an element type named "bf16" / "fp16" / "fp32"."""
    return {"bf16": round_bf16, "fp16": round_fp16,
            "fp32": lambda x: _f64(x).astype(np.float32).astype(np.float64)}[dtype]


def _identity(x):
    return x


def rounded_model(q, k, v, dO, gamma: float, softmax: bool = True, causal: bool = True, num_prefix: int = 0,
                  rnd=_identity, out_rnd=_identity):
    """(O, dQ, dK, dV) in float64 with the roundings the reference kernels
    apply to their MFMA/dot operands, so that a kernel's error can be set
    beside the error its own arithmetic makes unavoidable:

    * P is rounded (``rnd``) before P V (rbf_attention.py:201) and P^T dO
      (422); the forward's row sum uses the unrounded P (196-198); the
      forward's P is taken relative to the row maximum (191-194), whose
      power-of-two-free scale the rounding sees;
    * dS is rounded before dS^T Q (432) and dS K (621); the key-norm column
      sum of dK uses the unrounded dS (431, 447);
    * Delta is formed from the stored (rounded) O (275-276);
    * every output is rounded to the element type (``out_rnd``; 207-213,
      447-460, 626-640).

    Q/K pre-scaling in the element type (151, 361, 561) is not modelled (the
    kernels here scale in fp32), so the model's error is a lower bound of
    the reference kernel's.  With both roundings the identity this is exactly
    softmax_forward/softmax_backward (non_softmax_*)."""
    q, k, v, dO = _f64(q), _f64(k), _f64(v), _f64(dO)
    N = q.shape[2]
    vis = visibility(N, causal, num_prefix)
    outs = [np.empty_like(x) for x in (v, q, k, v)]
    for b, h, (qs, ks, vs, dos) in _slices(q, k, v, dO):
        lg = np.where(vis, rbf_logits(qs, ks, gamma), -np.inf)
        if softmax:
            # the logits' -gamma||q||^2 is a per-row constant: P and dS are
            # those of the kernels' 2 gamma q.k - gamma ||k||^2
            ex = np.exp(lg - lg.max(axis=-1, keepdims=True))
            den = ex.sum(axis=-1, keepdims=True)
            o_st = out_rnd((rnd(ex) @ vs) / den)
            prob = ex / den
            grad_s = prob * (dos @ vs.T - (o_st * dos).sum(axis=-1, keepdims=True))
            q_term = 0.0  # the q-norm-free logits have no d/dq of -gamma||q||^2
        else:
            prob = np.exp(lg)
            o_st = out_rnd(rnd(prob) @ vs)
            grad_s = prob * (dos @ vs.T)
            q_term = grad_s.sum(axis=1)[:, None] * qs
        r_gs = rnd(grad_s)
        outs[0][b, h] = o_st
        outs[1][b, h] = out_rnd(2.0 * gamma * (r_gs @ ks - q_term))
        outs[2][b, h] = out_rnd(2.0 * gamma * (r_gs.T @ qs - grad_s.sum(axis=0)[:, None] * ks))
        outs[3][b, h] = out_rnd(rnd(prob).T @ dos)
    return tuple(outs)


def decode_forward(q, k, v, gamma: float, softmax: bool = True, lens=None, rnd=_identity, out_rnd=_identity):
    """KV-cache decode: q (B,H,T,D) against caches k, v (B,H,L,D).  Query t of
    batch b sits at position lens[b] - T + t (lens defaults to L) and sees
    keys [0, that position]: rows lens[b]-T .. lens[b]-1 of the causal forward
    over the first lens[b] cached tokens (the reference has no decode path;
    this is its causal attention restricted to the last T query rows, with
    rbf_attention.py:1547-1553 logits).  Returns (O, L) in float64; L is the
    base-2 LSE as in softmax_forward, and None for the non-softmax variant.
    rnd / out_rnd: the rounding of P and of the output, as in rounded_model
    (identity: exact)."""
    q, k, v = _f64(q), _f64(k), _f64(v)
    B, H, T, D = q.shape
    Lc = k.shape[2]
    lens = [Lc] * B if lens is None else [int(x) for x in lens]
    O = np.zeros_like(q)
    Lse = np.empty((B, H, T))
    for b in range(B):
        n = lens[b]
        pos = np.arange(n - T, n)[:, None]
        mask = np.arange(n)[None, :] <= pos
        for h in range(H):
            s = rbf_logits(q[b, h], k[b, h, :n], gamma)
            s = np.where(mask, s, -np.inf)
            if softmax:
                m = s.max(axis=-1, keepdims=True)
                e = np.exp(s - m)
                l = e.sum(axis=-1, keepdims=True)
                O[b, h] = out_rnd((rnd(e) @ v[b, h, :n]) / l)
                Lse[b, h] = (m[:, 0] + np.log(l[:, 0]) + gamma * np.einsum("td,td->t", q[b, h], q[b, h])) * LOG2E
            else:
                O[b, h] = out_rnd(rnd(np.exp(s)) @ v[b, h, :n])
    return O, (Lse if softmax else None)


def augment(q, k):
    """The augmented-dimension operands of test_equivalence.py:17-25:
    q' = [q, 1], k' = [k, -||k||^2/2], zero-padded to a multiple of 8."""
    q, k = _f64(q), _f64(k)
    kk = np.einsum("...nd,...nd->...n", k, k)[..., None]
    qp = np.concatenate([q, np.ones_like(q[..., :1])], axis=-1)
    kp = np.concatenate([k, -0.5 * kk], axis=-1)
    pad = (8 - qp.shape[-1] % 8) % 8
    if pad:
        widths = [(0, 0)] * (qp.ndim - 1) + [(0, pad)]
        qp = np.pad(qp, widths)
        kp = np.pad(kp, widths)
    return qp, kp


def softmax_forward_augmented(q, k, v, gamma: float, causal: bool = True, num_prefix: int = 0):
    """Second, independent restatement: textbook attention on the augmented
    operands with scale 2*gamma (test_equivalence.py:9-33)."""
    qp, kp = augment(q, k)
    v = _f64(v)
    N = qp.shape[2]
    mask = visibility(N, causal, num_prefix)
    O = np.empty_like(v)
    for b, h, (qs, ks, vs) in _slices(qp, kp, v):
        s = np.where(mask, 2.0 * gamma * (qs @ ks.T), -np.inf)
        e = np.exp(s - s.max(axis=-1, keepdims=True))
        O[b, h] = (e / e.sum(axis=-1, keepdims=True)) @ vs
    return O


# ---------------------------------------------------------------------------
# Brute force: pure-Python loops, tiny inputs only (B = H = 1, N <= 8).
# ---------------------------------------------------------------------------
def brute_force(q, k, v, dO, gamma: float, softmax: bool, causal: bool = True, num_prefix: int = 0):
    """Forward and backward of one (N, D) slice by explicit loops.

    Returns (O, dQ, dK, dV) as nested lists.  The gradient is assembled from
    the chain rule term by term: dO -> P (through O = P V), P -> logits
    (softmax Jacobian or exp'), logits -> q, k (d/dq of -gamma||q-k||^2).
    """
    q, k, v, dO = (_f64(x).tolist() for x in (q, k, v, dO))
    N, D = len(q), len(q[0])

    def vis(i, j):
        return (not causal) or j <= i or j < num_prefix

    logit = [[-gamma * sum((q[i][d] - k[j][d]) ** 2 for d in range(D)) for j in range(N)] for i in range(N)]
    P = [[0.0] * N for _ in range(N)]
    for i in range(N):
        if softmax:
            mx = max(logit[i][j] for j in range(N) if vis(i, j))
            den = sum(math.exp(logit[i][j] - mx) for j in range(N) if vis(i, j))
            for j in range(N):
                P[i][j] = math.exp(logit[i][j] - mx) / den if vis(i, j) else 0.0
        else:
            for j in range(N):
                P[i][j] = math.exp(logit[i][j]) if vis(i, j) else 0.0
    O = [[sum(P[i][j] * v[j][d] for j in range(N)) for d in range(D)] for i in range(N)]
    # dL/dP_ij = sum_d dO_id v_jd
    gP = [[sum(dO[i][d] * v[j][d] for d in range(D)) for j in range(N)] for i in range(N)]
    dV = [[sum(P[i][j] * dO[i][d] for i in range(N)) for d in range(D)] for j in range(N)]
    # dL/dlogit_ij
    gS = [[0.0] * N for _ in range(N)]
    for i in range(N):
        for j in range(N):
            if not vis(i, j):
                continue
            if softmax:
                # dP_ij'/dlogit_ij = P_ij' (delta_jj' - P_ij)
                gS[i][j] = sum(gP[i][jj] * P[i][jj] * ((1.0 if jj == j else 0.0) - P[i][j]) for jj in range(N))
            else:
                gS[i][j] = gP[i][j] * P[i][j]
    # dlogit_ij/dq_i = -2 gamma (q_i - k_j) ; dlogit_ij/dk_j = +2 gamma (q_i - k_j)
    dQ = [[sum(gS[i][j] * -2.0 * gamma * (q[i][d] - k[j][d]) for j in range(N)) for d in range(D)] for i in range(N)]
    dK = [[sum(gS[i][j] * 2.0 * gamma * (q[i][d] - k[j][d]) for i in range(N)) for d in range(D)] for j in range(N)]
    return O, dQ, dK, dV
