"""Pins of the CPU oracle (oracle/rbf_oracle.py).  CPU only.

Each check compares the oracle with something it does not share code or
formulas with: a second restatement, torch's float64 library routines
(scaled_dot_product_attention and its autograd), central finite differences,
pure-Python loops, or a mathematical invariant.  The mutation tests at the end
apply plausible mistakes to the oracle's own source and require that at least
one pin then fails.
"""
import inspect
import math
import types

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import rbf_oracle as ro

RNG = np.random.default_rng(1234)


def rand(*shape, scale=1.0):
    return RNG.standard_normal(shape) * scale


def t64(x):
    return torch.tensor(np.asarray(x), dtype=torch.float64)


def sdpa_mask(n, causal, num_prefix):
    return torch.tensor(ro.visibility(n, causal, num_prefix))


# ---------------------------------------------------------------------------
# Pin checks, parameterised by the oracle namespace so that mutants can be
# run through the same checks.
# ---------------------------------------------------------------------------
def pin_forward_vs_augmented(o, causal=True, num_prefix=0):
    q, k, v = rand(2, 2, 19, 12), rand(2, 2, 19, 12, scale=1.7), rand(2, 2, 19, 12)
    g = 0.21
    O1, _ = o.softmax_forward(q, k, v, g, causal, num_prefix)
    O2 = o.softmax_forward_augmented(q, k, v, g, causal, num_prefix)
    return np.abs(O1 - O2).max() < 1e-12


def pin_forward_vs_torch_sdpa(o, causal=True, num_prefix=0):
    """Augmented operands through torch's own float64 SDPA (a library routine)."""
    q, k, v = rand(2, 3, 17, 16), rand(2, 3, 17, 16), rand(2, 3, 17, 16)
    g = 1.0 / math.sqrt(16)
    qp, kp = o.augment(q, k)
    ref = F.scaled_dot_product_attention(
        t64(qp), t64(kp), t64(v), attn_mask=sdpa_mask(17, causal, num_prefix), scale=2 * g
    ).numpy()
    O, _ = o.softmax_forward(q, k, v, g, causal, num_prefix)
    return np.abs(O - ref).max() < 1e-12


def _torch_softmax_grads(q, k, v, dO, g, causal, num_prefix):
    """Gradients by torch autograd through the augmented SDPA form: the
    augmentation (k' = [k, -||k||^2/2]) and SDPA's backward are torch's."""
    tq, tk, tv = (t64(x).requires_grad_(True) for x in (q, k, v))
    ones = torch.ones_like(tq[..., :1])
    qp = torch.cat([tq, ones], -1)
    kp = torch.cat([tk, -0.5 * (tk * tk).sum(-1, keepdim=True)], -1)
    out = F.scaled_dot_product_attention(qp, kp, tv, attn_mask=sdpa_mask(q.shape[2], causal, num_prefix), scale=2 * g)
    out.backward(t64(dO))
    return tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy()


def pin_softmax_grads_vs_autograd(o, causal=True, num_prefix=0):
    q, k, v, dO = rand(2, 2, 15, 8), rand(2, 2, 15, 8, scale=1.5), rand(2, 2, 15, 8), rand(2, 2, 15, 8)
    g = 0.3
    ref = _torch_softmax_grads(q, k, v, dO, g, causal, num_prefix)
    got = o.softmax_backward(q, k, v, dO, g, causal, num_prefix)
    return all(np.abs(a - b).max() < 1e-11 for a, b in zip(got, ref))


def _torch_nonsoftmax(q, k, v, g, causal, num_prefix):
    # exp(-gamma * ||q - k||^2) via torch.cdist (a library routine, not the
    # oracle's expansion), masked, times V.
    d2 = torch.cdist(q, k) ** 2
    p = torch.exp(-g * d2) * sdpa_mask(q.shape[-2], causal, num_prefix)
    return p @ v


def pin_nonsoftmax_vs_autograd(o, causal=True, num_prefix=0):
    q, k, v, dO = (rand(2, 2, 13, 8, scale=0.5) for _ in range(4))
    g = 0.25
    tq, tk, tv = (t64(x).requires_grad_(True) for x in (q, k, v))
    out = _torch_nonsoftmax(tq, tk, tv, g, causal, num_prefix)
    out.backward(t64(dO))
    O = o.non_softmax_forward(q, k, v, g, causal, num_prefix)
    got = o.non_softmax_backward(q, k, v, dO, g, causal, num_prefix)
    ok = np.abs(O - out.detach().numpy()).max() < 1e-12
    ref = (tq.grad.numpy(), tk.grad.numpy(), tv.grad.numpy())
    return ok and all(np.abs(a - b).max() < 1e-11 for a, b in zip(got, ref))


def pin_brute_force(o, softmax=True, causal=True, num_prefix=0):
    q, k, v, dO = rand(1, 1, 6, 3), rand(1, 1, 6, 3), rand(1, 1, 6, 3), rand(1, 1, 6, 3)
    g = 0.4
    bO, bdq, bdk, bdv = (np.array(x) for x in ro.brute_force(q[0, 0], k[0, 0], v[0, 0], dO[0, 0], g, softmax, causal, num_prefix))
    if softmax:
        O, _ = o.softmax_forward(q, k, v, g, causal, num_prefix)
        grads = o.softmax_backward(q, k, v, dO, g, causal, num_prefix)
    else:
        O = o.non_softmax_forward(q, k, v, g, causal, num_prefix)
        grads = o.non_softmax_backward(q, k, v, dO, g, causal, num_prefix)
    pairs = [(O[0, 0], bO)] + [(a[0, 0], b) for a, b in zip(grads, (bdq, bdk, bdv))]
    return all(np.abs(a - b).max() < 1e-12 for a, b in pairs)


def pin_lse(o, causal=True, num_prefix=0):
    """L * ln2 equals torch.logsumexp of the augmented logits (no q-norm)."""
    q, k, v = rand(1, 2, 11, 8), rand(1, 2, 11, 8, scale=2.0), rand(1, 2, 11, 8)
    g = 0.35
    qp, kp = o.augment(q, k)
    s = 2 * g * (t64(qp) @ t64(kp).transpose(-1, -2))
    s = s.masked_fill(~sdpa_mask(11, causal, num_prefix), float("-inf"))
    ref = torch.logsumexp(s, -1).numpy()
    _, L = o.softmax_forward(q, k, v, g, causal, num_prefix)
    return np.abs(L * math.log(2) - ref).max() < 1e-12


def pin_finite_differences(o, softmax=True):
    """Central differences of loss = sum(O * dO) at a few coordinates."""
    q, k, v, dO = rand(1, 1, 7, 4), rand(1, 1, 7, 4), rand(1, 1, 7, 4), rand(1, 1, 7, 4)
    g = 0.3

    def loss(q_, k_, v_):
        O = o.softmax_forward(q_, k_, v_, g)[0] if softmax else o.non_softmax_forward(q_, k_, v_, g)
        return float((O * dO).sum())

    grads = (o.softmax_backward if softmax else o.non_softmax_backward)(q, k, v, dO, g)
    eps = 1e-6
    for which, gref in zip(range(3), grads):
        for idx in [(0, 0, 0, 0), (0, 0, 3, 2), (0, 0, 6, 1), (0, 0, 2, 3)]:
            args = [q.copy(), k.copy(), v.copy()]
            args[which][idx] += eps
            up = loss(*args)
            args[which][idx] -= 2 * eps
            dn = loss(*args)
            fd = (up - dn) / (2 * eps)
            if abs(fd - gref[idx]) > 1e-6 * max(1.0, abs(fd)):
                return False
    return True


def pin_decode_vs_forward(o, softmax=True, ragged=False):
    """Decode = the last T query rows of the causal forward over the first
    lens[b] cached tokens (the forward itself is pinned above)."""
    B, H, L, T, D = 2, 2, 23, 3, 8
    qf, k, v = rand(B, H, L, D), rand(B, H, L, D, scale=1.3), rand(B, H, L, D)
    g = 0.17
    lens = [L, 14] if ragged else [L, L]
    qd = np.stack([qf[b, :, lens[b] - T:lens[b]] for b in range(B)])
    O, Ld = o.decode_forward(qd, k, v, g, softmax, lens if ragged else None)
    for b in range(B):
        n = lens[b]
        if softmax:
            Of, Lf = o.softmax_forward(qf[b:b + 1, :, :n], k[b:b + 1, :, :n], v[b:b + 1, :, :n], g)
            if np.abs(Ld[b] - Lf[0, :, n - T:]).max() > 1e-12:
                return False
        else:
            Of = o.non_softmax_forward(qf[b:b + 1, :, :n], k[b:b + 1, :, :n], v[b:b + 1, :, :n], g)
        if np.abs(O[b] - Of[0, :, n - T:]).max() > 1e-12:
            return False
    return True


ALL_PINS = [
    lambda o: pin_forward_vs_augmented(o),
    lambda o: pin_forward_vs_augmented(o, num_prefix=4),
    lambda o: pin_forward_vs_augmented(o, causal=False),
    lambda o: pin_forward_vs_torch_sdpa(o),
    lambda o: pin_forward_vs_torch_sdpa(o, num_prefix=3),
    lambda o: pin_forward_vs_torch_sdpa(o, causal=False),
    lambda o: pin_softmax_grads_vs_autograd(o),
    lambda o: pin_softmax_grads_vs_autograd(o, num_prefix=4),
    lambda o: pin_softmax_grads_vs_autograd(o, causal=False),
    lambda o: pin_nonsoftmax_vs_autograd(o),
    lambda o: pin_nonsoftmax_vs_autograd(o, num_prefix=2),
    lambda o: pin_nonsoftmax_vs_autograd(o, causal=False),
    lambda o: pin_brute_force(o, softmax=True),
    lambda o: pin_brute_force(o, softmax=False),
    lambda o: pin_brute_force(o, softmax=True, num_prefix=3),
    lambda o: pin_brute_force(o, softmax=False, causal=False),
    lambda o: pin_lse(o),
    lambda o: pin_lse(o, num_prefix=2),
    lambda o: pin_finite_differences(o, softmax=True),
    lambda o: pin_finite_differences(o, softmax=False),
    lambda o: pin_decode_vs_forward(o, softmax=True),
    lambda o: pin_decode_vs_forward(o, softmax=True, ragged=True),
    lambda o: pin_decode_vs_forward(o, softmax=False, ragged=True),
]


# --- the rounding model (rounded_model) ---------------------------------------
def pin_rounded_identity_limit(o, softmax=True, causal=True, num_prefix=0):
    """Without rounding the model is the exact oracle."""
    q, k, v, dO = rand(2, 2, 13, 8), rand(2, 2, 13, 8, scale=1.3), rand(2, 2, 13, 8), rand(2, 2, 13, 8)
    g = 0.27
    got = o.rounded_model(q, k, v, dO, g, softmax, causal, num_prefix)
    if softmax:
        ref = (o.softmax_forward(q, k, v, g, causal, num_prefix)[0],) + o.softmax_backward(q, k, v, dO, g, causal,
                                                                                         num_prefix)
    else:
        ref = (o.non_softmax_forward(q, k, v, g, causal, num_prefix),) + o.non_softmax_backward(q, k, v, dO, g, causal,
                                                                                              num_prefix)
    return all(np.abs(a - b).max() < 1e-12 for a, b in zip(got, ref))


def brute_rounded(q, k, v, dO, g, softmax, rnd, causal=True, num_prefix=0):
    """Pure-Python loops of the reference kernels' arithmetic with a scalar
    rounding at each point where they round to the element type: P before
    P V and P^T dO, dS before dS^T Q and dS K, every stored output; row sums,
    column sums and Delta's O read from the stored (rounded) output."""
    q, k, v, dO = (np.asarray(x, dtype=np.float64).tolist() for x in (q, k, v, dO))
    N, D = len(q), len(q[0])
    r = lambda x: float(rnd(np.array([x]))[0])  # noqa: E731

    def vis(i, j):
        return (not causal) or j <= i or j < num_prefix

    lg = [[-g * sum((q[i][d] - k[j][d]) ** 2 for d in range(D)) for j in range(N)] for i in range(N)]
    P = [[0.0] * N for _ in range(N)]
    O = [[0.0] * D for _ in range(N)]
    for i in range(N):
        if softmax:
            mx = max(lg[i][j] for j in range(N) if vis(i, j))
            e = [math.exp(lg[i][j] - mx) if vis(i, j) else 0.0 for j in range(N)]
            den = sum(e)
            for d in range(D):
                O[i][d] = r(sum(r(e[j]) * v[j][d] for j in range(N)) / den)
            P[i] = [x / den for x in e]
        else:
            P[i] = [math.exp(lg[i][j]) if vis(i, j) else 0.0 for j in range(N)]
            for d in range(D):
                O[i][d] = r(sum(r(P[i][j]) * v[j][d] for j in range(N)))
    dS = [[0.0] * N for _ in range(N)]
    for i in range(N):
        dl = sum(O[i][d] * dO[i][d] for d in range(D)) if softmax else 0.0
        for j in range(N):
            dS[i][j] = P[i][j] * (sum(dO[i][d] * v[j][d] for d in range(D)) - dl)
    dV = [[r(sum(r(P[i][j]) * dO[i][d] for i in range(N))) for d in range(D)] for j in range(N)]
    dQ = [[r(2 * g * (sum(r(dS[i][j]) * k[j][d] for j in range(N))
                      - (0.0 if softmax else sum(dS[i]) * q[i][d]))) for d in range(D)] for i in range(N)]
    dK = [[r(2 * g * (sum(r(dS[i][j]) * q[i][d] for i in range(N)) - sum(dS[i][j] for i in range(N)) * k[j][d]))
           for d in range(D)] for j in range(N)]
    return O, dQ, dK, dV


def pin_rounded_vs_brute(o, softmax=True, causal=True, num_prefix=0, dtype="bf16"):
    """The vectorised model against the loops, with real bf16/fp16 rounding
    (whose effects are ~2^-9 / 2^-11, far above float64 noise)."""
    q, k, v, dO = rand(1, 1, 6, 5), rand(1, 1, 6, 5, scale=1.4), rand(1, 1, 6, 5), rand(1, 1, 6, 5)
    g = 0.4
    rnd = o.rounder(dtype)
    got = o.rounded_model(q, k, v, dO, g, softmax, causal, num_prefix, rnd=rnd, out_rnd=rnd)
    ref = brute_rounded(q[0, 0], k[0, 0], v[0, 0], dO[0, 0], g, softmax, rnd, causal, num_prefix)
    return all(np.abs(a[0, 0] - np.array(b)).max() < 1e-12 for a, b in zip(got, ref))


def pin_rounded_decode_vs_model(o, softmax=True):
    """decode_forward with rounding equals the last T output rows of
    rounded_model over the whole cache (full lengths)."""
    q, k, v = rand(1, 2, 9, 8), rand(1, 2, 9, 8, scale=1.2), rand(1, 2, 9, 8)
    g, T = 0.3, 3
    r = o.rounder("bf16")
    full = o.rounded_model(q, k, v, rand(1, 2, 9, 8), g, softmax, rnd=r, out_rnd=r)[0]
    dec, _ = o.decode_forward(q[:, :, -T:], k, v, g, softmax, rnd=r, out_rnd=r)
    return np.abs(dec - full[:, :, -T:]).max() < 1e-12


ALL_PINS += [
    lambda o: pin_rounded_decode_vs_model(o, True),
    lambda o: pin_rounded_decode_vs_model(o, False),
    lambda o: pin_rounded_identity_limit(o, True),
    lambda o: pin_rounded_identity_limit(o, False),
    lambda o: pin_rounded_identity_limit(o, True, True, 3),
    lambda o: pin_rounded_identity_limit(o, False, False),
    lambda o: pin_rounded_vs_brute(o, True),
    lambda o: pin_rounded_vs_brute(o, False),
    lambda o: pin_rounded_vs_brute(o, True, True, 2, "fp16"),
    lambda o: pin_rounded_vs_brute(o, False, False, 0, "fp16"),
]


def test_rounding_helpers():
    """bf16 / fp16 rounding against torch's own conversions (ties to even)."""
    x = np.concatenate([rand(4000, scale=3.0), [1 / 3, 2 / 3, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -7.2, 0.0]])
    np.testing.assert_array_equal(ro.round_bf16(x), t64(x).to(torch.bfloat16).double().numpy())
    np.testing.assert_array_equal(ro.round_fp16(x), t64(x).to(torch.float16).double().numpy())
    assert ro.round_bf16(np.array([1 + 2 ** -8]))[0] == 1.0 and ro.round_bf16(np.array([1 + 3 * 2 ** -8]))[0] == 1 + 2 ** -6


def test_rounded_model_error_is_bf16_sized():
    """With bf16 rounding the model moves O by about the relative bf16
    precision (2^-9 per rounded P, averaged over the row) -- and not by zero:
    the rounding is really applied."""
    q, k, v, dO = rand(1, 2, 64, 32), rand(1, 2, 64, 32), rand(1, 2, 64, 32), rand(1, 2, 64, 32)
    g = 1 / (2 * math.sqrt(32))
    exact = ro.rounded_model(q, k, v, dO, g)
    model = ro.rounded_model(q, k, v, dO, g, rnd=ro.round_bf16, out_rnd=ro.round_bf16)
    for a, b in zip(model, exact):
        rel = np.linalg.norm(a - b) / np.linalg.norm(b)
        assert 1e-4 < rel < 1e-2, rel


@pytest.mark.parametrize("i", range(len(ALL_PINS)))
def test_pin(i):
    assert ALL_PINS[i](ro)


# ---------------------------------------------------------------------------
# Invariants
# ---------------------------------------------------------------------------
def test_row0_sees_only_key0():
    q, k, v = rand(1, 2, 9, 8), rand(1, 2, 9, 8), rand(1, 2, 9, 8)
    O, _ = ro.softmax_forward(q, k, v, 0.2)
    np.testing.assert_allclose(O[:, :, 0], v[:, :, 0], rtol=0, atol=1e-15)


def test_equal_key_norms_reduce_to_sdpa():
    """With every ||k_j|| equal the key-norm penalty is a per-row constant, so
    RBF softmax attention equals textbook attention with scale 2*gamma."""
    q, k, v = rand(2, 2, 14, 16), rand(2, 2, 14, 16), rand(2, 2, 14, 16)
    k = 3.0 * k / np.linalg.norm(k, axis=-1, keepdims=True)
    g = 0.125
    ref = F.scaled_dot_product_attention(t64(q), t64(k), t64(v), is_causal=True, scale=2 * g).numpy()
    O, _ = ro.softmax_forward(q, k, v, g)
    np.testing.assert_allclose(O, ref, rtol=0, atol=1e-12)


def test_softmax_dS_rowsum_vanishes():
    """sum_j dS_ij = 0, so dQ does not depend on the -gamma||q||^2 term."""
    q, k, v, dO = (rand(1, 1, 10, 6) for _ in range(4))
    g = 0.3
    N = 10
    mask = ro.visibility(N)
    s = np.where(mask, ro.rbf_logits(q[0, 0], k[0, 0], g), -np.inf)
    P = np.exp(s - s.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    dP = dO[0, 0] @ v[0, 0].T
    dS = P * (dP - (P * dP).sum(-1, keepdims=True))
    assert np.abs(dS.sum(-1)).max() < 1e-13
    dQ, _, _ = ro.softmax_backward(q, k, v, dO, g)
    np.testing.assert_allclose(dQ[0, 0], 2 * g * dS @ k[0, 0], rtol=0, atol=1e-12)


def test_nonsoftmax_single_key_identity():
    q = rand(1, 1, 1, 8)
    v = rand(1, 1, 1, 8)
    O = ro.non_softmax_forward(q, q.copy(), v, 0.7)
    # exp(-gamma * 0) = 1 up to the rounding of the ||q||^2 + ||k||^2 - 2q.k expansion
    np.testing.assert_allclose(O, v, rtol=0, atol=1e-13)


def test_mask_matches_reference_causal_mask():
    """num_prefix = 0 is the reference's triu(1) mask (rbf_attention.py:1556-1565)."""
    for n in (1, 5, 33):
        ref = ~torch.ones(n, n, dtype=torch.bool).triu(1).numpy()
        assert (ro.visibility(n, True, 0) == ref).all()
        assert (ro.visibility(n, True, 1) == ref).all()  # key 0 is already visible to all
        assert ro.visibility(n, False).all()


def test_prefix_mask_rows():
    m = ro.visibility(8, True, 4)
    assert m[0, :4].all() and not m[0, 4:].any()
    assert m[2, 3] and not m[2, 4]
    assert m[6, :7].all() and not m[6, 7]


# ---------------------------------------------------------------------------
# Mutation tests: plausible mistakes planted in the oracle's own source must
# make at least one pin fail.
# ---------------------------------------------------------------------------
MUTATIONS = {
    "dropped_factor_2_in_cross_term": ("- 2.0 * q @ np.swapaxes(k, -1, -2)", "- q @ np.swapaxes(k, -1, -2)"),
    "dropped_key_norm": ("return -gamma * (qq + kk - 2.0", "return -gamma * (qq + 0 * kk - 2.0"),
    "strict_causal_mask": ("return (j <= i) | (j < num_prefix)", "return (j < i) | (j < num_prefix)"),
    "prefix_ignored": ("return (j <= i) | (j < num_prefix)", "return (j <= i)"),
    "dK_missing_colsum": (
        "dK[b, h] = 2.0 * gamma * (dS.T @ qs - dS.sum(axis=0)[:, None] * ks)\n    return dQ, dK, dV\n\n\ndef non_softmax_forward",
        "dK[b, h] = 2.0 * gamma * (dS.T @ qs)\n    return dQ, dK, dV\n\n\ndef non_softmax_forward",
    ),
    "dV_untransposed_P": ("dV[b, h] = P.T @ dos\n        dQ[b, h] = 2.0 * gamma * (dS @ ks - dS.sum(axis=1)[:, None] * qs)\n        dK[b, h] = 2.0 * gamma * (dS.T @ qs - dS.sum(axis=0)[:, None] * ks)\n    return dQ, dK, dV\n\n\ndef non_softmax_forward",
                          "dV[b, h] = P @ dos\n        dQ[b, h] = 2.0 * gamma * (dS @ ks - dS.sum(axis=1)[:, None] * qs)\n        dK[b, h] = 2.0 * gamma * (dS.T @ qs - dS.sum(axis=0)[:, None] * ks)\n    return dQ, dK, dV\n\n\ndef non_softmax_forward"),
    "delta_sign": ("dS = P * (dP - delta)", "dS = P * (dP + delta)"),
    "nonsoftmax_dQ_sign": (
        "dS = P * (dos @ vs.T)\n        dV[b, h] = P.T @ dos\n        dQ[b, h] = 2.0 * gamma * (dS @ ks - dS.sum(axis=1)[:, None] * qs)",
        "dS = P * (dos @ vs.T)\n        dV[b, h] = P.T @ dos\n        dQ[b, h] = 2.0 * gamma * (dS @ ks + dS.sum(axis=1)[:, None] * qs)",
    ),
    "lse_natural_log": ("* LOG2E\n    return O, L", "\n    return O, L"),
    "lse_missing_qnorm": ("L[b, h] = (m + np.log(l) + gamma * np.einsum(\"nd,nd->n\", qs, qs)) * LOG2E",
                          "L[b, h] = (m + np.log(l)) * LOG2E"),
    "augment_wrong_half": ("kp = np.concatenate([k, -0.5 * kk], axis=-1)", "kp = np.concatenate([k, -kk], axis=-1)"),
    "decode_position_off_by_one": ("pos = np.arange(n - T, n)[:, None]", "pos = np.arange(n - T - 1, n - 1)[:, None]"),
    "decode_ignores_lengths": ("lens = [Lc] * B if lens is None else [int(x) for x in lens]", "lens = [Lc] * B"),
    # the rounding model: rounding at the wrong places, or a dropped term
    "rounded_colsum_of_rounded_dS": ("grad_s.sum(axis=0)[:, None] * ks))", "r_gs.sum(axis=0)[:, None] * ks))"),
    "rounded_dV_unrounded_P": ("out_rnd(rnd(prob).T @ dos)", "out_rnd(prob.T @ dos)"),
    "rounded_delta_from_unstored_O": ("(o_st * dos).sum(axis=-1, keepdims=True)",
                                      "((rnd(ex) @ vs) / den * dos).sum(axis=-1, keepdims=True)"),
    "rounded_row_sum_of_rounded_P": ("den = ex.sum(axis=-1, keepdims=True)", "den = rnd(ex).sum(axis=-1, keepdims=True)"),
    "rounded_nonsoftmax_dQ_norm_term": ("q_term = grad_s.sum(axis=1)[:, None] * qs", "q_term = 0.0"),
    "rounded_decode_unrounded_P": ("out_rnd(rnd(np.exp(s)) @ v[b, h, :n])", "out_rnd(np.exp(s) @ v[b, h, :n])"),
    "rounded_decode_row_sum_of_rounded_P": ("out_rnd((rnd(e) @ v[b, h, :n]) / l)",
                                            "out_rnd((rnd(e) @ v[b, h, :n]) / rnd(e).sum(axis=-1, keepdims=True))"),
    "rounded_dQ_unrounded_dS": ("out_rnd(2.0 * gamma * (r_gs @ ks - q_term))", "out_rnd(2.0 * gamma * (grad_s @ ks - q_term))"),
}


def _mutant(name):
    src = inspect.getsource(ro)
    old, new = MUTATIONS[name]
    assert src.count(old) == 1, f"mutation {name}: anchor not found exactly once"
    mod = types.ModuleType(f"ro_mutant_{name}")
    exec(compile(src.replace(old, new), f"<mutant {name}>", "exec"), mod.__dict__)
    return mod


@pytest.mark.parametrize("name", sorted(MUTATIONS))
def test_pins_catch_mutation(name):
    m = _mutant(name)
    results = []
    for pin in ALL_PINS:
        try:
            results.append(bool(pin(m)))
        except Exception:
            results.append(False)
    assert not all(results), f"no pin detects the mutation {name}"
