"""Position term fused into the Q/K reads (the model's SuSiE embedding,
rbf_attention.py:1666-1688): attention(q, k, v, pos=P) must equal
attention(q + P, k + P, v), forward and gradients, and autograd must return
dP = sum_b (dq + dk) for a term shared by the batch."""
import math

import pytest
import torch

import rbf_attention_amd as ra
from rbf_attention_amd import _lib

pytestmark = pytest.mark.gpu


def inputs(B, H, N, D, dtype, dev, seed, shared=True):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, N, D, generator=g).to(dtype).to(dev) for _ in range(4))
    P = (torch.randn(1 if shared else B, H, N, D, generator=g) * 0.5).to(dtype).to(dev)
    return q, k, v, do, P


def run(fn, q, k, v, do, P, fused, **kw):
    q, k, v = (t.clone().requires_grad_(True) for t in (q, k, v))
    if fused:
        P = P.clone().requires_grad_(True)
        out = fn(q, k, v, True, pos=P, **kw)
    else:
        out = fn(q + P, k + P, v, True, **kw)
    out.backward(do)
    torch.cuda.synchronize()
    return out.detach(), q.grad, k.grad, v.grad, (P.grad if fused else None)


@pytest.mark.parametrize(
    "B,H,N,D,dtype,softmax,shared",
    [
        (16, 16, 516, 64, torch.bfloat16, True, True),
        (16, 16, 300, 64, torch.bfloat16, False, True),
        (16, 16, 516, 64, torch.float16, True, True),
        (16, 16, 200, 40, torch.bfloat16, True, False),
    ],
)
def test_fused_pos_equals_added_inputs(cuda_device, B, H, N, D, dtype, softmax, shared):
    """B*H = 256: fused and unfused calls take the same head-resident
    kernels, so the results agree bit for bit."""
    q, k, v, do, P = inputs(B, H, N, D, dtype, cuda_device, seed=N + D, shared=shared)
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    kw = dict(sm_scale=1.0 / (2 * math.sqrt(D)))
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = B, H, N, D, 1, 0.1
    assert _lib.pos_supported(a)
    fused = run(fn, q, k, v, do, P, True, **kw)
    plain = run(fn, q, k, v, do, P, False, **kw)
    for name, x, y in zip(("O", "dQ", "dK", "dV"), fused[:4], plain[:4]):
        assert torch.equal(x, y), f"{name}: max diff {(x.float() - y.float()).abs().max().item():.3e}"
    dq, dk = plain[1].float(), plain[2].float()
    dP = (dq + dk).sum(0, keepdim=True) if shared else dq + dk
    err = (fused[4].float() - dP).abs().max().item()
    assert err <= 1e-2 * max(1.0, dP.abs().max().item()), err


@pytest.mark.parametrize("B,H,D", [(2, 2, 64), (2, 2, 128)])
def test_pos_small_batch_and_fallback(cuda_device, B, H, D):
    """Few heads (fused, head-resident kernels) and D = 128 (not fused: the
    op adds the term itself): same values as the unfused call within the
    bf16 tolerance of the parity tests."""
    q, k, v, do, P = inputs(B, H, 300, D, torch.bfloat16, cuda_device, seed=D)
    fused = run(ra.run_triton_rbf, q, k, v, do, P, True, sm_scale=0.05)
    plain = run(ra.run_triton_rbf, q, k, v, do, P, False, sm_scale=0.05)
    for name, x, y in zip(("O", "dQ", "dK", "dV"), fused[:4], plain[:4]):
        x, y = x.double(), y.double()
        rel = ((x - y).norm() / y.norm()).item()
        assert rel <= 1e-2, f"{name}: rel_l2 {rel:.3e}"


def test_pos_against_oracle_c5_shape(cuda_device):
    """The model's shape (config 5: B*H = 256 heads, N = 512 + 4 registers,
    D = 64, bf16, a SuSiE-like term shared by the batch, token-major output,
    the reference's gamma = 1/sqrt(D)) against the float64 oracle evaluated on
    bf16(q + P) and bf16(k + P) (the sums the model's separate adds would
    store, rbf_attention.py:1666-1688): O, dQ, dK, dV on six (b, h) slices,
    and the term's gradient dP = sum_b (dq + dk) on two heads (all 32 batch
    entries each)."""
    import numpy as np

    from oracle import rbf_oracle as ro
    from test_parity_gpu import check, np64

    B, H, N, D = 32, 8, 516, 64
    gamma = 1.0 / math.sqrt(D)
    q, k, v, do, _ = inputs(B, H, N, D, torch.bfloat16, cuda_device, seed=5)
    g = torch.Generator().manual_seed(6)
    t = torch.arange(N - 4, dtype=torch.float32)[:, None] / (10000.0 ** (torch.arange(0, D, 2) / D))
    sus = torch.cat([t.sin(), t.cos()], -1)  # the SuSiE table, rows 4..N-1
    P = torch.cat([torch.randn(H, 4, D, generator=g) * 0.02, sus.expand(H, N - 4, D)], 1)[None]
    P = P.to(torch.bfloat16).to(cuda_device)
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0, _lib.DTYPE_CODES[torch.bfloat16]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = B, H, N, D, 1, gamma
    assert _lib.pos_supported(a)
    qq, kk, vv, pp = (x.clone().requires_grad_(True) for x in (q, k, v, P))
    out = ra.run_triton_rbf(qq, kk, vv, True, pos=pp, token_major=True)
    assert out.transpose(1, 2).is_contiguous()
    out.backward(do)
    torch.cuda.synchronize()
    qs, ks = (q + P), (k + P)  # rounded to bf16, as the model's adds store them
    r = ro.rounder("bf16")
    for b, h in ((0, 0), (5, 2), (13, 4), (20, 1), (27, 6), (31, 7)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        arr = [np64(x)[sl] for x in (qs, ks, v, do)]
        O, _ = ro.softmax_forward(arr[0], arr[1], arr[2], gamma)
        grads = ro.softmax_backward(*arr, gamma)
        model = ro.rounded_model(*arr, gamma, rnd=r, out_rnd=r)
        for i, (name, got, ref) in enumerate(zip(("O", "dQ", "dK", "dV"), (out, qq.grad, kk.grad, vv.grad),
                                                 (O,) + grads)):
            check(f"pos C5 b{b}h{h} {name}", got[sl], ref, torch.bfloat16, kind=name, model=model[i])
    for h in (0, 7):
        arr = [np64(x)[:, h:h + 1] for x in (qs, ks, v, do)]
        dq, dk, _ = ro.softmax_backward(*arr, gamma)
        dP = (dq + dk).sum(axis=0, keepdims=True)
        check(f"pos C5 dP h{h}", pp.grad[:, h:h + 1], dP, torch.bfloat16)
        assert np.isfinite(np64(pp.grad)).all()


@pytest.mark.parametrize(
    "B,H,N,D,dtype,softmax,shared,causal,npre",
    [
        (2, 3, 700, 64, torch.bfloat16, True, True, True, 0),  # N > 576
        (2, 2, 300, 128, torch.bfloat16, True, False, True, 0),  # D = 128 (paired dK/dV kernel)
        (2, 2, 260, 32, torch.bfloat16, False, True, True, 0),  # D = 32, non-softmax
        (1, 3, 700, 64, torch.float16, True, True, False, 0),  # fp16, not causal
        (2, 2, 650, 64, torch.bfloat16, True, False, True, 4),  # register tokens seen by every query
        (2, 2, 150, 64, torch.float32, True, True, True, 0),  # fp32
        (2, 2, 150, 96, torch.float32, False, False, True, 0),  # fp32, D = 96 padded to 128
    ],
)
def test_pos_streaming_against_oracle(cuda_device, B, H, N, D, dtype, softmax, shared, causal, npre):
    """Shapes outside the head-resident kernels: the op adds the term (q + P,
    k + P, each sum rounded to the element type) and runs the streaming
    kernels; autograd forms the term's gradient.  O, dQ, dK, dV against the
    float64 oracle evaluated on those rounded sums, to the parity tests'
    bounds (and, for 16-bit types, within the rounding model's ratio), and the
    term's gradient against the oracle's sum_b (dq + dk) (dq + dk per batch
    entry for a per-batch term)."""
    import numpy as np

    from oracle import rbf_oracle as ro
    from test_parity_gpu import check, np64

    gamma = 1.0 / (2 * math.sqrt(D))
    q, k, v, do, P = inputs(B, H, N, D, dtype, cuda_device, seed=N + D + B, shared=shared)
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = B, H, N, D, int(causal), gamma
    assert not _lib.pos_supported(a)
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    qq, kk, vv, pp = (x.clone().requires_grad_(True) for x in (q, k, v, P))
    out = fn(qq, kk, vv, causal, sm_scale=gamma, num_prefix=npre, pos=pp)
    out.backward(do)
    torch.cuda.synchronize()
    qs, ks = q + P, k + P  # rounded to the element type, as separate adds store them
    fwd = ro.softmax_forward if softmax else ro.non_softmax_forward
    bwd = ro.softmax_backward if softmax else ro.non_softmax_backward
    r = ro.rounder("bf16" if dtype == torch.bfloat16 else "fp16") if dtype != torch.float32 else None
    name0 = f"pos stream {str(dtype)[6:]} N{N} D{D} {'sm' if softmax else 'ns'}{'' if causal else ' nc'} p{npre}"
    for b in range(B):
        for h in range(H):
            sl = (slice(b, b + 1), slice(h, h + 1))
            arr = [np64(x)[sl] for x in (qs, ks, v, do)]
            O = fwd(arr[0], arr[1], arr[2], gamma, causal, npre)
            O = O[0] if softmax else O
            grads = bwd(*arr, gamma, causal, npre)
            model = (ro.rounded_model(*arr, gamma, softmax=softmax, causal=causal, num_prefix=npre, rnd=r, out_rnd=r)
                     if r is not None else [None] * 4)
            for i, (name, got, ref) in enumerate(zip(("O", "dQ", "dK", "dV"), (out, qq.grad, kk.grad, vv.grad),
                                                     (O,) + tuple(grads))):
                check(f"{name0} b{b}h{h} {name}", got[sl], ref, dtype, kind=name, model=model[i])
    for h in range(H):
        arr = [np64(x)[:, h:h + 1] for x in (qs, ks, v, do)]
        dq, dk, _ = bwd(*arr, gamma, causal, npre)
        dP = (dq + dk).sum(axis=0, keepdims=True) if shared else dq + dk
        check(f"{name0} dP h{h}", pp.grad[:, h:h + 1], dP, dtype)
    assert np.isfinite(np64(pp.grad)).all()


def draw_fused_cases(n, seed=1688):
    """The fused path's whole range, every dimension drawn at once: 16-bit,
    32 < D <= 64, N <= 576 (the head-resident kernels take a term at any
    number of heads), a term shared by the batch or one per entry, both
    variants, masks, register prefixes, gamma, token-major output."""
    import numpy as np

    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        D = 8 * int(rng.integers(5, 9))
        # log-uniform over 1..576, or uniform over the longest heads 400..576
        N = int(np.exp(rng.uniform(0.0, np.log(576.0)))) if rng.random() < 0.5 else int(rng.integers(400, 577))
        if rng.random() < 0.4:  # at least one head per CU, as at the model's shape
            B, H = int(rng.integers(16, 41)), 16
        else:
            B, H = int(rng.integers(1, 41)), int(rng.choice([1, 2, 4, 8]))
        dtype = (torch.bfloat16, torch.float16)[int(rng.random() < 0.35)]
        softmax = bool(rng.random() < 0.6)
        causal = bool(rng.random() < 0.8)
        npre = 0 if rng.random() < 0.5 else int(rng.integers(1, min(N, 64) + 1))
        gamma = float(rng.choice([1.0 / math.sqrt(D), 0.5 / math.sqrt(D), rng.uniform(0.02, 0.2)]))
        shared = bool(rng.random() < 0.6)
        token_major = bool(rng.random() < 0.35)
        cases.append((i, B, H, N, D, dtype, softmax, causal, npre, gamma, shared, token_major))
    return cases


FUSED_CASES = draw_fused_cases(16)


def fused_id(c):
    i, B, H, N, D, dtype, softmax, causal, npre, gamma, shared, tm = c
    return (f"f{i}_B{B}H{H}N{N}D{D}_{str(dtype)[6:]}_{'sm' if softmax else 'ns'}_{'causal' if causal else 'full'}"
            f"_p{npre}_{'shared' if shared else 'perbatch'}{'_tm' if tm else ''}")


def test_fused_draw_coverage():
    """The draw spans fewer and more heads than the 256 CUs, both variants,
    both kinds of term, short and long heads and token-major output."""
    heads = [c[1] * c[2] for c in FUSED_CASES]
    assert min(heads) < 256 <= max(heads)
    assert {c[6] for c in FUSED_CASES} == {True, False} and {c[10] for c in FUSED_CASES} == {True, False}
    assert min(c[3] for c in FUSED_CASES) < 64 and max(c[3] for c in FUSED_CASES) > 448
    assert any(c[11] for c in FUSED_CASES) and any(c[8] for c in FUSED_CASES)


@pytest.mark.parametrize("case", FUSED_CASES, ids=fused_id)
def test_fused_pos_random_against_oracle(cuda_device, case):
    """The fused term against the float64 oracle on the rounded sums
    (q + P, k + P): O, dQ, dK, dV on the first and last (b, h) slices, and the
    term's gradient on the last head (sum over the batch for a shared term)."""
    import numpy as np

    from oracle import rbf_oracle as ro
    from test_parity_gpu import check, np64

    i, B, H, N, D, dtype, softmax, causal, npre, gamma, shared, token_major = case
    q, k, v, do, P = inputs(B, H, N, D, dtype, cuda_device, seed=4000 + i, shared=shared)
    if not softmax:  # keep the unnormalised weights away from underflow
        q, k, P = q * 0.5, k * 0.5, P * 0.5
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = B, H, N, D, int(causal), gamma
    assert _lib.pos_supported(a)
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    qq, kk, vv, pp = (x.clone().requires_grad_(True) for x in (q, k, v, P))
    print(f"case {fused_id(case)} gamma={gamma:.4f}", flush=True)
    out = fn(qq, kk, vv, causal, sm_scale=gamma, num_prefix=npre, pos=pp, token_major=token_major)
    out.backward(do)
    torch.cuda.synchronize()
    if token_major:  # (B, H, N, D) view of (B, N, H, D) storage
        assert out.shape == (B, H, N, D) and out.transpose(1, 2).is_contiguous()
    qs, ks = q + P, k + P  # rounded to the element type, as separate adds store them
    fwd = ro.softmax_forward if softmax else ro.non_softmax_forward
    bwd = ro.softmax_backward if softmax else ro.non_softmax_backward
    r = ro.rounder("bf16" if dtype == torch.bfloat16 else "fp16")
    for b, h in ((0, 0), (B - 1, H - 1)):
        sl = (slice(b, b + 1), slice(h, h + 1))
        arr = [np64(x)[sl] for x in (qs, ks, v, do)]
        O = fwd(arr[0], arr[1], arr[2], gamma, causal, npre)
        O = O[0] if softmax else O
        grads = bwd(*arr, gamma, causal, npre)
        model = ro.rounded_model(*arr, gamma, softmax=softmax, causal=causal, num_prefix=npre, rnd=r, out_rnd=r)
        for j, (name, got, ref) in enumerate(zip(("O", "dQ", "dK", "dV"), (out, qq.grad, kk.grad, vv.grad),
                                                 (O,) + tuple(grads))):
            check(f"{fused_id(case)} b{b}h{h} {name}", got[sl], ref, dtype, kind=name, model=model[j])
    h = H - 1
    arr = [np64(x)[:, h:h + 1] for x in (qs, ks, v, do)]
    dq, dk, _ = bwd(*arr, gamma, causal, npre)
    dP = (dq + dk).sum(axis=0, keepdims=True) if shared else dq + dk
    check(f"{fused_id(case)} dP h{h}", pp.grad[:, h:h + 1], dP, dtype)
    assert np.isfinite(np64(pp.grad)).all()
