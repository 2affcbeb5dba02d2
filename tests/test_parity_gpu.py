"""GPU parity of the HIP kernels against the CPU oracle (float64 restatement
of the reference math, oracle/rbf_oracle.py) on identical seeded inputs.

Tolerances (plus what storing a result in bf16 and the
reference kernels' own roundings make unavoidable):
  * fp32 inputs: max-abs error <= 1e-4 on O, dQ, dK, dV.
  * bf16 / fp16 inputs, every tensor: relative L2 error <= 1e-2.
  * O and dV, elementwise: |got - ref| <= 2e-2 + half an ulp of |ref| in the
    element type (storing a value of magnitude >= 8 in bf16 alone moves it by
    up to 2^-5 > 2e-2).  Where the rounding model below misses that bound on
    some elements (C4: ~2000-term unnormalised sums of bf16-rounded P), the
    kernel may miss it on at most 1.25x as many.
  * dQ and dK, tensor-wide: max |got - ref| <= 2e-2 + 2^-7 max|ref|.  An
    elementwise bound would be wrong for dK = 2g(dS^T Q - colsum(dS) k), whose
    small entries come from the cancellation of large terms.
  * Against the rounding model (oracle.rbf_oracle.rounded_model: the exact
    math with P and dS rounded to the element type where the reference
    kernels round them, rbf_attention.py:201, 422, 432, 621, and outputs
    rounded): the kernel's relative L2 error is at most 1.2x the model's, on
    tensors of >= 4096 elements (fewer make the ratio noisy).  So the
    kernels' errors are those of the reference's own arithmetic, not more.
    Not for dQ/dK of the far-query cases: with |q| ~ 48 their dK amplifies
    the output rounding of a few rows' O (through Delta) by |q|, so one
    realization of that rounding against another differs by up to ~1.4x (a
    CPU backward fed the kernel's own O and L reproduces its dK exactly, and
    the kernel's per-row O and Delta errors are distributed as the model's).
  * A reference that is zero or numerically zero, every entry below 1e-5
    next to inputs of order 1 (dQ for N = 1: one visible key, dS = 0; for
    N = 2 with a nearly one-hot P: ~4e-7), is checked with max-abs <= 1e-5
    instead of a relative norm, which there measures only rounding noise.
  * dQ and dK at N <= 2 are checked at rel-L2 <= 3e-2: with one or two
    visible keys they are proportional to a single dS_ij, and Delta_i = rowsum(O * dO) is
    taken from the bf16 output as in the reference kernel
    (rbf_attention.py:275-276), whose rounding then sets the relative error.
  * Where the rounding model itself misses the rel-L2 bound (dQ of a
    handful of visible keys, e.g. N = 6 in fp16: 1.86e-2), the kernel's
    rel-L2 may not exceed 1.2x the model's, whatever the tensor's size.
Big configurations are compared on sampled (b, h) slices -- every slice is an
independent problem -- plus size-independent properties at full size.
Set RBF_PARITY_LOG=<file> to append every comparison's metrics as JSON lines.
"""
import json
import math
import os

import numpy as np
import pytest
import torch

import rbf_attention_amd as ra
from oracle import rbf_oracle as ro
from rbf_attention_amd import _lib
from rbf_attention_amd import workloads as wl

pytestmark = pytest.mark.gpu

ULP_BF16 = 2.0 ** -7
DTYPE_NAMES = {torch.bfloat16: "bf16", torch.float16: "fp16", torch.float32: "fp32"}
MODEL_RATIO = 1.2  # kernel rel-L2 error / rounding model's, at most
MODEL_MIN_ELEMS = 4096


def np64(t):
    return t.detach().to("cpu", torch.float64).numpy()


def half_ulp(x, dtype):
    """Half the spacing of the element type's numbers at |x| (0 at x = 0)."""
    mant = 10 if dtype == torch.float16 else 7
    a = np.abs(x)
    e = np.floor(np.log2(np.where(a > 0, a, 1.0)))
    return np.where(a > 0, np.exp2(e - mant - 1), 0.0)


def errors(got, ref, dtype, elementwise):
    err = np.abs(got - ref)
    ref_norm = np.linalg.norm(ref)
    out = {
        "max_abs": float(err.max()) if err.size else 0.0,
        "rel_l2": float(np.linalg.norm(got - ref) / ref_norm) if ref_norm > 0 else float("nan"),
        "max_ref": float(np.abs(ref).max()) if ref.size else 0.0,
    }
    if elementwise and err.size:
        out["n_viol"] = int((err > 2e-2 + half_ulp(ref, dtype)).sum())
    return out


def check(name, got, ref, dtype, rel_l2_max=1e-2, kind=None, model=None, model_ratio=True):
    """kind: "O"/"dV" (elementwise bound), "dQ"/"dK" (tensor-wide bound), or
    None (tensor-wide, for comparisons against something other than the
    oracle); model: the rounding model's output for the same inputs, whose
    error the kernel's may exceed by MODEL_RATIO at most (if model_ratio)."""
    got = np64(got)
    elementwise = kind in ("O", "dV") and dtype != torch.float32
    e = errors(got, ref, dtype, elementwise)
    m = errors(model, ref, dtype, elementwise) if model is not None else None
    info = (f"{name}: max_abs={e['max_abs']:.3e} rel_l2={e['rel_l2']:.3e} max|ref|={e['max_ref']:.3e}"
            + (f" viol={e['n_viol']}" if elementwise else "")
            + (f" | model max_abs={m['max_abs']:.3e} rel_l2={m['rel_l2']:.3e}"
               + (f" viol={m['n_viol']}" if elementwise else "") if m else ""))
    print(info, flush=True)
    log = os.environ.get("RBF_PARITY_LOG")
    if log:
        with open(log, "a") as f:
            f.write(json.dumps({"name": name, "dtype": str(dtype), **e, "model": m}) + "\n")
    assert np.isfinite(got).all(), f"{name}: non-finite values"
    if dtype == torch.float32:
        assert e["max_abs"] <= 1e-4, info
        return
    if not e["max_ref"] >= 1e-5:
        assert e["max_abs"] <= 1e-5, info
        return
    rel_max = rel_l2_max
    if m is not None and m["rel_l2"] > rel_l2_max:
        # the reference's own arithmetic misses the bound: the kernel may not do worse
        rel_max = MODEL_RATIO * m["rel_l2"]
    assert e["rel_l2"] <= rel_max, info
    if elementwise:
        allowed = 0 if m is None else math.ceil(1.25 * m["n_viol"])
        assert e["n_viol"] <= allowed, info
    else:
        assert e["max_abs"] <= 2e-2 + ULP_BF16 * e["max_ref"], info
    if m is not None and model_ratio and ref.size >= MODEL_MIN_ELEMS:
        assert e["rel_l2"] <= MODEL_RATIO * m["rel_l2"] + 1e-6, info


def run_ours(q, k, v, do, softmax, causal, gamma, num_prefix):
    q, k, v = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    out = fn(q, k, v, causal, sm_scale=gamma, num_prefix=num_prefix)
    out.backward(do)
    torch.cuda.synchronize()
    return out, q.grad, k.grad, v.grad


def oracle_all(q, k, v, do, softmax, causal, gamma, num_prefix, sl=None, with_model=False):
    """(O, dQ, dK, dV) of the float64 oracle, its L (softmax), and -- when
    with_model and the inputs are 16-bit -- the rounding model's outputs."""
    arrs = [np64(t) for t in (q, k, v, do)]
    if sl is not None:
        arrs = [a[sl] for a in arrs]
    qn, kn, vn, don = arrs
    if softmax:
        O, L = ro.softmax_forward(qn, kn, vn, gamma, causal, num_prefix)
        refs = (O,) + ro.softmax_backward(qn, kn, vn, don, gamma, causal, num_prefix)
    else:
        O, L = ro.non_softmax_forward(qn, kn, vn, gamma, causal, num_prefix), None
        refs = (O,) + ro.non_softmax_backward(qn, kn, vn, don, gamma, causal, num_prefix)
    model = None
    if with_model and q.dtype != torch.float32:
        r = ro.rounder(DTYPE_NAMES[q.dtype])
        model = ro.rounded_model(qn, kn, vn, don, gamma, softmax, causal, num_prefix, rnd=r, out_rnd=r)
    return refs, L, model


def compare_case(q, k, v, do, softmax=True, causal=True, gamma=None, num_prefix=0, sl=None, tag="", outs=None,
                 ill_conditioned=False):
    """Runs the kernels (unless their outputs are given) and checks O, dQ, dK,
    dV -- on the (b, h) slices sl, if given -- against the oracle.
    ill_conditioned: queries far from every key (see the module docstring):
    no rounding-model ratio for dQ and dK."""
    D = q.shape[-1]
    g = gamma if gamma is not None else 1.0 / math.sqrt(D)
    print(f"case {tag} shape={tuple(q.shape)} {q.dtype} softmax={softmax} causal={causal} "
          f"gamma={g:.5f} num_prefix={num_prefix}", flush=True)
    if outs is None:
        outs = run_ours(q, k, v, do, softmax, causal, gamma, num_prefix)
    refs, _, model = oracle_all(q, k, v, do, softmax, causal, g, num_prefix, sl, with_model=True)
    for i, (name, got, ref) in enumerate(zip(("O", "dQ", "dK", "dV"), outs, refs)):
        rel = 3e-2 if (name in ("dQ", "dK") and q.shape[2] <= 2) else 1e-2
        check(f"{tag} {name}", got if sl is None else got[sl], ref, q.dtype, rel, kind=name,
              model=None if model is None else model[i],
              model_ratio=not (ill_conditioned and name in ("dQ", "dK")))
    return outs


def to_dev(ts, dev):
    return [t.to(dev) for t in ts]


# ---------------------------------------------------------------------------
# Benchmark configurations
# ---------------------------------------------------------------------------
def test_c1_tiny_fp32(cuda_device):
    w = wl.C1_TINY
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    compare_case(q, k, v, do, gamma=w.sm_scale, tag="C1")


def test_c1_reference_default_gamma_through_v5_ops(cuda_device):
    """gamma = 1/sqrt(D) through torch.ops.rbf_attn_v5 and its autograd."""
    w = wl.C1_TINY
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    compare_case(q, k, v, do, gamma=None, tag="C1-v5")


def test_c1_lse_matches_oracle(cuda_device):
    w = wl.C1_TINY
    q, k, v, _ = to_dev(wl.make_inputs(w), cuda_device)
    out, L = torch.ops.rbf_attn_amd.scaled_fwd_ex(q, k, v, True, w.sm_scale, 0)
    _, Lref = ro.softmax_forward(np64(q), np64(k), np64(v), w.sm_scale)
    err = np.abs(np64(L) - Lref).max()
    print(f"L max_abs={err:.3e}")
    assert err <= 1e-4


@pytest.mark.parametrize("gamma_kind", ["baseline", "reference"])
def test_c2_model_bf16(cuda_device, gamma_kind):
    w = wl.C2_MODEL
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    gamma = w.sm_scale if gamma_kind == "baseline" else None
    compare_case(q, k, v, do, gamma=gamma, tag=f"C2-{gamma_kind}")


def test_c2_registers_visible_to_all(cuda_device):
    w = wl.C2_MODEL.with_(B=4)
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    compare_case(q, k, v, do, gamma=w.sm_scale, num_prefix=4, tag="C2-prefix4")


@pytest.fixture(scope="module")
def c3_run(cuda_device):
    """C3 inputs and kernel outputs (about 1 GiB on the GPU), computed once for
    the slice checks and freed when the module's tests are done, whichever of
    them run and in whatever order."""
    w = wl.C3_LONG
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    outs = run_ours(q, k, v, do, True, True, w.sm_scale, 0)
    yield (q, k, v, do), outs
    del q, k, v, do, outs
    torch.cuda.empty_cache()


@pytest.mark.parametrize("b,h", [(0, 0), (1, 5), (2, 10), (3, 15)])
def test_c3_long_bf16_sampled(c3_run, b, h):
    """Four (b, h) slices of C3 against the oracle, the last head included."""
    (q, k, v, do), outs = c3_run
    sl = (slice(b, b + 1), slice(h, h + 1))
    compare_case(q, k, v, do, gamma=wl.C3_LONG.sm_scale, sl=sl, tag=f"C3 b{b}h{h}", outs=outs)


def test_c3_long_bf16_full_size_properties(c3_run):
    """Finite everywhere; the zero register row 0 sees only key 0 (v_0 = 0),
    so O[:, :, 0] == 0 exactly."""
    _, outs = c3_run
    for t in outs:
        assert torch.isfinite(t).all()
    assert (outs[0][:, :, 0] == 0).all()


def test_c4_nonsoftmax_bf16_sampled(cuda_device):
    w = wl.C4_NONSOFTMAX
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    sl = (slice(1, 16, 2), slice(1, 8, 3))  # 8 x 3 = 24 slices, the last (b, h) = (15, 7) included
    outs = compare_case(q, k, v, do, softmax=False, gamma=w.sm_scale, sl=sl, tag="C4")
    for t in outs:
        assert torch.isfinite(t).all()


# ---------------------------------------------------------------------------
# Shapes, dtypes, masks, variants
# ---------------------------------------------------------------------------
def rand_inputs(B, H, N, D, dtype, dev, std=1.0, seed=0, key_scale=0.0):
    w = wl.Workload("adhoc", B=B, H=H, content=N, D=D, dtype={torch.bfloat16: "bf16", torch.float16: "fp16",
                                                            torch.float32: "fp32"}[dtype],
                    registers=0, std=std, key_lognormal=key_scale, seed=seed)
    return to_dev(wl.make_inputs(w), dev)


@pytest.mark.parametrize("N", [1, 2, 31, 32, 33, 64, 65, 100, 129, 255])
@pytest.mark.parametrize("softmax", [True, False])
def test_ragged_lengths(cuda_device, N, softmax):
    q, k, v, do = rand_inputs(2, 2, N, 64, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=N)
    compare_case(q, k, v, do, softmax=softmax, tag=f"N{N}")


@pytest.mark.parametrize("D", [8, 16, 40, 60, 72, 96, 128])
def test_head_dims(cuda_device, D):
    q, k, v, do = rand_inputs(1, 3, 77, D, torch.bfloat16, cuda_device, seed=D)
    compare_case(q, k, v, do, tag=f"D{D}")


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.float32, torch.bfloat16])
@pytest.mark.parametrize("softmax", [True, False])
def test_dtypes(cuda_device, dtype, softmax, D):
    q, k, v, do = rand_inputs(2, 2, 150, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=3)
    compare_case(q, k, v, do, softmax=softmax, tag=f"{dtype} D{D}")


@pytest.mark.parametrize("causal,num_prefix", [(False, 0), (True, 4), (True, 40), (True, 300)])
@pytest.mark.parametrize("softmax", [True, False])
def test_masks(cuda_device, causal, num_prefix, softmax):
    q, k, v, do = rand_inputs(1, 2, 200, 64, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=7)
    compare_case(q, k, v, do, softmax=softmax, causal=causal, num_prefix=num_prefix, gamma=0.0625,
                 tag=f"mask c{causal} p{num_prefix}")


@pytest.mark.parametrize(
    "D,N,dtype,softmax,causal,num_prefix",
    [(128, 2200, torch.bfloat16, True, False, 0), (128, 2200, torch.bfloat16, True, True, 40),
     (128, 2200, torch.float16, False, True, 300), (64, 4300, torch.bfloat16, True, False, 0),
     (64, 4300, torch.bfloat16, False, True, 300), (64, 4300, torch.float16, True, True, 4)],
)
def test_masks_long(cuda_device, D, N, dtype, softmax, causal, num_prefix):
    """Non-causal and register-token masks on the long-sequence streaming
    kernels with LDS-DMA tiles (D = 128: paired dK/dV kernel; D = 64: DMA
    dK/dV from N = 4096), whose query-tile ranges start at the first tile when
    keys are visible to every query."""
    q, k, v, do = rand_inputs(1, 1, N, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=N + D + num_prefix)
    compare_case(q, k, v, do, softmax=softmax, causal=causal, num_prefix=num_prefix, gamma=1.0 / (2 * math.sqrt(D)),
                 tag=f"mask long D{D} N{N} {dtype} sm{softmax} c{causal} p{num_prefix}")


@pytest.mark.parametrize("D", [64, 128])
def test_heavy_tailed_keys(cuda_device, D):
    q, k, v, do = rand_inputs(2, 4, 300, D, torch.bfloat16, cuda_device, seed=11, key_scale=0.5)
    compare_case(q, k, v, do, gamma=1.0 / (2 * math.sqrt(D)), tag=f"lognormal D{D}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32, torch.float16])
@pytest.mark.parametrize("shift", [3.9, 6.0])
def test_queries_far_from_every_key(cuda_device, dtype, shift):
    """Queries of the first 90 tokens of every other head moved far from all
    keys, so that even their nearest key sits ~100 (shift 3.9) or ~220
    (shift 6) powers of two below the forward's static logit bound
    c*0.5*||q||^2.  The first case stays on the static offset with row sums
    near 2^-40; the second drops below 2^-60 and makes those work-groups
    recompute with an online max."""
    q, k, v, do = rand_inputs(2, 4, 200, 64, dtype, cuda_device, seed=17)
    q = q.clone()
    q[:, ::2, :90] += shift
    compare_case(q, k, v, do, gamma=0.0625, tag=f"far{shift} {dtype}", ill_conditioned=True)


@pytest.mark.parametrize(
    "N,D,dtype,softmax,causal,num_prefix,shift",
    [
        (516, 64, torch.bfloat16, False, True, 0, 0.0),
        (300, 64, torch.bfloat16, True, False, 0, 0.0),
        (516, 64, torch.bfloat16, True, True, 4, 0.0),
        (300, 64, torch.float16, True, True, 0, 0.0),
        (200, 40, torch.bfloat16, True, True, 0, 0.0),
        (300, 64, torch.bfloat16, True, True, 0, 6.0),
        (576, 64, torch.bfloat16, True, True, 0, 0.0),  # 18 blocks: the largest head that fits LDS
        (576, 64, torch.bfloat16, False, True, 0, 0.0),
        (577, 64, torch.bfloat16, True, True, 0, 0.0),  # one token more: the streaming kernels
    ],
)
def test_head_resident_shapes(cuda_device, N, D, dtype, softmax, causal, num_prefix, shift):
    """B*H = 256 heads of at most 576 tokens: the forward and dQ run as one
    work-group per head with the head's K and V resident in LDS.  Variants:
    non-softmax, non-causal, register prefix, fp16 (online max), D = 40, and
    queries far from every key (the forward's per-block rerun with an online
    max).  Compared on a 2 x 2 corner of (b, h) slices."""
    q, k, v, do = rand_inputs(16, 16, N, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=N + D)
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.gamma = 16, 16, N, D, int(causal), 0.1
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(q))
    assert _lib.bwd_kernels(a) == (1 if N <= 576 else 2)
    if shift:
        q = q.clone()
        q[:2, ::2, :90] += shift
    compare_case(q, k, v, do, softmax=softmax, causal=causal, num_prefix=num_prefix, gamma=1.0 / (2 * math.sqrt(D)),
                 sl=(slice(0, 2), slice(0, 2)), tag=f"hr N{N} D{D} {dtype} sm{softmax} c{causal} p{num_prefix} far{shift}",
                 ill_conditioned=shift > 0)


@pytest.mark.parametrize("causal", [True, False])
def test_flex_attention_cross_check(cuda_device, causal):
    """Cross-check against torch's own flex_attention on the GPU (the
    reference's comparator path, rbf_attention.py:1590-1605, run in fp32 on
    the same bf16 inputs, unfused): O and the autograd gradients agree with
    the HIP kernels to the bf16 tolerance, and flex itself agrees with the
    float64 oracle."""
    import warnings

    from rbf_attention_amd.flex import rbf_flex_attention

    w = wl.C2_MODEL.with_(B=2, H=4)
    q, k, v, do = to_dev(wl.make_inputs(w), cuda_device)
    g = w.sm_scale
    ours = run_ours(q, k, v, do, True, causal, g, 0)
    qf, kf, vf = (t.detach().float().clone().requires_grad_(True) for t in (q, k, v))
    with warnings.catch_warnings():
        warnings.simplefilter("ignore")
        of = rbf_flex_attention(qf, kf, vf, is_causal=causal, sm_scale=g)
    of.backward(do.float())
    torch.cuda.synchronize()
    flex = (of, qf.grad, kf.grad, vf.grad)
    refs, _, _ = oracle_all(q, k, v, do, True, causal, g, 0)
    for name, a, f, r in zip(("O", "dQ", "dK", "dV"), ours, flex, refs):
        check(f"flex c{causal} {name} (ours vs flex)", a, np64(f), q.dtype)
        fe = float(np.abs(np64(f) - r).max())
        assert fe <= 1e-3 * max(1.0, float(np.abs(r).max())), f"flex vs oracle {name}: {fe}"


@pytest.mark.parametrize("softmax", [True, False])
def test_token_major_output(cuda_device, softmax):
    """token_major=True: same values and gradients bit for bit, and the model's
    (B, H, N, D) -> (B, N, H*D) transpose + reshape is a view."""
    q, k, v, do = rand_inputs(2, 4, 100, 64, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=5)
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    res = []
    for tm in (False, True):
        qq, kk, vv = (t.detach().clone().requires_grad_(True) for t in (q, k, v))
        out = fn(qq, kk, vv, True, sm_scale=0.0625, token_major=tm)
        flat = out.transpose(1, 2).reshape(2, 100, 4 * 64)
        if tm:
            assert flat.data_ptr() == out.data_ptr() and flat.is_contiguous()
        flat.backward(do.transpose(1, 2).reshape(2, 100, 256))
        torch.cuda.synchronize()
        res.append((out.detach(), qq.grad, kk.grad, vv.grad))
    for a, b in zip(*res):
        assert torch.equal(a, b)


def test_strided_views_like_the_model(cuda_device):
    """q/k/v as views of one packed projection, dout as a permuted view
    (rbf_attention.py:1659-1662, 1761)."""
    B, N, H, D = 2, 130, 4, 64
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B, N, 3 * H * D, generator=g).to(torch.bfloat16).to(cuda_device)
    q, k, v = qkv.view(B, N, 3, H, D).permute(2, 0, 3, 1, 4)
    do = torch.randn(B, N, H, D, generator=g).to(torch.bfloat16).to(cuda_device).permute(0, 2, 1, 3)
    assert not q.is_contiguous() and not do.is_contiguous()
    compare_case(q, k, v, do, tag="strided")


@pytest.mark.parametrize(
    "D,N,dtype,softmax",
    [(128, 300, torch.bfloat16, True), (128, 2113, torch.bfloat16, True), (128, 2113, torch.float16, False),
     (64, 700, torch.bfloat16, True), (64, 4200, torch.bfloat16, True), (64, 4200, torch.float16, False)],
)
def test_strided_views_dma_tiles(cuda_device, D, N, dtype, softmax):
    """q/k/v as views of one packed projection and a permuted dout, for the
    streaming kernels whose tiles are staged by LDS-DMA (16-bit, D = 64 or
    128) through buffer resources whose row pitch is the view's token stride
    (3 H D, or H D for dout); rows past N (N not a multiple of the 64-row
    tile) read zeros.  D = 128: N = 300 takes the binned short-sequence
    kernels, N = 2113 the long-sequence ones (paired dK/dV kernel); D = 64
    (B * H below the CU count, so no head-resident kernels): N = 700 DMA
    forward and dQ, N = 4200 also the DMA dK/dV.  Checked on the first and
    the last (b, h) slice."""
    B, H = 2, 3
    g = torch.Generator().manual_seed(N)
    qkv = (torch.randn(B, N, 3 * H * D, generator=g) * (1.0 if softmax else 0.5)).to(dtype).to(cuda_device)
    q, k, v = qkv.view(B, N, 3, H, D).permute(2, 0, 3, 1, 4)
    do = torch.randn(B, N, H, D, generator=g).to(dtype).to(cuda_device).permute(0, 2, 1, 3)
    assert not q.is_contiguous() and q.stride(2) == 3 * H * D and do.stride(2) == H * D
    gamma = 1.0 / (2 * math.sqrt(D))
    outs = run_ours(q, k, v, do, softmax, True, gamma, 0)
    for sl in ((slice(0, 1), slice(0, 1)), (slice(B - 1, B), slice(H - 1, H))):
        compare_case(q, k, v, do, softmax=softmax, gamma=gamma, sl=sl, outs=outs,
                     tag=f"strided D{D} N{N} b{sl[0].start}h{sl[1].start}")


@pytest.mark.parametrize(
    "D,N,which,softmax",
    [(64, 700, "kv", True), (128, 2113, "kv", True), (128, 2113, "qdo", True), (64, 4200, "qdo", False),
     (128, 2113, "kv", False)],
)
def test_zero_token_stride_operands(cuda_device, D, N, which, softmax):
    """Operands expanded along the token axis (x.expand(B, H, N, D): token
    stride 0), passed to the ops as they are.  Such rows cannot be staged by
    LDS-DMA, whose buffer range is N * stride bytes (empty at stride 0), so
    the launchers take the register-staged kernels for them; the shapes are
    ones whose contiguous operands take LDS-DMA tiles (D = 64 at N = 700:
    forward and dQ; D = 128 at N = 2113: forward, dQ and dK/dV; D = 64 at
    N = 4200: dK/dV).  "kv": K and V expanded (the tiles of the forward and
    dQ), "qdo": Q and dO expanded (the tiles of dK/dV)."""
    B, H = 1, 2
    q, k, v, do = rand_inputs(B, H, N, D, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=N + D)
    if which == "kv":
        k = k[:, :, 5:6].expand(B, H, N, D)
        v = v[:, :, 7:8].expand(B, H, N, D)
        assert k.stride(2) == 0 and v.stride(2) == 0
    else:
        q = q[:, :, 3:4].expand(B, H, N, D)
        do = do[:, :, 9:10].expand(B, H, N, D)
        assert q.stride(2) == 0 and do.stride(2) == 0
    gamma = 1.0 / (2 * math.sqrt(D))
    if softmax:
        out, L = torch.ops.rbf_attn_amd.scaled_fwd_ex(q, k, v, True, gamma, 0)
        grads = torch.ops.rbf_attn_amd.scaled_bwd_ex(q, k, v, out, L, do, True, gamma, 0)
    else:
        out = torch.ops.rbf_attn_amd.non_softmax_fwd_ex(q, k, v, True, gamma, 0)
        grads = torch.ops.rbf_attn_amd.non_softmax_bwd_ex(q, k, v, do, True, gamma, 0)
    torch.cuda.synchronize()
    compare_case(q, k, v, do, softmax=softmax, gamma=gamma, outs=(out,) + tuple(grads),
                 tag=f"stride0 {which} D{D} N{N} sm{softmax}")


@pytest.mark.parametrize("softmax", [True, False])
def test_one_launch_backward_equals_two_stages(cuda_device, softmax):
    """At B*H = 256 heads of N <= 576 the backward is one launch (both passes
    of a head in one work-group, the per-query term passed through LDS); it
    must give the two-launch form's dQ, dK, dV and workspace bit for bit."""
    B, H, N, D, dtype = 16, 16, 516, 64, torch.bfloat16
    q, k, v, do = rand_inputs(B, H, N, D, dtype, cuda_device, std=1.0 if softmax else 0.5, seed=33)
    bufs = {"q": q, "k": k, "v": v, "dout": do}
    for f in ("o", "dq", "dk", "dv"):
        bufs[f] = torch.zeros_like(q)
    bufs["lse"] = torch.zeros((B, H, N), device=cuda_device, dtype=torch.float32)
    bufs["delta"] = torch.zeros_like(bufs["lse"])
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.num_prefix, a.gamma = B, H, N, D, 1, 4, 1.0 / (2 * math.sqrt(D))
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(bufs[f]))
    a.lse, a.delta = bufs["lse"].data_ptr(), bufs["delta"].data_ptr()
    assert _lib.bwd_kernels(a) == 1
    sp = torch.cuda.current_stream(cuda_device).cuda_stream
    _lib.call("rbf_attn_fwd", a, sp)
    keep = ("dq", "dk", "dv", "lse", "delta")
    _lib.call("rbf_attn_bwd", a, sp)
    one = {f: bufs[f].clone() for f in keep}
    for f in ("dq", "dk", "dv", "delta"):
        bufs[f].zero_()
    if not softmax:
        bufs["lse"].zero_()  # the non-softmax backward's norm-offset workspace
    _lib.call("rbf_attn_bwd_stage", a, sp, 1)
    _lib.call("rbf_attn_bwd_stage", a, sp, 2)
    torch.cuda.synchronize()
    for f in keep:
        assert torch.equal(one[f], bufs[f]), f"{f}: max diff {(one[f].float() - bufs[f].float()).abs().max().item():.3e}"
    assert one["dq"].abs().sum() > 0 and one["dk"].abs().sum() > 0


@pytest.mark.parametrize(
    "B,H,N,D,softmax",
    [
        (2, 4, 300, 64, True),  # streaming kernels, register staging
        (32, 8, 516, 64, True),  # head-resident forward, one-launch backward
        (1, 2, 2113, 128, True),  # LDS-DMA forward, dQ and paired dK/dV
        (1, 2, 4200, 64, False),  # LDS-DMA D = 64 kernels, non-softmax
    ],
)
def test_deterministic(cuda_device, B, H, N, D, softmax):
    """Two runs on the same inputs give the same bits: no atomics, no
    order-dependent reductions, whatever the staging."""
    q, k, v, do = rand_inputs(B, H, N, D, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=21)
    a = run_ours(q, k, v, do, softmax, True, None, 0)
    b = run_ours(q, k, v, do, softmax, True, None, 0)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_autograd_function_aliases(cuda_device):
    q, k, v, do = rand_inputs(1, 2, 96, 64, torch.bfloat16, cuda_device, seed=4)
    ref = run_ours(q, k, v, do, True, True, None, 0)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = ra.TritonRBFAttention.apply(qq, kk, vv, True)
    out.backward(do)
    for x, y in zip((out, qq.grad, kk.grad, vv.grad), ref):
        assert torch.equal(x, y)
    ref2 = run_ours(q, k, v, do * 0.5, False, True, None, 0)
    qq, kk, vv = (t.clone().requires_grad_(True) for t in (q, k, v))
    out = ra.TritonNonSoftmaxRBFAttention.apply(qq, kk, vv, True)
    out.backward(do * 0.5)
    for x, y in zip((out, qq.grad, kk.grad, vv.grad), ref2):
        assert torch.equal(x, y)


@pytest.mark.parametrize("softmax", [True, False])
@pytest.mark.parametrize("opts", ["reference", "extended"])
def test_eager_wrappers_equal_registered_ops(cuda_device, softmax, opts):
    """Eager run_triton_rbf / run_triton_non_softmax_rbf take an
    autograd.Function over the ops' implementations instead of the
    torch.library dispatch; output (values and strides) and every gradient,
    the position term's included, must equal the registered ops' bit for bit."""
    q, k, v, do = rand_inputs(2, 4, 130, 64, torch.bfloat16, cuda_device, std=1.0 if softmax else 0.5, seed=7)
    P = (torch.randn(1, 4, 130, 64, generator=torch.Generator().manual_seed(8)) * 0.3).to(torch.bfloat16).to(cuda_device)
    ext = opts == "extended"
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    if ext:
        kw = dict(sm_scale=0.0625, num_prefix=4, token_major=True)
        op = torch.ops.rbf_attn_amd.scaled_fwd_ex if softmax else torch.ops.rbf_attn_amd.non_softmax_fwd_ex
        call_op = lambda a, b, c, p: op(a, b, c, True, 0.0625, 4, True, p)
    else:
        kw = {}
        op = torch.ops.rbf_attn_v5.scaled_fwd if softmax else torch.ops.rbf_attn_v5.non_softmax_fwd
        call_op = lambda a, b, c, p: op(a, b, c, True)
    results = []
    for path in ("eager", "op"):
        leaves = [t.clone().requires_grad_(True) for t in (q, k, v)] + ([P.clone().requires_grad_(True)] if ext else [])
        pos = leaves[3] if ext else None
        if path == "eager":
            out = fn(leaves[0], leaves[1], leaves[2], True, pos=pos, **kw)
            assert type(out.grad_fn).__name__ == "_EagerRbfAttentionBackward"
        else:
            out = call_op(leaves[0], leaves[1], leaves[2], pos)
            out = out[0] if softmax else out
            assert type(out.grad_fn).__name__ != "_EagerRbfAttentionBackward"
        out.backward(do)
        torch.cuda.synchronize()
        results.append([out.detach()] + [t.grad for t in leaves])
    for i, (x, y) in enumerate(zip(*results)):
        assert x.shape == y.shape and x.stride() == y.stride(), (i, x.stride(), y.stride())
        assert torch.equal(x, y), f"tensor {i}: max diff {(x.float() - y.float()).abs().max().item():.3e}"
    # without autograd recording: no_grad and inference mode give the same output
    for ctx in (torch.no_grad, torch.inference_mode):
        with ctx():
            out = fn(q, k, v, True, pos=P if ext else None, **kw)
        assert out.grad_fn is None and torch.equal(out, results[0][0])


def test_size_one_dims_take_any_stride(cuda_device):
    """torch gives a dimension of size 1 an arbitrary stride (the tensor still
    counts as contiguous); such a stride is never used and must not trip the
    C ABI's 16-byte stride check."""
    q, k, v, do = rand_inputs(1, 2, 70, 64, torch.bfloat16, cuda_device, seed=9)
    odd = [t.as_strided(t.shape, (3,) + t.stride()[1:]) for t in (q, k, v)]
    assert all(t.is_contiguous() for t in odd)
    for fn in (ra.run_triton_rbf, ra.run_triton_non_softmax_rbf):
        assert torch.equal(fn(*odd, True), fn(q, k, v, True))


def test_empty_batch(cuda_device):
    q = torch.zeros(0, 2, 16, 64, device=cuda_device, dtype=torch.bfloat16)
    out = ra.run_triton_rbf(q, q, q)
    assert out.shape == q.shape


# ---------------------------------------------------------------------------
# Committed fixtures (tests/golden/c1_slices.npz): fp32, compared directly.
# ---------------------------------------------------------------------------
def test_golden_fixture_fp32(cuda_device):
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c1_slices.npz")
    gold = np.load(path)
    g = float(gold["gamma"])
    q, k, v, do = (torch.from_numpy(gold[n]).to(cuda_device) for n in ("q", "k", "v", "do"))
    outs = run_ours(q, k, v, do, True, True, g, 0)
    for name, got in zip(("O", "dq", "dk", "dv"), outs):
        check(f"golden softmax {name}", got, gold[f"softmax_{name}"].astype(np.float64), torch.float32)
    _, L = torch.ops.rbf_attn_amd.scaled_fwd_ex(q, k, v, True, g, 0)
    check("golden softmax L", L, gold["softmax_L"].astype(np.float64), torch.float32)
    outs = run_ours(0.5 * q, 0.5 * k, 0.5 * v, 0.5 * do, False, True, g, 0)
    for name, got in zip(("O", "dq", "dk", "dv"), outs):
        check(f"golden non-softmax {name}", got, gold[f"nonsoftmax_{name}"].astype(np.float64), torch.float32)
