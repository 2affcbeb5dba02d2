"""Property tests of the C ABI's argument validation (CPU only: no call here
reaches a launch).

Each drawn call starts from a valid problem of random shape, dtype, variant
and mask, then plants one or more documented defects (include/rbf_attn.h
names the error code of each).  Whatever the combination, the entry point
must return the code of one of the planted defects and leave a message,
before any HIP call.  Valid problems with no work return 0 and no message.
The draws are derandomized (the same calls every run), so the CPU suite stays
reproducible."""
import ctypes

import pytest
from hypothesis import given, settings, strategies as st

import torch  # noqa: F401  (binds the library to torch's HIP runtime)

from rbf_attention_amd import _lib

from test_capi import FAKE, lib  # noqa: F401  (module fixture)

ARGS, DTYPE, STRIDE, HEADDIM, SHAPE, PTR = -1, -2, -3, -4, -5, -6
FWD_TENSORS = ("q", "k", "v", "o")
BWD_TENSORS = FWD_TENSORS + ("dout", "dq", "dk", "dv")


def base_args(B, H, N, D, dtype, variant, causal, num_prefix, gamma):
    esz = 4 if dtype == 2 else 2
    a = _lib.Args()
    a.abi_version = _lib.ABI_VERSION
    a.variant, a.dtype = variant, dtype
    a.B, a.H, a.N, a.D = B, H, N, D
    a.causal, a.num_prefix, a.gamma = causal, num_prefix, gamma
    for i, f in enumerate(BWD_TENSORS):
        # (B, H, N, D) contiguous strides, each a multiple of 16 bytes
        setattr(a, f, _lib.Tensor(FAKE + 0x1000000 * i, H * N * D, N * D, D))
    a.lse = FAKE + 0x10000000
    a.delta = FAKE + 0x11000000
    assert (D * esz) % 16 == 0
    return a


valid = st.fixed_dictionaries(dict(
    B=st.integers(1, 64), H=st.integers(1, 64), N=st.integers(1, 20000),
    D=st.sampled_from(range(8, 257, 8)), dtype=st.sampled_from((0, 1, 2)), variant=st.sampled_from((0, 1)),
    causal=st.sampled_from((0, 1)), num_prefix=st.integers(0, 600),
    gamma=st.floats(1e-4, 10.0, allow_nan=False, allow_infinity=False)))

# Defects: each plant(args, draw) changes args and returns the code it must produce.
def _bad_abi(a, d):
    a.abi_version = d(st.sampled_from((0, 1, _lib.ABI_VERSION + 1, -7)))
    return ARGS


def _bad_variant(a, d):
    a.variant = d(st.sampled_from((2, 3, -1, 99)))
    return ARGS


def _bad_dtype(a, d):
    a.dtype = d(st.sampled_from((3, 4, -1, 255)))
    return DTYPE


def _bad_headdim(a, d):
    a.D = d(st.sampled_from((0, 4, 12, 60, 100, 132, 264, 512, -8)))
    return HEADDIM


def _bad_size(a, d):
    setattr(a, d(st.sampled_from(("B", "H", "N"))), d(st.integers(-(1 << 30), -1)))
    return SHAPE


def _bad_causal(a, d):
    a.causal = d(st.sampled_from((2, -1, 7)))
    return ARGS


def _bad_prefix(a, d):
    a.num_prefix = d(st.integers(-(1 << 20), -1))
    return ARGS


def _bad_gamma(a, d):
    a.gamma = d(st.sampled_from((0.0, -0.5, float("nan"), float("inf"), -float("inf"))))
    return ARGS


def _huge_n(a, d):
    a.N = d(st.integers((1 << 30) + 1, (1 << 31) - 1))
    return SHAPE


def _null_tensor(tensors):
    def plant(a, d):
        name = d(st.sampled_from(tensors))
        t = getattr(a, name)
        setattr(a, name, _lib.Tensor(None, t.stride_b, t.stride_h, t.stride_n))
        return PTR
    return plant


def _misaligned_base(tensors):
    def plant(a, d):
        name = d(st.sampled_from(tensors))
        t = getattr(a, name)
        if t.ptr is None:  # already planted as a null tensor, which stays reported
            return PTR
        setattr(a, name, _lib.Tensor(t.ptr + d(st.sampled_from((2, 4, 8, 12))), t.stride_b, t.stride_h, t.stride_n))
        return STRIDE
    return plant


def _bad_stride(tensors):
    def plant(a, d):
        name = d(st.sampled_from(tensors))
        t = getattr(a, name)
        esz = 4 if a.dtype == 2 else 2
        bad = (16 * d(st.integers(0, 1000)) + 8) // esz  # 8 bytes past a multiple of 16
        which = d(st.sampled_from(("stride_b", "stride_h", "stride_n")))
        s = dict(stride_b=t.stride_b, stride_h=t.stride_h, stride_n=t.stride_n)
        s[which] = bad
        setattr(a, name, _lib.Tensor(t.ptr, s["stride_b"], s["stride_h"], s["stride_n"]))
        return STRIDE
    return plant


def _null_lse(a, d):
    a.lse = None
    return PTR


def _null_delta(a, d):
    a.delta = None
    return PTR


def defects(fn, variant):
    """The defects that apply to one entry point and variant, following the
    header's per-field rules: the backward reads o only for the softmax
    variant (for Delta); lse is the forward's L (softmax) or, for the
    non-softmax backward, a workspace -- which the no-allocation backward
    replaces, as it replaces delta (a softmax-only workspace)."""
    softmax = variant == 0
    if fn == "rbf_attn_fwd":
        tensors = FWD_TENSORS
    else:
        tensors = tuple(t for t in BWD_TENSORS if t != "o" or softmax)
    out = [_bad_abi, _bad_variant, _bad_dtype, _bad_headdim, _bad_size, _bad_causal, _bad_prefix, _bad_gamma,
           _huge_n, _null_tensor(tensors), _misaligned_base(tensors), _bad_stride(tensors)]
    if softmax or fn == "rbf_attn_bwd":
        out.append(_null_lse)
    if softmax and fn == "rbf_attn_bwd":
        out.append(_null_delta)
    return out


@settings(max_examples=1500, deadline=None, derandomize=True)
@given(fn=st.sampled_from(("rbf_attn_fwd", "rbf_attn_bwd", "rbf_attn_bwd_noalloc")), v=valid, data=st.data())
def test_planted_defects_are_reported(lib, fn, v, data):
    # small enough for the no-allocation entry point's workspace, so that only
    # the planted defects can fail
    v["N"] = min(v["N"], _lib.NOALLOC_MAX_ROWS // (v["B"] * v["H"]))
    a = base_args(**v)
    pool = defects(fn, v["variant"])
    picks = data.draw(st.lists(st.sampled_from(range(len(pool))), min_size=1, max_size=4, unique=True))
    codes = {pool[i](a, data.draw) for i in picks}
    rc = getattr(lib, fn)(ctypes.byref(a), None)
    msg = lib.rbf_attn_last_error().decode()
    assert rc in codes, (rc, codes, msg)
    assert msg, rc


@settings(max_examples=200, deadline=None, derandomize=True)
@given(fn=st.sampled_from(("rbf_attn_fwd", "rbf_attn_bwd", "rbf_attn_bwd_noalloc")), v=valid,
       zero=st.sampled_from(("B", "H", "N")))
def test_empty_problems_do_nothing(lib, fn, v, zero):
    v[zero] = 0
    a = base_args(**v)
    assert getattr(lib, fn)(ctypes.byref(a), None) == 0
    assert lib.rbf_attn_last_error().decode() == ""


@pytest.mark.parametrize("fn", ["rbf_attn_fwd", "rbf_attn_bwd"])
def test_error_cleared_by_next_valid_call(lib, fn):
    """A message describes the last call only."""
    a = base_args(2, 2, 64, 64, 0, 0, 1, 0, 0.1)
    a.D = 60
    assert getattr(lib, fn)(ctypes.byref(a), None) == HEADDIM
    assert lib.rbf_attn_last_error().decode()
    a.D, a.N = 64, 0
    assert getattr(lib, fn)(ctypes.byref(a), None) == 0
    assert lib.rbf_attn_last_error().decode() == ""
