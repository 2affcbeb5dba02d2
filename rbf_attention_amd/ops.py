"""torch.library operators for RBF attention on MI355X.

Drop-in surface of the reference (rbf_attention.py):
  * ``rbf_attn_v5::scaled_fwd(q, k, v, is_causal) -> (out, L)``        (651-690)
  * ``rbf_attn_v5::scaled_bwd(q, k, v, out, L, dout, is_causal, sm_scale)
        -> (dq, dk, dv)``                                               (702-810)
  * ``rbf_attn_v5::non_softmax_fwd(q, k, v, is_causal) -> out``        (1355-1391)
  * ``rbf_attn_v5::non_softmax_bwd(q, k, v, dout, is_causal, sm_scale)
        -> (dq, dk, dv)``                                               (1399-1480)
  each with a fake (meta) implementation and autograd registration
  (822-842, 1492-1511), plus ``run_triton_rbf`` / ``run_triton_non_softmax_rbf``
  (848-853).

Same names, schemas and semantics: gamma (the reference's ``sm_scale``) is
1/sqrt(D) in the forward ops, L is the base-2 log-sum-exp of
2*gamma*q.k - gamma*||k||^2, outputs are freshly allocated contiguous tensors,
and the autograd backward ignores the gradient of L.

Extensions, in a separate namespace so the reference schemas stay exact:
``rbf_attn_amd::{scaled,non_softmax}_{fwd,bwd}_ex`` take an explicit
``sm_scale`` (gamma) and ``num_prefix`` (keys j < num_prefix are visible to every
query: register tokens).  ``run_triton_rbf(..., sm_scale=, num_prefix=)``
routes to them when either differs from the reference default.

Every op runs the HIP kernels of librbfattn.so; there is no CPU or PyTorch
fallback.  Unsupported inputs raise.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.utils._python_dispatch as _python_dispatch

from . import _lib

_V5 = "rbf_attn_v5"
_EX = "rbf_attn_amd"


# ---------------------------------------------------------------------------
# Input handling
# ---------------------------------------------------------------------------
def _check_inputs(name: str, *ts: torch.Tensor) -> None:
    q = ts[0]
    if q.dim() != 4:
        raise ValueError(f"{name}: expected (B, H, N, D) tensors, got q of shape {tuple(q.shape)}")
    for t in ts:
        if t.shape != q.shape:
            raise ValueError(f"{name}: shape mismatch {tuple(t.shape)} vs {tuple(q.shape)}")
        if t.dtype != q.dtype:
            raise TypeError(f"{name}: dtype mismatch {t.dtype} vs {q.dtype}")
        if t.device != q.device:
            raise ValueError(f"{name}: device mismatch {t.device} vs {q.device}")
    if q.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"{name}: unsupported dtype {q.dtype} (bf16, fp16, fp32)")
    if q.shape[-1] > 256:
        raise ValueError(f"{name}: head dim {q.shape[-1]} > 256 is not supported")
    if q.device.type != "cuda":
        raise RuntimeError(
            f"{name}: tensors are on {q.device}; the RBF attention kernels run only on a ROCm GPU "
            "(there is no CPU fallback)"
        )


def _padded_dim(d: int) -> int:
    return max(8, (d + 7) // 8 * 8)


def _prep(t: torch.Tensor, dpad: int) -> torch.Tensor:
    """Meet the C-ABI layout contract: unit last stride, 16-byte aligned base
    and strides, head dim a multiple of 8.  Copies only when needed."""
    d = t.shape[-1]
    if dpad != d:
        return torch.nn.functional.pad(t, (0, dpad - d))
    if t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t  # strides are multiples of d, a multiple of 8 elements
    esz = t.element_size()
    ok = (
        t.stride(-1) == 1
        and t.data_ptr() % 16 == 0
        and all((s * esz) % 16 == 0 for s in t.stride()[:3])
    )
    return t if ok else t.contiguous()


def _base_args(variant: int, q: torch.Tensor, is_causal: bool, sm_scale: float, num_prefix: int, dpad: int):
    B, H, N, _ = q.shape
    a = _lib.Args()
    a.abi_version = _lib.ABI_VERSION
    a.variant = variant
    a.dtype = _lib.DTYPE_CODES[q.dtype]
    a.B, a.H, a.N, a.D = B, H, N, dpad
    a.causal = 1 if is_causal else 0
    a.num_prefix = int(num_prefix)
    a.gamma = float(sm_scale)
    return a


def _stream(device: torch.device) -> int:
    """The current stream of the tensors' device (raw handle)."""
    return torch._C._cuda_getCurrentRawStream(device.index)


def _call_on(device: torch.device, fn: str, a) -> None:
    """One C-ABI call on the current stream of `device`, with that device
    current during the call."""
    if torch.cuda.current_device() == device.index:
        _lib.call(fn, a, _stream(device))
    else:
        with torch.cuda.device(device):
            _lib.call(fn, a, _stream(device))


def _launch(fn: str, a, device: torch.device) -> None:
    if a.B * a.H * a.N == 0:
        return  # empty problem: nothing to compute (data pointers may be NULL)
    _call_on(device, fn, a)


def _launch_pos(fn: str, a, pos: torch.Tensor, device: torch.device) -> None:
    if a.B * a.H * a.N == 0:
        return
    with torch.cuda.device(device):
        _lib.call_pos(fn, a, _lib.pos_desc(pos), _stream(device))


def _check_pos(name: str, q: torch.Tensor, pos: torch.Tensor) -> None:
    B, H, N, D = q.shape
    if pos.dim() != 4 or tuple(pos.shape[1:]) != (H, N, D) or pos.shape[0] not in (1, B):
        raise ValueError(f"{name}: pos must be (1 or B, H, N, D) = (1|{B}, {H}, {N}, {D}), got {tuple(pos.shape)}")
    if pos.dtype != q.dtype or pos.device != q.device:
        raise TypeError(f"{name}: pos must match q's dtype and device")


def _with_pos(name: str, a, q, k, pos, dp: int):
    """Position term for a launch: the (1 or B, H, N, dp) operand for the
    fused entry points when the library fuses it for these args (the
    head-resident kernels), else None after adding it to q and k here -- the
    same values (each sum rounded to the element type), as separate
    elementwise adds."""
    if pos is None:
        return q, k, None
    _check_pos(name, q, pos)
    if _lib.pos_supported(a):
        return q, k, _prep(pos, dp)
    return q + pos, k + pos, None


def _unpad(t: torch.Tensor, d: int) -> torch.Tensor:
    return t if t.shape[-1] == d else t[..., :d].contiguous()


# ---------------------------------------------------------------------------
# Implementations (shared by the reference-schema ops and the _ex ops)
# ---------------------------------------------------------------------------
def _alloc_out(q: torch.Tensor, dp: int, token_major: bool) -> torch.Tensor:
    """(B, H, N, dp) output.  token_major: backed by a (B, N, H, dp) buffer, so
    that ``out.transpose(1, 2).reshape(B, N, H * dp)`` -- the layout the model's
    output projection reads (rbf_attention.py:1761) -- is a view, not a copy."""
    B, H, N, _ = q.shape
    if token_major:
        return torch.empty((B, N, H, dp), device=q.device, dtype=q.dtype).transpose(1, 2)
    return torch.empty((B, H, N, dp), device=q.device, dtype=q.dtype)


def _softmax_fwd(q, k, v, is_causal: bool, sm_scale: float, num_prefix: int, token_major: bool = False, pos=None):
    _check_inputs("scaled_fwd", q, k, v)
    B, H, N, D = q.shape
    dp = _padded_dim(D)
    a = _base_args(_lib.SOFTMAX, q, is_causal, sm_scale, num_prefix, dp)
    q, k, pos_ = _with_pos("scaled_fwd", a, q, k, pos, dp)
    q_, k_, v_ = _prep(q, dp), _prep(k, dp), _prep(v, dp)
    out = _alloc_out(q, dp, token_major and dp == D)
    L = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    a.q, a.k, a.v, a.o = (_lib.tensor_desc(t) for t in (q_, k_, v_, out))
    a.lse = L.data_ptr()
    if pos_ is None:
        _launch("rbf_attn_fwd", a, q.device)
    else:
        _launch_pos("rbf_attn_fwd_pos", a, pos_, q.device)
    return _unpad(out, D), L


def _softmax_bwd(q, k, v, out, L, dout, is_causal: bool, sm_scale: float, num_prefix: int, pos=None):
    _check_inputs("scaled_bwd", q, k, v, out, dout)
    B, H, N, D = q.shape
    if L.shape != (B, H, N) or L.dtype != torch.float32:
        raise ValueError(f"scaled_bwd: L must be float32 of shape {(B, H, N)}, got {L.dtype} {tuple(L.shape)}")
    dp = _padded_dim(D)
    a = _base_args(_lib.SOFTMAX, q, is_causal, sm_scale, num_prefix, dp)
    q, k, pos_ = _with_pos("scaled_bwd", a, q, k, pos, dp)
    q_, k_, v_, o_, do_ = (_prep(t, dp) for t in (q, k, v, out, dout))
    L_ = L.contiguous()
    delta = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    dq = torch.empty((B, H, N, dp), device=q.device, dtype=q.dtype)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    a.q, a.k, a.v, a.o, a.dout = (_lib.tensor_desc(t) for t in (q_, k_, v_, o_, do_))
    a.dq, a.dk, a.dv = (_lib.tensor_desc(t) for t in (dq, dk, dv))
    a.lse = L_.data_ptr()
    a.delta = delta.data_ptr()
    if pos_ is None:
        _launch("rbf_attn_bwd", a, q.device)
    else:
        _launch_pos("rbf_attn_bwd_pos", a, pos_, q.device)
    return _unpad(dq, D), _unpad(dk, D), _unpad(dv, D)


def _non_softmax_fwd(q, k, v, is_causal: bool, sm_scale: float, num_prefix: int, token_major: bool = False,
                     pos=None):
    _check_inputs("non_softmax_fwd", q, k, v)
    B, H, N, D = q.shape
    dp = _padded_dim(D)
    a = _base_args(_lib.NON_SOFTMAX, q, is_causal, sm_scale, num_prefix, dp)
    q, k, pos_ = _with_pos("non_softmax_fwd", a, q, k, pos, dp)
    q_, k_, v_ = _prep(q, dp), _prep(k, dp), _prep(v, dp)
    out = _alloc_out(q, dp, token_major and dp == D)
    a.q, a.k, a.v, a.o = (_lib.tensor_desc(t) for t in (q_, k_, v_, out))
    if pos_ is None:
        _launch("rbf_attn_fwd", a, q.device)
    else:
        _launch_pos("rbf_attn_fwd_pos", a, pos_, q.device)
    return _unpad(out, D)


def _non_softmax_bwd(q, k, v, dout, is_causal: bool, sm_scale: float, num_prefix: int, pos=None):
    _check_inputs("non_softmax_bwd", q, k, v, dout)
    B, H, N, D = q.shape
    dp = _padded_dim(D)
    a = _base_args(_lib.NON_SOFTMAX, q, is_causal, sm_scale, num_prefix, dp)
    q, k, pos_ = _with_pos("non_softmax_bwd", a, q, k, pos, dp)
    q_, k_, v_, do_ = (_prep(t, dp) for t in (q, k, v, dout))
    qoff = torch.empty((B, H, N), device=q.device, dtype=torch.float32)
    dq = torch.empty((B, H, N, dp), device=q.device, dtype=q.dtype)
    dk = torch.empty_like(dq)
    dv = torch.empty_like(dq)
    a.q, a.k, a.v, a.dout = (_lib.tensor_desc(t) for t in (q_, k_, v_, do_))
    a.dq, a.dk, a.dv = (_lib.tensor_desc(t) for t in (dq, dk, dv))
    a.lse = qoff.data_ptr()
    if pos_ is None:
        _launch("rbf_attn_bwd", a, q.device)
    else:
        _launch_pos("rbf_attn_bwd_pos", a, pos_, q.device)
    return _unpad(dq, D), _unpad(dk, D), _unpad(dv, D)


def _default_scale(q: torch.Tensor) -> float:
    # rbf_attention.py:660, 827, 1362, 1496
    return 1.0 / math.sqrt(q.shape[-1])


# ---------------------------------------------------------------------------
# Reference-schema ops: rbf_attn_v5::*
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_V5}::scaled_fwd", mutates_args=())
def rbf_scaled_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool) -> tuple[torch.Tensor, torch.Tensor]:
    return _softmax_fwd(q, k, v, is_causal, _default_scale(q), 0)


@rbf_scaled_fwd.register_fake
def _(q, k, v, is_causal):
    B, H, N, _ = q.shape
    return (
        torch.empty_like(q, memory_format=torch.contiguous_format),
        torch.empty((B, H, N), device=q.device, dtype=torch.float32),
    )


@torch.library.custom_op(f"{_V5}::scaled_bwd", mutates_args=())
def rbf_scaled_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    L: torch.Tensor,
    dout: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _softmax_bwd(q, k, v, out, L, dout, is_causal, sm_scale, 0)


@rbf_scaled_bwd.register_fake
def _(q, k, v, out, L, dout, is_causal, sm_scale):
    return (
        torch.empty_like(q, memory_format=torch.contiguous_format),
        torch.empty_like(k, memory_format=torch.contiguous_format),
        torch.empty_like(v, memory_format=torch.contiguous_format),
    )


def _scaled_setup_context(ctx, inputs, output):
    q, k, v, is_causal = inputs
    out, L = output
    ctx.save_for_backward(q, k, v, out, L)
    ctx.is_causal = is_causal
    ctx.sm_scale = _default_scale(q)


def _scaled_backward(ctx, dout, dL):
    # dL is ignored, as in the reference (rbf_attention.py:830-835).
    q, k, v, out, L = ctx.saved_tensors
    dq, dk, dv = torch.ops.rbf_attn_v5.scaled_bwd(q, k, v, out, L, dout, ctx.is_causal, ctx.sm_scale)
    return dq, dk, dv, None


torch.library.register_autograd(f"{_V5}::scaled_fwd", _scaled_backward, setup_context=_scaled_setup_context)


@torch.library.custom_op(f"{_V5}::non_softmax_fwd", mutates_args=())
def rbf_non_softmax_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, is_causal: bool) -> torch.Tensor:
    return _non_softmax_fwd(q, k, v, is_causal, _default_scale(q), 0)


@rbf_non_softmax_fwd.register_fake
def _(q, k, v, is_causal):
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@torch.library.custom_op(f"{_V5}::non_softmax_bwd", mutates_args=())
def rbf_non_softmax_bwd(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _non_softmax_bwd(q, k, v, dout, is_causal, sm_scale, 0)


@rbf_non_softmax_bwd.register_fake
def _(q, k, v, dout, is_causal, sm_scale):
    return (
        torch.empty_like(q, memory_format=torch.contiguous_format),
        torch.empty_like(k, memory_format=torch.contiguous_format),
        torch.empty_like(v, memory_format=torch.contiguous_format),
    )


def _non_softmax_setup_context(ctx, inputs, output):
    q, k, v, is_causal = inputs
    ctx.save_for_backward(q, k, v)
    ctx.is_causal = is_causal
    ctx.sm_scale = _default_scale(q)


def _non_softmax_backward(ctx, dout):
    q, k, v = ctx.saved_tensors
    dq, dk, dv = torch.ops.rbf_attn_v5.non_softmax_bwd(q, k, v, dout, ctx.is_causal, ctx.sm_scale)
    return dq, dk, dv, None


torch.library.register_autograd(
    f"{_V5}::non_softmax_fwd", _non_softmax_backward, setup_context=_non_softmax_setup_context
)


# ---------------------------------------------------------------------------
# Extended ops: explicit gamma (sm_scale) and register-prefix visibility.
# ---------------------------------------------------------------------------
@torch.library.custom_op(f"{_EX}::scaled_fwd_ex", mutates_args=())
def rbf_scaled_fwd_ex(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
    num_prefix: int,
    token_major: bool = False,
    pos: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    return _softmax_fwd(q, k, v, is_causal, sm_scale, num_prefix, token_major, pos)


def _fake_out(q: torch.Tensor, token_major: bool) -> torch.Tensor:
    dp = _padded_dim(q.shape[-1])
    if token_major and dp == q.shape[-1]:
        B, H, N, D = q.shape
        return torch.empty((B, N, H, D), device=q.device, dtype=q.dtype).transpose(1, 2)
    return torch.empty_like(q, memory_format=torch.contiguous_format)


@rbf_scaled_fwd_ex.register_fake
def _(q, k, v, is_causal, sm_scale, num_prefix, token_major=False, pos=None):
    B, H, N, _ = q.shape
    return _fake_out(q, token_major), torch.empty((B, H, N), device=q.device, dtype=torch.float32)


@torch.library.custom_op(f"{_EX}::scaled_bwd_ex", mutates_args=())
def rbf_scaled_bwd_ex(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    out: torch.Tensor,
    L: torch.Tensor,
    dout: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
    num_prefix: int,
    pos: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _softmax_bwd(q, k, v, out, L, dout, is_causal, sm_scale, num_prefix, pos)


@rbf_scaled_bwd_ex.register_fake
def _(q, k, v, out, L, dout, is_causal, sm_scale, num_prefix, pos=None):
    return tuple(torch.empty_like(t, memory_format=torch.contiguous_format) for t in (q, k, v))


def _pos_grad(pos, dq, dk):
    """Gradient of the position term added to q and k: dq + dk, summed over
    the batch when the term is shared by it."""
    if pos is None:
        return None
    g = dq + dk
    return g.sum(dim=0, keepdim=True) if pos.shape[0] == 1 and g.shape[0] != 1 else g


def _scaled_ex_setup_context(ctx, inputs, output):
    q, k, v, is_causal, sm_scale, num_prefix = inputs[:6]
    pos = inputs[7] if len(inputs) > 7 else None
    out, L = output
    ctx.save_for_backward(q, k, v, out, L, pos)
    ctx.is_causal, ctx.sm_scale, ctx.num_prefix = is_causal, sm_scale, num_prefix


def _scaled_ex_backward(ctx, dout, dL):
    q, k, v, out, L, pos = ctx.saved_tensors
    dq, dk, dv = torch.ops.rbf_attn_amd.scaled_bwd_ex(
        q, k, v, out, L, dout, ctx.is_causal, ctx.sm_scale, ctx.num_prefix, pos
    )
    return dq, dk, dv, None, None, None, None, _pos_grad(pos, dq, dk)


torch.library.register_autograd(f"{_EX}::scaled_fwd_ex", _scaled_ex_backward, setup_context=_scaled_ex_setup_context)


@torch.library.custom_op(f"{_EX}::non_softmax_fwd_ex", mutates_args=())
def rbf_non_softmax_fwd_ex(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
    num_prefix: int,
    token_major: bool = False,
    pos: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    return _non_softmax_fwd(q, k, v, is_causal, sm_scale, num_prefix, token_major, pos)


@rbf_non_softmax_fwd_ex.register_fake
def _(q, k, v, is_causal, sm_scale, num_prefix, token_major=False, pos=None):
    return _fake_out(q, token_major)


@torch.library.custom_op(f"{_EX}::non_softmax_bwd_ex", mutates_args=())
def rbf_non_softmax_bwd_ex(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    dout: torch.Tensor,
    is_causal: bool,
    sm_scale: float,
    num_prefix: int,
    pos: Optional[torch.Tensor] = None,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    return _non_softmax_bwd(q, k, v, dout, is_causal, sm_scale, num_prefix, pos)


@rbf_non_softmax_bwd_ex.register_fake
def _(q, k, v, dout, is_causal, sm_scale, num_prefix, pos=None):
    return tuple(torch.empty_like(t, memory_format=torch.contiguous_format) for t in (q, k, v))


def _non_softmax_ex_setup_context(ctx, inputs, output):
    q, k, v, is_causal, sm_scale, num_prefix = inputs[:6]
    pos = inputs[7] if len(inputs) > 7 else None
    ctx.save_for_backward(q, k, v, pos)
    ctx.is_causal, ctx.sm_scale, ctx.num_prefix = is_causal, sm_scale, num_prefix


def _non_softmax_ex_backward(ctx, dout):
    q, k, v, pos = ctx.saved_tensors
    dq, dk, dv = torch.ops.rbf_attn_amd.non_softmax_bwd_ex(
        q, k, v, dout, ctx.is_causal, ctx.sm_scale, ctx.num_prefix, pos
    )
    return dq, dk, dv, None, None, None, None, _pos_grad(pos, dq, dk)


torch.library.register_autograd(
    f"{_EX}::non_softmax_fwd_ex", _non_softmax_ex_backward, setup_context=_non_softmax_ex_setup_context
)


# ---------------------------------------------------------------------------
# KV-cache decode (no reference counterpart: the reference has no decode path)
# ---------------------------------------------------------------------------
def _decode(q, k_cache, v_cache, cache_lens, softmax: bool, sm_scale: float):
    if q.dim() != 4 or k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("decode: q must be (B, H, T, D) and the caches (B, H, L, D)")
    B, H, T, D = q.shape
    if k_cache.shape != v_cache.shape or k_cache.shape[:2] != (B, H) or k_cache.shape[3] != D:
        raise ValueError(f"decode: cache shapes {tuple(k_cache.shape)} / {tuple(v_cache.shape)} do not match q {tuple(q.shape)}")
    for t in (k_cache, v_cache):
        if t.dtype != q.dtype or t.device != q.device:
            raise TypeError("decode: q and the caches must share dtype and device")
    if q.dtype not in _lib.DTYPE_CODES:
        raise TypeError(f"decode: unsupported dtype {q.dtype} (bf16, fp16, fp32)")
    if q.device.type != "cuda":
        raise RuntimeError("decode: the kernels run only on a ROCm GPU (there is no CPU fallback)")
    if D > 256:
        raise ValueError(f"decode: head dim {D} > 256 is not supported")
    if not 1 <= T <= 32:
        raise ValueError(f"decode: {T} query tokens per step unsupported (1..32)")
    L = k_cache.shape[2]
    if L < T:
        raise ValueError(f"decode: cache length {L} < {T} query tokens")
    dp = _padded_dim(D)
    q_, k_, v_ = _prep(q, dp), _prep(k_cache, dp), _prep(v_cache, dp)
    out = torch.empty((B, H, T, dp), device=q.device, dtype=q.dtype)
    lse = torch.empty((B, H, T), device=q.device, dtype=torch.float32)
    if B * H == 0:
        return _unpad(out, D), lse
    a = _lib.DecodeArgs()
    a.abi_version = _lib.ABI_VERSION
    a.variant = _lib.SOFTMAX if softmax else _lib.NON_SOFTMAX
    a.dtype = _lib.DTYPE_CODES[q.dtype]
    a.B, a.H, a.T, a.D, a.L = B, H, T, dp, L
    a.gamma = float(sm_scale)
    a.q, a.k, a.v, a.o = (_lib.tensor_desc(t) for t in (q_, k_, v_, out))
    lens = None
    if cache_lens is not None:
        lens = cache_lens.to(device=q.device, dtype=torch.int32).contiguous()
        if lens.shape != (B,):
            raise ValueError(f"decode: cache_lens must have shape ({B},)")
        a.lens = lens.data_ptr()
    a.lse = lse.data_ptr() if softmax else None
    nbytes = _lib.decode_workspace_size(a)
    ws = torch.empty((nbytes + 15) // 16 * 4, device=q.device, dtype=torch.float32)
    a.workspace = ws.data_ptr()
    a.workspace_bytes = nbytes
    _call_on(q.device, "rbf_attn_decode", a)
    return _unpad(out, D), lse


@torch.library.custom_op(f"{_EX}::decode", mutates_args=())
def rbf_decode_op(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    cache_lens: torch.Tensor | None,
    softmax: bool,
    sm_scale: float,
) -> tuple[torch.Tensor, torch.Tensor]:
    return _decode(q, k_cache, v_cache, cache_lens, softmax, sm_scale)


@rbf_decode_op.register_fake
def _(q, k_cache, v_cache, cache_lens, softmax, sm_scale):
    B, H, T, _ = q.shape
    return torch.empty_like(q, memory_format=torch.contiguous_format), torch.empty(
        (B, H, T), device=q.device, dtype=torch.float32
    )


def rbf_decode(q, k_cache, v_cache, cache_lens=None, *, softmax=True, sm_scale=None):
    """Attention of T new query tokens (q: (B, H, T, D), 1 <= T <= 32) against
    a KV cache (B, H, L, D) that already holds their keys and values.  Query t
    of batch b sits at position cache_lens[b] - T + t (cache_lens defaults to
    L for every b) and sees keys [0, that position].  Returns (out, L) with L
    the base-2 log-sum-exp (softmax; unspecified for the non-softmax variant).
    Forward only."""
    scale = _default_scale(q) if sm_scale is None else float(sm_scale)
    if _eager_plain(q, k_cache, v_cache) and (cache_lens is None or type(cache_lens) is torch.Tensor):
        return _decode(q, k_cache, v_cache, cache_lens, bool(softmax), scale)  # the op's implementation
    return torch.ops.rbf_attn_amd.decode(q, k_cache, v_cache, cache_lens, bool(softmax), scale)


# ---------------------------------------------------------------------------
# Public wrappers (rbf_attention.py:848-853) and autograd.Function aliases.
# ---------------------------------------------------------------------------
class _EagerRbfAttention(torch.autograd.Function):
    """The wrappers' eager path: the ops' kernels and autograd formula (same
    implementations, so bit-identical results) without the torch.library
    dispatch, whose Python layers cost ~140 us of host time per forward +
    backward (MI355X box: 213 us through ``rbf_attn_v5::scaled_fwd`` and its
    registered autograd against 73 us this way, tiny shapes)."""

    @staticmethod
    def forward(ctx, q, k, v, pos, softmax, is_causal, scale, num_prefix, token_major):
        if softmax:
            out, L = _softmax_fwd(q, k, v, is_causal, scale, num_prefix, token_major, pos)
            ctx.save_for_backward(q, k, v, out, L, pos)
        else:
            out = _non_softmax_fwd(q, k, v, is_causal, scale, num_prefix, token_major, pos)
            ctx.save_for_backward(q, k, v, pos)
        ctx.cfg = (softmax, is_causal, scale, num_prefix)
        return out

    @staticmethod
    def backward(ctx, dout):
        softmax, is_causal, scale, num_prefix = ctx.cfg
        if softmax:
            q, k, v, out, L, pos = ctx.saved_tensors
            dq, dk, dv = _softmax_bwd(q, k, v, out, L, dout, is_causal, scale, num_prefix, pos)
        else:
            q, k, v, pos = ctx.saved_tensors
            dq, dk, dv = _non_softmax_bwd(q, k, v, dout, is_causal, scale, num_prefix, pos)
        return dq, dk, dv, _pos_grad(pos, dq, dk), None, None, None, None, None


def _eager_plain(*ts) -> bool:
    """Whether a wrapper call may take the eager path: plain GPU tensors (no
    subclass: fake, functional, distributed ...; no meta or CPU tensors), not
    under torch.compile / export tracing, no dispatch mode and no functorch
    transform.  Everything else goes through the registered ops, which those
    mechanisms know (and which raise for CPU tensors)."""
    if torch.compiler.is_compiling() or torch._C._are_functorch_transforms_active():
        return False
    if _python_dispatch._get_current_dispatch_mode() is not None:
        return False
    return all(t is None or (type(t) is torch.Tensor and t.is_cuda) for t in ts)


def run_triton_rbf(q, k, v, is_causal=True, *, sm_scale=None, num_prefix=0, token_major=False, pos=None):
    """Softmax RBF attention.  With the default ``sm_scale`` (1/sqrt(D)),
    ``num_prefix=0``, ``token_major=False`` and no ``pos`` this is exactly the
    reference's ``run_triton_rbf``.  ``token_major=True`` returns the
    (B, H, N, D) output as a view of a (B, N, H, D) buffer (see
    ``_alloc_out``).  ``pos`` (1 or B, H, N, D): attention of q + pos and
    k + pos (the model's SuSiE embedding), fused into the kernels' Q/K reads
    where the library supports it; its gradient is returned by autograd.
    Eager calls on plain tensors run the ops' implementations directly
    (``_EagerRbfAttention``); traced and transformed calls run the ops."""
    if _eager_plain(q, k, v, pos):
        scale = _default_scale(q) if sm_scale is None else float(sm_scale)
        return _EagerRbfAttention.apply(q, k, v, pos, True, bool(is_causal), scale, int(num_prefix), bool(token_major))
    if sm_scale is None and num_prefix == 0 and not token_major and pos is None:
        return torch.ops.rbf_attn_v5.scaled_fwd(q, k, v, is_causal)[0]
    scale = _default_scale(q) if sm_scale is None else float(sm_scale)
    return torch.ops.rbf_attn_amd.scaled_fwd_ex(q, k, v, is_causal, scale, int(num_prefix), bool(token_major), pos)[0]


def run_triton_non_softmax_rbf(q, k, v, is_causal=True, *, sm_scale=None, num_prefix=0, token_major=False, pos=None):
    """Non-softmax RBF attention, sum_j exp(-gamma||q_i-k_j||^2) v_j (pos and
    the eager path as in ``run_triton_rbf``)."""
    if _eager_plain(q, k, v, pos):
        scale = _default_scale(q) if sm_scale is None else float(sm_scale)
        return _EagerRbfAttention.apply(q, k, v, pos, False, bool(is_causal), scale, int(num_prefix), bool(token_major))
    if sm_scale is None and num_prefix == 0 and not token_major and pos is None:
        return torch.ops.rbf_attn_v5.non_softmax_fwd(q, k, v, is_causal)
    scale = _default_scale(q) if sm_scale is None else float(sm_scale)
    return torch.ops.rbf_attn_amd.non_softmax_fwd_ex(
        q, k, v, is_causal, scale, int(num_prefix), bool(token_major), pos
    )


class TritonRBFAttention(torch.autograd.Function):
    """``TritonRBFAttention.apply(q, k, v, is_causal=True, sm_scale=None,
    num_prefix=0)`` -> out.  Same kernels as ``run_triton_rbf``."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal=True, sm_scale=None, num_prefix=0):
        scale = _default_scale(q) if sm_scale is None else float(sm_scale)
        out, L = _softmax_fwd(q, k, v, bool(is_causal), scale, int(num_prefix))
        ctx.save_for_backward(q, k, v, out, L)
        ctx.cfg = (bool(is_causal), scale, int(num_prefix))
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, out, L = ctx.saved_tensors
        dq, dk, dv = _softmax_bwd(q, k, v, out, L, dout, *ctx.cfg)
        return dq, dk, dv, None, None, None


class TritonNonSoftmaxRBFAttention(torch.autograd.Function):
    """``TritonNonSoftmaxRBFAttention.apply(q, k, v, is_causal=True,
    sm_scale=None, num_prefix=0)`` -> out."""

    @staticmethod
    def forward(ctx, q, k, v, is_causal=True, sm_scale=None, num_prefix=0):
        scale = _default_scale(q) if sm_scale is None else float(sm_scale)
        out = _non_softmax_fwd(q, k, v, bool(is_causal), scale, int(num_prefix))
        ctx.save_for_backward(q, k, v)
        ctx.cfg = (bool(is_causal), scale, int(num_prefix))
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v = ctx.saved_tensors
        dq, dk, dv = _non_softmax_bwd(q, k, v, dout, *ctx.cfg)
        return dq, dk, dv, None, None, None
