"""rbf_attn_bwd_noalloc (the backward whose per-query workspace is the
library's static device array) against rbf_attn_bwd (caller workspace),
through the C ABI: bit-identical dq, dk, dv on two calls in a row, the
second with a smaller problem, for both variants and both backward forms
(one head-resident launch, and the two streaming launches); captured in a
HIP graph (the first call of the process, so that the per-device lookup of
the array runs under capture) and replayed; and at the largest problem the
array holds, B * H * N = RBF_ATTN_NOALLOC_MAX_ROWS."""
import math

import pytest
import torch

from rbf_attention_amd import _lib

pytestmark = pytest.mark.gpu


def make(B, H, N, D, dtype, dev, softmax, seed):
    g = torch.Generator().manual_seed(seed)
    std = 1.0 if softmax else 0.5
    bufs = {f: (torch.randn(B, H, N, D, generator=g) * std).to(dtype).to(dev) for f in ("q", "k", "v", "dout")}
    for f in ("o", "dq", "dk", "dv"):
        bufs[f] = torch.zeros(B, H, N, D, device=dev, dtype=dtype)
    bufs["lse"] = torch.zeros(B, H, N, device=dev, dtype=torch.float32)
    bufs["delta"] = torch.zeros_like(bufs["lse"])
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[dtype]
    a.B, a.H, a.N, a.D, a.causal, a.num_prefix, a.gamma = B, H, N, D, 1, 0, 1.0 / (2 * math.sqrt(D))
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(bufs[f]))
    a.lse, a.delta = bufs["lse"].data_ptr(), bufs["delta"].data_ptr()
    return bufs, a


def run_pair(bufs, a, sp):
    """(dq, dk, dv) of rbf_attn_bwd, then of rbf_attn_bwd_noalloc on the same
    inputs with the caller workspaces poisoned (NaN) and detached from args."""
    _lib.call("rbf_attn_fwd", a, sp)
    _lib.call("rbf_attn_bwd", a, sp)
    ref = [bufs[f].clone() for f in ("dq", "dk", "dv")]
    for f in ("dq", "dk", "dv"):
        bufs[f].zero_()
    if a.variant == 1:
        bufs["lse"].fill_(float("nan"))  # the non-softmax workspace slot: must not be read
        a.lse = None
    bufs["delta"].fill_(float("nan"))
    a.delta = None
    _lib.call("rbf_attn_bwd_noalloc", a, sp)
    torch.cuda.synchronize()
    return ref, [bufs[f] for f in ("dq", "dk", "dv")]


def test_noalloc_graph_capture_replays(cuda_device):
    """The entry point is for callers under graph capture: captured (as the
    process's first call of it, when run first in a fresh process or in the
    suite), its replays reproduce rbf_attn_bwd bit for bit, three times, with
    the outputs cleared and eager work run between the replays."""
    bufs, a = make(2, 4, 700, 128, torch.bfloat16, cuda_device, True, seed=31)
    sp = torch.cuda.current_stream(cuda_device).cuda_stream
    _lib.call("rbf_attn_fwd", a, sp)
    _lib.call("rbf_attn_bwd", a, sp)
    torch.cuda.synchronize()
    ref = [bufs[f].clone() for f in ("dq", "dk", "dv")]
    a.delta = None
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(cuda_device)
    side.wait_stream(torch.cuda.current_stream(cuda_device))
    with torch.cuda.stream(side):
        with torch.cuda.graph(graph, stream=side):
            _lib.call("rbf_attn_bwd_noalloc", a, torch.cuda.current_stream(cuda_device).cuda_stream)
    torch.cuda.current_stream(cuda_device).wait_stream(side)
    for rep in range(3):
        for f in ("dq", "dk", "dv"):
            bufs[f].zero_()
        _ = (bufs["q"].float() * 2).sum().item()  # eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        for name, x in zip(("dq", "dk", "dv"), ref):
            y = bufs[name]
            assert torch.equal(x, y), f"replay {rep} {name}: max diff {(x.float() - y.float()).abs().max().item():.3e}"


@pytest.mark.parametrize("softmax", [True, False])
@pytest.mark.parametrize("shapes", [((16, 16, 516, 64), (2, 3, 200, 64)), ((2, 4, 700, 128), (1, 2, 90, 128))])
def test_noalloc_equals_bwd_twice(cuda_device, softmax, shapes):
    sp = torch.cuda.current_stream(cuda_device).cuda_stream
    for i, (B, H, N, D) in enumerate(shapes):
        print(f"noalloc softmax={softmax} call {i}: B={B} H={H} N={N} D={D}", flush=True)
        bufs, a = make(B, H, N, D, torch.bfloat16, cuda_device, softmax, seed=N + i)
        ref, got = run_pair(bufs, a, sp)
        for name, x, y in zip(("dq", "dk", "dv"), ref, got):
            assert torch.isfinite(y).all(), name
            assert torch.equal(x, y), f"{name}: max diff {(x.float() - y.float()).abs().max().item():.3e}"
        assert ref[0].abs().sum() > 0


def test_noalloc_at_max_rows(cuda_device):
    """B * H * N = RBF_ATTN_NOALLOC_MAX_ROWS: the last entry of the array is
    written and read; then a smaller call."""
    sp = torch.cuda.current_stream(cuda_device).cuda_stream
    for i, (B, H, N, D) in enumerate(((16, 64, 1024, 64), (1, 3, 333, 64))):
        assert i == 1 or B * H * N == _lib.NOALLOC_MAX_ROWS
        print(f"noalloc max rows call {i}: B={B} H={H} N={N} D={D}", flush=True)
        bufs, a = make(B, H, N, D, torch.bfloat16, cuda_device, True, seed=40 + i)
        ref, got = run_pair(bufs, a, sp)
        for name, x, y in zip(("dq", "dk", "dv"), ref, got):
            assert torch.equal(x, y), f"{name}: max diff {(x.float() - y.float()).abs().max().item():.3e}"
        del bufs, ref, got
        torch.cuda.empty_cache()


def test_noalloc_rejects_oversize(cuda_device):
    bufs, a = make(1, 1, 64, 64, torch.bfloat16, cuda_device, True, seed=1)
    a.B, a.H, a.N = 1, 1, _lib.NOALLOC_MAX_ROWS + 1  # validated before any pointer is used
    with pytest.raises(_lib.RbfAttnError, match="workspace"):
        _lib.call("rbf_attn_bwd_noalloc", a, torch.cuda.current_stream(cuda_device).cuda_stream)
