"""The C-ABI entry points only enqueue kernels on the caller's stream: they
allocate nothing, never synchronise and issue no memset, so a forward +
backward step can be captured in a HIP graph and replayed.  Every replay must
give the eager results bit for bit; eager work and synchronisations run
between the replays, and the outputs are cleared before each one."""
import pytest
import torch

from rbf_attention_amd import _lib

pytestmark = pytest.mark.gpu


def setup(B, H, N, D, softmax, dev, seed):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, N, D, generator=g).to(torch.bfloat16).to(dev) for _ in range(4))
    bufs = {"q": q, "k": k, "v": v, "dout": do}
    for f in ("o", "dq", "dk", "dv"):
        bufs[f] = torch.zeros_like(q)
    bufs["lse"] = torch.zeros((B, H, N), device=dev, dtype=torch.float32)
    bufs["delta"] = torch.zeros_like(bufs["lse"])
    a = _lib.Args()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0 if softmax else 1, _lib.DTYPE_CODES[torch.bfloat16]
    a.B, a.H, a.N, a.D, a.causal, a.num_prefix, a.gamma = B, H, N, D, 1, 4, 1.0 / (2 * D ** 0.5)
    for f in ("q", "k", "v", "o", "dout", "dq", "dk", "dv"):
        setattr(a, f, _lib.tensor_desc(bufs[f]))
    a.lse, a.delta = bufs["lse"].data_ptr(), bufs["delta"].data_ptr()
    return a, bufs


def step(a):
    sp = torch.cuda.current_stream().cuda_stream
    _lib.call("rbf_attn_fwd", a, sp)
    _lib.call("rbf_attn_bwd", a, sp)


@pytest.mark.parametrize(
    "B,H,N,D,softmax",
    [
        (16, 16, 516, 64, True),  # head-resident forward, one-launch backward
        (16, 16, 300, 64, False),  # the same, non-softmax
        (2, 4, 700, 64, True),  # streaming kernels, two backward launches
        (1, 2, 1030, 128, True),  # streaming D = 128 (paired dK/dV kernel)
    ],
)
def test_graph_replay_matches_eager(cuda_device, B, H, N, D, softmax):
    print(f"graph replay B={B} H={H} N={N} D={D} softmax={softmax}", flush=True)
    a, bufs = setup(B, H, N, D, softmax, cuda_device, seed=N + D)
    outs = ("o", "lse", "dq", "dk", "dv", "delta")
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(a)  # eager reference (also settles the library's one-time queries before capture)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ref = {f: bufs[f].clone() for f in outs}

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(a)
    torch.cuda.synchronize()
    for rep in range(3):
        for f in outs:
            bufs[f].zero_()
        noise = torch.randn(1 << 20, device=cuda_device).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for f in outs:
            assert torch.equal(bufs[f], ref[f]), f"replay {rep}: {f} differs from eager"
        assert torch.isfinite(noise)


@pytest.mark.parametrize(
    "B,H,N,D,softmax,pos",
    [
        (16, 16, 516, 64, True, False),  # head-resident kernels
        (16, 16, 516, 64, True, True),  # fused position term and its gradient
        (2, 4, 700, 64, False, False),  # streaming kernels, non-softmax
    ],
)
def test_op_graph_replay_matches_eager(cuda_device, B, H, N, D, softmax, pos):
    """The torch ops and their autograd under capture: forward through
    run_triton_rbf / run_triton_non_softmax_rbf, then backward, recorded in one
    graph (outputs and gradients come from the graph's memory pool).  New
    input values copied into the captured inputs give, on replay, the eager
    results on those values bit for bit."""
    import rbf_attention_amd as ra

    print(f"op graph replay B={B} H={H} N={N} D={D} softmax={softmax} pos={pos}", flush=True)
    fn = ra.run_triton_rbf if softmax else ra.run_triton_non_softmax_rbf
    kw = dict(sm_scale=1.0 / (2 * D ** 0.5), num_prefix=4)

    def draw(seed):
        g = torch.Generator().manual_seed(seed)
        ts = [torch.randn(B, H, N, D, generator=g) * (1.0 if softmax else 0.5) for _ in range(4)]
        p = torch.randn(1, H, N, D, generator=g) * 0.1
        return [t.to(torch.bfloat16).to(cuda_device) for t in ts + [p]]

    def eager(vals):
        q, k, v, do, p = (t.clone() for t in vals)
        leaves = [q, k, v] + ([p] if pos else [])
        for t in leaves:
            t.requires_grad_(True)
        out = fn(q, k, v, True, pos=p if pos else None, **kw)
        out.backward(do)
        torch.cuda.synchronize()
        return [out.detach()] + [t.grad for t in leaves]

    static = [t.clone() for t in draw(1)]
    sq, sk, sv, sdo, sp = static
    leaves = [sq, sk, sv] + ([sp] if pos else [])
    for t in leaves:
        t.requires_grad_(True)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up outside the capture
        for _ in range(2):
            for t in leaves:
                t.grad = None
            fn(sq, sk, sv, True, pos=sp if pos else None, **kw).backward(sdo)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    for t in leaves:
        t.grad = None
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        sout = fn(sq, sk, sv, True, pos=sp if pos else None, **kw)
        sout.backward(sdo)
    torch.cuda.synchronize()
    for rep, seed in enumerate((2, 3, 2)):
        vals = draw(seed)
        ref = eager(vals)
        with torch.no_grad():
            for dst, src in zip(static, vals):
                dst.copy_(src)
        noise = torch.randn(1 << 20, device=cuda_device).sum()  # unrelated eager work between replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got = [sout.detach()] + [t.grad for t in leaves]
        for name, a, b in zip(("out", "dq", "dk", "dv", "dpos"), got, ref):
            assert torch.equal(a, b), f"replay {rep} (seed {seed}): {name} differs from eager"
        assert torch.isfinite(noise)
