"""CPU tests of the C-ABI library: it loads, exports every symbol that
include/rbf_attn.h declares, and rejects bad arguments with the documented
error codes before any HIP call (no GPU work is issued here)."""
import ctypes
import os
import re

import pytest
import torch  # noqa: F401  (binds the library to torch's HIP runtime)

from rbf_attention_amd import _lib

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "rbf_attn.h")


def header_functions():
    src = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(rbf_attn_\w+)\s*\(", src, re.M)))


def header_define(name):
    m = re.search(rf"#define\s+{name}\s+(-?\d+)", open(HEADER).read())
    return int(m.group(1))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(_lib.LIB_PATH):
        pytest.fail(f"{_lib.LIB_PATH} missing: run `python -m rbf_attention_amd.build` (or __graft_entry__.build())")
    return _lib.load()


def test_exports_match_header(lib):
    names = header_functions()
    assert set(names) == set(_lib.EXPORTS), names
    for n in names:
        assert hasattr(lib, n), n


def test_abi_version(lib):
    assert lib.rbf_attn_abi_version() == header_define("RBF_ATTN_ABI_VERSION") == _lib.ABI_VERSION


def test_error_codes_match_header():
    for code, name in _lib.ERRORS.items():
        assert header_define(f"RBF_ATTN_{name}") == code


def test_struct_layout():
    # 10 int32/float fields, 8 tensors of 32 bytes, 2 pointers
    assert ctypes.sizeof(_lib.Tensor) == 32
    assert _lib.Args.q.offset == 40
    assert ctypes.sizeof(_lib.Args) == 40 + 8 * 32 + 16


FAKE = 0x10000  # aligned, never dereferenced: every call below fails validation or is empty


def good_args(**over):
    a = _lib.Args()
    a.abi_version = _lib.ABI_VERSION
    a.variant = 0
    a.dtype = 0
    a.B, a.H, a.N, a.D = 2, 3, 64, 64
    a.causal = 1
    a.num_prefix = 0
    a.gamma = 0.125
    for i, f in enumerate(("q", "k", "v", "o", "dout", "dq", "dk", "dv")):
        setattr(a, f, _lib.Tensor(FAKE + 0x100000 * i, 3 * 64 * 64, 64 * 64, 64))
    a.lse = FAKE + 0x1000000
    a.delta = FAKE + 0x2000000
    for k, v in over.items():
        setattr(a, k, v)
    return a


def call(lib, fn, a):
    return getattr(lib, fn)(ctypes.byref(a) if a is not None else None, None)


@pytest.mark.parametrize("fn", ["rbf_attn_fwd", "rbf_attn_bwd"])
@pytest.mark.parametrize(
    "over,code",
    [
        (dict(abi_version=1), -1),
        (dict(variant=5), -1),
        (dict(dtype=7), -2),
        (dict(D=60), -4),
        (dict(D=132), -4),
        (dict(D=264), -4),
        (dict(D=0), -4),
        (dict(B=-1), -5),
        (dict(causal=2), -1),
        (dict(num_prefix=-1), -1),
        (dict(gamma=0.0), -1),
        (dict(gamma=float("nan")), -1),
        (dict(q=_lib.Tensor(None, 0, 0, 0)), -6),
        (dict(k=_lib.Tensor(FAKE + 2, 3 * 64 * 64, 64 * 64, 64)), -3),
        (dict(v=_lib.Tensor(FAKE, 3 * 64 * 64, 64 * 64, 63)), -3),
        (dict(lse=None), -6),
    ],
)
def test_validation(lib, fn, over, code):
    a = good_args(**over)
    assert call(lib, fn, a) == code
    assert lib.rbf_attn_last_error().decode()


def test_null_args(lib):
    assert call(lib, "rbf_attn_fwd", None) == -1
    assert call(lib, "rbf_attn_bwd", None) == -1


def test_bwd_requires_delta_for_softmax_only(lib):
    assert call(lib, "rbf_attn_bwd", good_args(delta=None, N=0)) == -6
    assert call(lib, "rbf_attn_bwd", good_args(delta=None, N=0, variant=1)) == 0


def test_fp32_alignment(lib):
    # fp32 row stride of 4 elements = 16 bytes is fine; 2 elements is not
    a = good_args(dtype=2, N=0)
    assert call(lib, "rbf_attn_fwd", a) == 0
    a = good_args(dtype=2, N=0, q=_lib.Tensor(FAKE, 64, 64, 2))
    assert call(lib, "rbf_attn_fwd", a) == -3


def test_noalloc_validation(lib):
    """rbf_attn_bwd_noalloc: same validation as rbf_attn_bwd, its workspace
    pointers are not required, and problems beyond the static workspace are
    rejected before any HIP call (nothing here reaches the device)."""
    m = re.search(r"#define\s+RBF_ATTN_NOALLOC_MAX_ROWS\s+\(1 << (\d+)\)", open(HEADER).read())
    assert m and (1 << int(m.group(1))) == _lib.NOALLOC_MAX_ROWS
    f = lib.rbf_attn_bwd_noalloc
    assert f(None, None) == -1
    big = good_args(B=16, H=64, N=1025)  # 1,049,600 rows > 2^20
    assert f(ctypes.byref(big), None) == -5
    assert "workspace" in lib.rbf_attn_last_error().decode()
    # at the limit: past the size check, stopped by the null q before any launch
    assert f(ctypes.byref(good_args(B=16, H=64, N=1024, q=_lib.Tensor(None, 0, 0, 0))), None) == -6
    assert f(ctypes.byref(good_args(D=60)), None) == -4
    # workspaces: delta never needed; lse needed for softmax (the forward's L) only
    assert f(ctypes.byref(good_args(N=0, delta=None)), None) == 0
    assert f(ctypes.byref(good_args(N=0, delta=None, lse=None)), None) == -6
    assert f(ctypes.byref(good_args(N=0, delta=None, lse=None, variant=1)), None) == 0
    assert f(ctypes.byref(good_args(q=_lib.Tensor(None, 0, 0, 0))), None) == -6


def test_empty_problem_is_noop(lib):
    for over in (dict(B=0), dict(H=0), dict(N=0)):
        assert call(lib, "rbf_attn_fwd", good_args(**over)) == 0
        assert call(lib, "rbf_attn_bwd", good_args(**over)) == 0
        assert lib.rbf_attn_last_error().decode() == ""


# ---------------------------------------------------------------------------
# position-term entry points (errors only: nothing here reaches a launch)
# ---------------------------------------------------------------------------
def test_pos_supported(lib):
    def sup(**over):
        return lib.rbf_attn_pos_supported(ctypes.byref(good_args(**over)))

    assert sup(N=516) == 1 and sup(N=576, dtype=1) == 1 and sup(D=40) == 1
    assert sup(dtype=2) == 0 and sup(D=128) == 0 and sup(D=32) == 0 and sup(N=577) == 0
    assert sup(dtype=7) == -2 and sup(D=60) == -4


def pos_term(stride_b=0, batch=1, ptr=FAKE + 0x3000000):
    return _lib.PosTerm(_lib.Tensor(ptr, stride_b, 64 * 64, 64), batch)


def test_pos_struct_layout():
    assert ctypes.sizeof(_lib.PosTerm) == 40 and _lib.PosTerm.batch.offset == 32


def test_pos_entry_points_reject_before_launch(lib):
    pos = pos_term()
    for fn in (lib.rbf_attn_fwd_pos, lib.rbf_attn_bwd_pos):
        assert fn(ctypes.byref(good_args()), None, None) == -6
        assert fn(ctypes.byref(good_args(D=128)), ctypes.byref(pos), None) == -8
        assert "576" in lib.rbf_attn_last_error().decode()
        assert fn(ctypes.byref(good_args(dtype=2)), ctypes.byref(pos), None) == -8
        bad = pos_term(ptr=FAKE + 0x3000008)
        assert fn(ctypes.byref(good_args()), ctypes.byref(bad), None) == -3
        assert fn(ctypes.byref(good_args(N=0)), ctypes.byref(pos), None) == 0


def test_pos_batch_extent(lib):
    """A term shared by the batch (batch = 1) is read at every b, so it must
    come with stride_b = 0: a batch-1 term passed with its own batch stride
    would be read past its end.  Both misuses are rejected before any launch
    (good_args has B = 2)."""
    for fn in (lib.rbf_attn_fwd_pos, lib.rbf_attn_bwd_pos):
        shared_with_stride = pos_term(stride_b=3 * 64 * 64, batch=1)
        assert fn(ctypes.byref(good_args()), ctypes.byref(shared_with_stride), None) == -3
        assert "stride_b" in lib.rbf_attn_last_error().decode()
        for batch in (0, 3, -1):
            assert fn(ctypes.byref(good_args()), ctypes.byref(pos_term(stride_b=64 * 64, batch=batch)), None) == -5
            assert "batch" in lib.rbf_attn_last_error().decode()
        # accepted descriptors (N = 0: validated, nothing launched)
        assert fn(ctypes.byref(good_args(N=0)), ctypes.byref(pos_term(stride_b=0, batch=1)), None) == 0
        assert fn(ctypes.byref(good_args(N=0)), ctypes.byref(pos_term(stride_b=3 * 64 * 64, batch=2)), None) == 0
        # one batch entry: its stride is never used
        assert fn(ctypes.byref(good_args(B=1, N=0)), ctypes.byref(pos_term(stride_b=7 * 64, batch=1)), None) == 0
    n = lib.rbf_attn_bwd_kernels(ctypes.byref(good_args(N=516)), ctypes.byref(pos_term(stride_b=64, batch=1)))
    assert n == -3


def test_pos_desc_of_shared_term():
    """The op layer's descriptor of a (1, H, N, D) term carries stride_b = 0
    whatever the tensor's own batch stride is."""
    t = torch.empty(1, 3, 64, 64)
    d = _lib.pos_desc(t)
    assert d.batch == 1 and d.t.stride_b == 0 and d.t.stride_h == 64 * 64
    t2 = torch.empty(2, 3, 64, 64)
    d2 = _lib.pos_desc(t2)
    assert d2.batch == 2 and d2.t.stride_b == 3 * 64 * 64


def test_bwd_kernels_query(lib):
    """Shapes decided without a device query: fp32 and D > 64 always take two
    launches, a fused position term on a head that fits takes one."""
    pos = pos_term()

    def n(over, p=None):
        return lib.rbf_attn_bwd_kernels(ctypes.byref(good_args(**over)), ctypes.byref(p) if p else None)

    assert n(dict(dtype=2)) == 2 and n(dict(D=128)) == 2 and n(dict(D=32)) == 2
    assert n(dict(N=516), pos) == 1 and n(dict(N=516, dtype=1), pos) == 1
    assert n(dict(N=577), pos) == -8 and n(dict(D=128), pos) == -8
    assert n(dict(N=0)) == 0
    assert n(dict(dtype=7)) == -2 and n(dict(D=60)) == -4
    assert lib.rbf_attn_bwd_kernels(None, None) == -1


# ---------------------------------------------------------------------------
# decode entry points
# ---------------------------------------------------------------------------
def test_decode_struct_layout():
    # 9 int32/float fields, padding, 4 tensors, 3 pointers, one uint64
    assert _lib.DecodeArgs.q.offset == 40
    assert _lib.DecodeArgs.lens.offset == 40 + 4 * 32
    assert ctypes.sizeof(_lib.DecodeArgs) == 40 + 4 * 32 + 4 * 8


def decode_args(**over):
    a = _lib.DecodeArgs()
    a.abi_version, a.variant, a.dtype = _lib.ABI_VERSION, 0, 0
    a.B, a.H, a.T, a.D, a.L = 2, 3, 1, 64, 1000
    a.gamma = 0.0625
    for f in ("q", "k", "v", "o"):
        setattr(a, f, _lib.Tensor(FAKE, 64 * 4096, 64 * 1024, 64))
    for kk, vv in over.items():
        setattr(a, kk, vv)
    return a


def test_decode_workspace_size(lib):
    # 6 (b, h) pairs want hundreds of work-groups but 1000 keys make only 8
    # tiles of 128: 8 splits x 4 waves = 32 partials of (64 + 2) floats per query.
    assert lib.rbf_attn_decode_workspace_size(ctypes.byref(decode_args())) == 6 * 32 * 1 * 66 * 4
    # fp32 runs 2 waves per 64-key tile: 16 tiles, 16 splits
    assert lib.rbf_attn_decode_workspace_size(ctypes.byref(decode_args(dtype=2))) == 6 * 32 * 1 * 66 * 4
    # 128 (b, h) pairs, 16K keys, 128 features: 512 work-groups = 4 splits
    big = decode_args(B=8, H=16, T=1, D=128, L=16384)
    assert lib.rbf_attn_decode_workspace_size(ctypes.byref(big)) == 128 * 16 * 1 * 130 * 4
    # 256 features: one work-group per CU, 256 in total = 2 splits x 4 waves
    wide = decode_args(B=8, H=16, T=1, D=256, L=16384)
    assert lib.rbf_attn_decode_workspace_size(ctypes.byref(wide)) == 128 * 8 * 1 * 258 * 4


@pytest.mark.parametrize("over", [dict(T=0), dict(T=33), dict(L=0), dict(T=4, L=3), dict(D=12), dict(D=264),
                                  dict(gamma=0.0), dict(variant=2), dict(dtype=5), dict(abi_version=0)])
def test_decode_validation(lib, over):
    a = decode_args(**over)
    assert lib.rbf_attn_decode_workspace_size(ctypes.byref(a)) == 0
    assert lib.rbf_attn_last_error() != b""
    assert lib.rbf_attn_decode(ctypes.byref(a), None) < 0


def test_decode_workspace_checks(lib):
    a = decode_args()
    assert lib.rbf_attn_decode(ctypes.byref(a), None) == header_define("RBF_ATTN_EINVAL_PTR")
    a.workspace, a.workspace_bytes = FAKE, 100
    assert lib.rbf_attn_decode(ctypes.byref(a), None) == header_define("RBF_ATTN_EINVAL_ARGS")
    b = decode_args(q=_lib.Tensor(FAKE + 8, 0, 0, 64))
    assert lib.rbf_attn_decode(ctypes.byref(b), None) == header_define("RBF_ATTN_EINVAL_STRIDE")


def test_decode_empty_batch_is_noop(lib):
    a = decode_args(B=0)
    assert lib.rbf_attn_decode(ctypes.byref(a), None) == 0
