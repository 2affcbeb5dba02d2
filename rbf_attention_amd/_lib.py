"""ctypes binding of librbfattn.so (declarations in include/rbf_attn.h).

The library is loaded lazily, after ``import torch``: torch ships its own
libamdhip64.so with the same SONAME as ROCm's, so the dynamic loader binds the
kernels' HIP runtime to torch's copy and the stream handles torch hands out
are valid in the library.  ``load()`` checks that only one HIP runtime is
mapped in the process.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must be imported before the library is loaded)

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(PKG_DIR, "librbfattn.so")

ABI_VERSION = 2
SOFTMAX = 0
NON_SOFTMAX = 1
DTYPE_CODES = {torch.bfloat16: 0, torch.float16: 1, torch.float32: 2}
NOALLOC_MAX_ROWS = 1 << 20  # RBF_ATTN_NOALLOC_MAX_ROWS: B*H*N limit of rbf_attn_bwd_noalloc

ERRORS = {
    -1: "EINVAL_ARGS",
    -2: "EINVAL_DTYPE",
    -3: "EINVAL_STRIDE",
    -4: "EINVAL_HEADDIM",
    -5: "EINVAL_SHAPE",
    -6: "EINVAL_PTR",
    -7: "ELAUNCH",
    -8: "EUNSUPPORTED",
}

# Every extern "C" entry point of include/rbf_attn.h.
EXPORTS = (
    "rbf_attn_fwd",
    "rbf_attn_bwd",
    "rbf_attn_bwd_stage",
    "rbf_attn_bwd_noalloc",
    "rbf_attn_fwd_pos",
    "rbf_attn_bwd_pos",
    "rbf_attn_bwd_kernels",
    "rbf_attn_pos_supported",
    "rbf_attn_decode_workspace_size",
    "rbf_attn_decode",
    "rbf_attn_last_error",
    "rbf_attn_abi_version",
)


class Tensor(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_b", ctypes.c_int64),
        ("stride_h", ctypes.c_int64),
        ("stride_n", ctypes.c_int64),
    ]


class PosTerm(ctypes.Structure):
    """rbf_attn_pos_term: a (batch, H, N, D) position term, batch 1 or B."""

    _fields_ = [("t", Tensor), ("batch", ctypes.c_int32)]


class Args(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("N", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("num_prefix", ctypes.c_int32),
        ("gamma", ctypes.c_float),
        ("q", Tensor),
        ("k", Tensor),
        ("v", Tensor),
        ("o", Tensor),
        ("dout", Tensor),
        ("dq", Tensor),
        ("dk", Tensor),
        ("dv", Tensor),
        ("lse", ctypes.c_void_p),
        ("delta", ctypes.c_void_p),
    ]


class DecodeArgs(ctypes.Structure):
    _fields_ = [
        ("abi_version", ctypes.c_int32),
        ("variant", ctypes.c_int32),
        ("dtype", ctypes.c_int32),
        ("B", ctypes.c_int32),
        ("H", ctypes.c_int32),
        ("T", ctypes.c_int32),
        ("D", ctypes.c_int32),
        ("L", ctypes.c_int32),
        ("gamma", ctypes.c_float),
        ("q", Tensor),
        ("k", Tensor),
        ("v", Tensor),
        ("o", Tensor),
        ("lens", ctypes.c_void_p),
        ("lse", ctypes.c_void_p),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_uint64),
    ]


class RbfAttnError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, code: int, message: str):
        self.code = code
        super().__init__(f"librbfattn: {ERRORS.get(code, code)}: {message}")


_lock = threading.Lock()
_lib = None


def _hip_runtimes_mapped() -> set[str]:
    paths = set()
    try:
        with open("/proc/self/maps") as f:
            for line in f:
                if "libamdhip64" in line:
                    paths.add(os.path.realpath(line.split()[-1]))
    except OSError:
        pass
    return paths


def load(path: str | None = None):
    """Load (once) and return the ctypes handle of librbfattn.so."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = path or LIB_PATH
        if not os.path.exists(path):
            raise RuntimeError(
                f"{path} is missing: build it with `python -m rbf_attention_amd.build` "
                "(there is no fallback implementation)"
            )
        lib = ctypes.CDLL(path)
        for name in EXPORTS:
            if not hasattr(lib, name):
                raise RuntimeError(f"{path} does not export {name}")
        lib.rbf_attn_fwd.argtypes = [ctypes.POINTER(Args), ctypes.c_void_p]
        lib.rbf_attn_fwd.restype = ctypes.c_int
        lib.rbf_attn_bwd.argtypes = [ctypes.POINTER(Args), ctypes.c_void_p]
        lib.rbf_attn_bwd.restype = ctypes.c_int
        lib.rbf_attn_bwd_stage.argtypes = [ctypes.POINTER(Args), ctypes.c_void_p, ctypes.c_int]
        lib.rbf_attn_bwd_stage.restype = ctypes.c_int
        lib.rbf_attn_bwd_noalloc.argtypes = [ctypes.POINTER(Args), ctypes.c_void_p]
        lib.rbf_attn_bwd_noalloc.restype = ctypes.c_int
        lib.rbf_attn_fwd_pos.argtypes = [ctypes.POINTER(Args), ctypes.POINTER(PosTerm), ctypes.c_void_p]
        lib.rbf_attn_fwd_pos.restype = ctypes.c_int
        lib.rbf_attn_bwd_pos.argtypes = [ctypes.POINTER(Args), ctypes.POINTER(PosTerm), ctypes.c_void_p]
        lib.rbf_attn_bwd_pos.restype = ctypes.c_int
        lib.rbf_attn_bwd_kernels.argtypes = [ctypes.POINTER(Args), ctypes.POINTER(PosTerm)]
        lib.rbf_attn_bwd_kernels.restype = ctypes.c_int
        lib.rbf_attn_pos_supported.argtypes = [ctypes.POINTER(Args)]
        lib.rbf_attn_pos_supported.restype = ctypes.c_int
        lib.rbf_attn_decode_workspace_size.argtypes = [ctypes.POINTER(DecodeArgs)]
        lib.rbf_attn_decode_workspace_size.restype = ctypes.c_uint64
        lib.rbf_attn_decode.argtypes = [ctypes.POINTER(DecodeArgs), ctypes.c_void_p]
        lib.rbf_attn_decode.restype = ctypes.c_int
        lib.rbf_attn_last_error.argtypes = []
        lib.rbf_attn_last_error.restype = ctypes.c_char_p
        lib.rbf_attn_abi_version.argtypes = []
        lib.rbf_attn_abi_version.restype = ctypes.c_int
        ver = lib.rbf_attn_abi_version()
        if ver != ABI_VERSION:
            raise RuntimeError(f"{path}: ABI version {ver}, expected {ABI_VERSION}")
        runtimes = _hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise RuntimeError(f"two HIP runtimes are mapped in this process: {sorted(runtimes)}")
        _lib = lib
        return lib


def tensor_desc(t: torch.Tensor | None) -> Tensor:
    """Descriptor of a (B, H, N, D) tensor.  The stride of a dimension of
    size 1 is never used (its only index is 0) and is passed as 0, so that
    torch's arbitrary strides for such dimensions pass the alignment check."""
    if t is None:
        return Tensor(None, 0, 0, 0)
    s, n = t.stride(), t.shape
    return Tensor(t.data_ptr(), s[0] if n[0] != 1 else 0, s[1] if n[1] != 1 else 0, s[2] if n[2] != 1 else 0)


def pos_desc(pos: torch.Tensor) -> PosTerm:
    """Descriptor of a (1 or B, H, N, D) position term; a batch-1 term is
    passed with stride_b = 0, as the library requires (it reads it at every b)."""
    batch = pos.shape[0]
    return PosTerm(tensor_desc(pos), batch)


def decode_workspace_size(args: DecodeArgs) -> int:
    lib = load()
    n = lib.rbf_attn_decode_workspace_size(ctypes.byref(args))
    if n == 0:
        raise RbfAttnError(-1, lib.rbf_attn_last_error().decode(errors="replace"))
    return int(n)


def call(fn_name: str, args, stream: int, *extra: int) -> None:
    lib = _lib if _lib is not None else load()
    rc = getattr(lib, fn_name)(ctypes.byref(args), ctypes.c_void_p(stream), *extra)
    if rc != 0:
        msg = lib.rbf_attn_last_error().decode(errors="replace")
        raise RbfAttnError(rc, msg)


def pos_supported(args: Args) -> bool:
    """Whether rbf_attn_{fwd,bwd}_pos fuse a position term for these args."""
    rc = load().rbf_attn_pos_supported(ctypes.byref(args))
    if rc < 0:
        raise RbfAttnError(rc, load().rbf_attn_last_error().decode(errors="replace"))
    return rc == 1


def bwd_kernels(args: Args, pos: PosTerm | None = None) -> int:
    """Kernels rbf_attn_bwd (or rbf_attn_bwd_pos with pos) enqueues for args."""
    lib = load()
    rc = lib.rbf_attn_bwd_kernels(ctypes.byref(args), ctypes.byref(pos) if pos is not None else None)
    if rc < 0:
        raise RbfAttnError(rc, lib.rbf_attn_last_error().decode(errors="replace"))
    return rc


def call_pos(fn_name: str, args, pos: PosTerm, stream: int) -> None:
    lib = load()
    rc = getattr(lib, fn_name)(ctypes.byref(args), ctypes.byref(pos), ctypes.c_void_p(stream))
    if rc != 0:
        raise RbfAttnError(rc, lib.rbf_attn_last_error().decode(errors="replace"))
