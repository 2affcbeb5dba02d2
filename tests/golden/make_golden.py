"""Write the committed regression fixtures under tests/golden/.

The reference ships no golden vectors (its tests only print), so these
fixtures are produced by this repository's float64 oracle
(oracle/rbf_oracle.py, itself pinned by tests/test_oracle.py) on the seeded
C1 inputs: the first (b, h) slices of benchmark config 1 (fp32, N = 128
content + 4 zero register tokens, D = 64, causal).  They freeze the oracle's
outputs so that a later change to the oracle or to the input generator is
caught (tests/test_golden.py), and give the GPU tests an input/output pair
that does not depend on recomputation.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import rbf_oracle as ro  # noqa: E402
from rbf_attention_amd import workloads as wl  # noqa: E402


def c1_slices():
    w = wl.C1_TINY
    q, k, v, do = (t.numpy() for t in wl.make_inputs(w))
    sl = (slice(0, 1), slice(0, 2))  # b = 0, h = 0..1
    return w, [np.ascontiguousarray(a[sl]) for a in (q, k, v, do)]


def main():
    w, (q, k, v, do) = c1_slices()
    g = w.sm_scale
    O, L = ro.softmax_forward(q, k, v, g)
    dq, dk, dv = ro.softmax_backward(q, k, v, do, g)
    # non-softmax on the same inputs scaled by 0.5 (keeps exp() in range)
    qs, ks, vs, dos = (0.5 * a for a in (q, k, v, do))
    On = ro.non_softmax_forward(qs, ks, vs, g)
    dqn, dkn, dvn = ro.non_softmax_backward(qs, ks, vs, dos, g)
    np.savez_compressed(
        os.path.join(HERE, "c1_slices.npz"),
        gamma=np.float64(g),
        q=q, k=k, v=v, do=do,
        softmax_O=O.astype(np.float32), softmax_L=L.astype(np.float32),
        softmax_dq=dq.astype(np.float32), softmax_dk=dk.astype(np.float32), softmax_dv=dv.astype(np.float32),
        nonsoftmax_O=On.astype(np.float32), nonsoftmax_dq=dqn.astype(np.float32),
        nonsoftmax_dk=dkn.astype(np.float32), nonsoftmax_dv=dvn.astype(np.float32),
    )
    print("wrote", os.path.join(HERE, "c1_slices.npz"))


if __name__ == "__main__":
    main()
