"""The committed fixtures (tests/golden/c1_slices.npz, written by
tests/golden/make_golden.py) against the seeded input generator and the
oracle.  CPU only."""
import os

import numpy as np
import pytest

from oracle import rbf_oracle as ro
from rbf_attention_amd import workloads as wl

PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "c1_slices.npz")


@pytest.fixture(scope="module")
def gold():
    return np.load(PATH)  # allow_pickle defaults to False


def test_inputs_match_seeded_generator(gold):
    q, k, v, do = (t.numpy()[:1, :2] for t in wl.make_inputs(wl.C1_TINY))
    for name, a in zip(("q", "k", "v", "do"), (q, k, v, do)):
        assert np.array_equal(gold[name], a), name


def test_oracle_reproduces_fixture(gold):
    q, k, v, do, g = gold["q"], gold["k"], gold["v"], gold["do"], float(gold["gamma"])
    O, L = ro.softmax_forward(q, k, v, g)
    grads = ro.softmax_backward(q, k, v, do, g)
    for name, a in zip(("O", "L", "dq", "dk", "dv"), (O, L) + grads):
        np.testing.assert_allclose(a, gold[f"softmax_{name}"], rtol=1e-6, atol=1e-7, err_msg=name)
    qs, ks, vs, dos = (0.5 * a for a in (q, k, v, do))
    On = ro.non_softmax_forward(qs, ks, vs, g)
    gn = ro.non_softmax_backward(qs, ks, vs, dos, g)
    for name, a in zip(("O", "dq", "dk", "dv"), (On,) + gn):
        np.testing.assert_allclose(a, gold[f"nonsoftmax_{name}"], rtol=1e-6, atol=1e-7, err_msg=name)


def test_register_rows_are_zero(gold):
    # the 4 prepended register tokens of q, k, v are zero; row 0 of O is v_0 = 0
    for name in ("q", "k", "v"):
        assert not gold[name][:, :, :4].any()
    assert not gold["softmax_O"][:, :, 0].any()
