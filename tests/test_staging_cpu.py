"""Host-side check of the LDS-DMA staging rule (rbf_attention_amd/csrc/
rbf_attn_staging.h, dma_rows_ok): the header is compiled on its own with g++
into a small driver that evaluates the rule on a table of operands.  Rows
that run backwards, collapse onto one (a tensor expanded along the token
axis: stride 0), overlap, or reach past a 2^31-byte buffer range must take
the register-staged kernels; forward, non-overlapping rows within the range
may take LDS-DMA."""
import os
import shutil
import subprocess

import pytest

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "rbf_attention_amd", "csrc")

DRIVER = r"""
#include <stdio.h>
#include "rbf_attn_staging.h"
int main() {
  long long n, s, d, e;
  while (scanf("%lld %lld %lld %lld", &n, &s, &d, &e) == 4) printf("%d\n", rbf::dma_rows_ok(n, s, d, e) ? 1 : 0);
  return 0;
}
"""

CASES = [
    # (N, stride_n, D, element bytes) -> may stage by LDS-DMA
    ((700, 64, 64, 2), True),  # contiguous rows
    ((2113, 3 * 3 * 128, 128, 2), True),  # token-major packed projection view
    ((700, 0, 64, 2), False),  # expanded along N
    ((2113, 0, 128, 2), False),
    ((700, -64, 64, 2), False),  # rows running backwards
    ((700, 32, 64, 2), False),  # overlapping rows: the last row's tail past N * stride
    ((700, 63, 64, 2), False),
    ((1, 0, 64, 2), False),  # a single row with stride 0: the range would be empty
    (((1 << 24) - 1, 64, 64, 2), True),  # just below 2^31 bytes
    ((1 << 24, 64, 64, 2), False),  # 2^31 bytes: past the 32-bit range field
    ((1 << 23, 128, 128, 2), False),
    ((0, 64, 64, 2), True),  # empty problem (never launched)
]


@pytest.fixture(scope="module")
def driver(tmp_path_factory):
    gxx = shutil.which("g++")
    if gxx is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("staging")
    src = d / "driver.cpp"
    src.write_text(DRIVER)
    exe = d / "driver"
    subprocess.run([gxx, "-std=c++17", "-O1", f"-I{CSRC}", str(src), "-o", str(exe)], check=True)
    return str(exe)


def test_dma_rows_rule(driver):
    inp = "".join(f"{n} {s} {dd} {e}\n" for (n, s, dd, e), _ in CASES)
    out = subprocess.run([driver], input=inp, capture_output=True, text=True, check=True).stdout.split()
    got = [o == "1" for o in out]
    assert got == [want for _, want in CASES], list(zip(CASES, got))


def _functions(src):
    """Launcher source split into (name, body) per `hipError_t name(` definition."""
    import re

    marks = [(m.start(), m.group(1)) for m in re.finditer(r"\nhipError_t (\w+)\(", src)]
    return [(name, src[a : (marks[i + 1][0] if i + 1 < len(marks) else len(src))]) for i, (a, name) in enumerate(marks)]


def test_launchers_use_the_rule():
    """Every LDS-DMA decision of the launchers goes through dma_rows_ok for
    both operands the chosen kernel stages: K and V (forward, dQ), Q and dO
    (dK/dV).  A forward's dO is unset, so it must not be checked there."""
    src = open(os.path.join(CSRC, "rbf_attn_launch.hip")).read()
    body = src[src.index("bool dma_pair_ok("):]
    body = body[: body.index("\n}\n")]
    assert "dma_rows_ok(p.N, stride_a, p.D, esz)" in body and "dma_rows_ok(p.N, stride_b, p.D, esz)" in body
    assert "use_dma_kv(const Params& p, int dp) { return dma_pair_ok(p, dp, p.sk[2], p.sv[2]); }" in src
    assert "use_dma_qdo(const Params& p, int dp) { return dma_pair_ok(p, dp, p.sq[2], p.sdo[2]); }" in src
    assert "use_dma(" not in src
    calls = "\n".join(l for l in src.split("\n") if not l.startswith("bool use_dma_"))  # drop the definitions
    seen = set()
    for name, fn in _functions(calls):
        kv, qdo = "use_dma_kv(" in fn, "use_dma_qdo(" in fn
        if name.startswith(("fwd_", "dq_")):
            assert not qdo, name
            seen.add(name) if kv else None
        elif name.startswith("dkdv_"):
            assert not kv, name
            seen.add(name) if qdo else None
        else:
            assert not (kv or qdo), name
    assert {"fwd_default", "dq_default", "dkdv_default"} <= seen, seen
