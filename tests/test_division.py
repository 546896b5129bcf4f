"""The kernels' division by a per-row divisor (kk_div / kk_div4 in
csrc/kk_internal.h: a correctly rounded reciprocal, a product and an FMA
correction) is bit-identical to IEEE division over the range they use it in
-- checked here on the CPU with the same operations in C (fmaf is the fused
multiply-add v_fma_f32 computes), exhaustively over every mantissa for four
divisors and on four million random pairs.  Dropping the guard on tiny
dividends must break it (their remainder underflows): the check can fail."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.fixture(scope="module")
def div_check(tmp_path_factory):
    cc = shutil.which("gcc") or shutil.which("cc")
    if not cc:
        pytest.skip("no C compiler")
    exe = str(tmp_path_factory.mktemp("div") / "div_check")
    subprocess.run([cc, "-O2", "-ffp-contract=off", os.path.join(HERE, "div_check.c"), "-o", exe,
                    "-lm"], check=True)
    return exe


def _run(exe, guard):
    out = subprocess.run([exe, str(guard)], check=True, capture_output=True, text=True).stdout
    fields = dict(kv.split("=") for kv in out.split())
    return int(fields["n"]), int(fields["bad"])


def test_reciprocal_fma_division_is_ieee(div_check):
    n, bad = _run(div_check, 1)
    assert n > 30_000_000 and bad == 0, (n, bad)


def test_tiny_dividends_need_the_division(div_check):
    n, bad = _run(div_check, 0)
    assert bad > 0, "without the lower bound on |a| the identity must fail somewhere"
