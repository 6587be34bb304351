"""Kernel 1's division route (r = RN(1/s) and one fma correction, then the hardware E4M3FN
conversion) gives the reference's codes: an exhaustive CPU walk over every BF16 max-abs in
the kernel's fast range and every BF16 value under it, in both scale modes
(tests/native/quotient_check.c, against the oracle's integer encoder)."""
from __future__ import annotations

import os
import re
import shutil
import subprocess

import pytest

from conftest import ROOT


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    cc = shutil.which("gcc")
    if cc is None:
        pytest.skip("gcc not found")
    exe = tmp_path_factory.mktemp("qc") / "quotient_check"
    src = [str(ROOT / "tests" / "native" / "quotient_check.c"), str(ROOT / "oracle" / "fp8_e4m3.c")]
    base = [cc, "-O2", "-ffp-contract=off", "-fopenmp", "-o", str(exe), *src, "-lm"]
    res = subprocess.run(base[:1] + ["-march=native"] + base[1:], capture_output=True, text=True)
    if res.returncode != 0:  # no -march=native: glibc's fmaf is correctly rounded too, only slower
        res = subprocess.run(base, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr
    return exe


def test_every_pair_gives_the_reference_code(checker):
    env = dict(os.environ, OMP_NUM_THREADS=str(min(8, os.cpu_count() or 1)))
    res = subprocess.run([str(checker)], capture_output=True, text=True, timeout=600, env=env)
    print(res.stdout)
    m = re.search(r"pairs (\d+) code_diff (\d+) q_diff (\d+) q_diff_at_or_above_2\^-10 (\d+)", res.stdout)
    assert m, res.stdout + res.stderr
    pairs, code_diff, q_diff, big = map(int, m.groups())
    assert pairs == 991_845_890           # both modes: sum over the fast max-abs range of (#x <= m)
    assert code_diff == 0 and big == 0
    assert res.returncode == 0
    # the fp32 quotients do differ (below 2^-10, where every code is 0): the check has teeth
    assert q_diff > 0
