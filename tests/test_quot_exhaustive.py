"""The vector quantizers encode a corrected reciprocal quotient instead of
the IEEE quotient x / scale (dsl_tool_amd/csrc/common.h, quot).  This runs
tests/quot_exhaustive.c, which shows over every bf16 input and every scale
the quantizers produce that both give the same E4M3 / E2M1 code."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.skipif(shutil.which("gcc") is None, reason="needs gcc")
def test_corrected_quotient_codes_match_ieee_quotient(tmp_path):
    exe = tmp_path / "quot_exhaustive"
    subprocess.run(["gcc", "-O2", "-fopenmp", "-ffp-contract=off",
                    os.path.join(HERE, "quot_exhaustive.c"), "-o", str(exe), "-lm"],
                   check=True, capture_output=True, text=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=900)
    print(res.stdout)
    assert res.returncode == 0, res.stdout + res.stderr
    lines = res.stdout.strip().splitlines()
    assert len(lines) == 4 and all(l.rstrip().endswith(" 0 mismatches") for l in lines)
