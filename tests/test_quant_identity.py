"""Exhaustive pin of the fp16 quotient identity that the fused rotation +
int4 quantizer kernel uses instead of a per-element division: for every
positive finite fp16 scale s and every finite fp16 x, the int4 code of
fp16(x * fl32(1/s)) equals the code of the correctly rounded fp16(x / s)
(the reference's __hdiv + __half2int_rn, signrot/kernels/fused.cu:100-104),
and the fp16 quotients themselves agree wherever |x / s| >= 2^-14.

The check is a C program (tests/c/quot_exact.c) over all 1.0e9 (s, x)
pairs; it also self-checks its fp16 converter (exact on every fp16 value,
ties to even at every midpoint)."""
import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


@pytest.mark.timeout(600)
def test_quotient_identity_exhaustive(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    exe = tmp_path / "quot_exact"
    subprocess.run([cc, "-O2", "-fopenmp", "-o", str(exe),
                    os.path.join(HERE, "c", "quot_exact.c"), "-lm"], check=True)
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))
    res = subprocess.run([str(exe)], capture_output=True, text=True, env=env, timeout=600)
    bad, checked = res.stdout.split()[-2:]
    assert res.returncode == 0, res.stdout
    assert int(bad) == 0
    assert int(checked) == 0x7BFF * 0x7C00
