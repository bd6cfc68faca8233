"""The bf16 quantiser's division-free code rule (quant_snap8 in
compact_amd/csrc/glu_math.h) equals rint(fp32(v / safe)), the reference's
code before the clamp (src/flashffn.py:1081-1083), for every bf16 value and
every fp16 scale, with the reciprocal up to 2 ulp off: an exhaustive check in
C (tests/quant_snap_check.c), compiled here with gcc.  A rule with the grid
constant one binade too coarse (4096 + 2048 = 6144: multiples of 2^-11) must
fail the same check, so the check can tell."""

import os
import shutil
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def _build(tmp_path, defines=()):
    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("gcc not found")
    exe = str(tmp_path / "quant_snap_check")
    src = os.path.join(HERE, "quant_snap_check.c")
    cmd = [gcc, "-O2", "-mfma", "-ffp-contract=off", "-fno-fast-math", *defines, src, "-o",
           exe, "-lm"]
    subprocess.run(cmd, check=True, capture_output=True, text=True)
    return exe


def test_snap_rule_exhaustive(tmp_path):
    exe = _build(tmp_path)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.startswith("ok "), r.stdout
    assert int(r.stdout.split()[1]) > 10 ** 8


def test_snap_rule_check_rejects_a_coarser_grid(tmp_path):
    exe = _build(tmp_path, ["-DCPT_SNAP_GRID=6144.0f"])
    r = subprocess.run([exe], capture_output=True, text=True, timeout=300)
    assert r.returncode == 1, r.stdout + r.stderr
    assert "FAIL" in r.stdout
