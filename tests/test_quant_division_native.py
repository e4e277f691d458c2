"""Exhaustive host check of the kernels' quantization division (CPU, no GPU).

The HIP kernels quantize W8A8 activations (w8a8.py:8-14) with one correctly
rounded division r = 1 / s per 128-group and, per element, y = x * r followed
by Markstein's fused correction (quant_div in csrc/common.hpp).
tests/native/test_quant_division.c checks for every finite bf16 and fp16
group absmax a and every x of the same type with |x| <= a that rint of that
quotient equals rint of the correctly rounded x / s, i.e. that the int8
values are the ones a plain division gives.
"""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SRC = ROOT / 'tests' / 'native' / 'test_quant_division.c'


def test_one_division_per_group_quantizes_like_division(tmp_path):
    cc = shutil.which('gcc') or shutil.which('cc')
    if cc is None:
        pytest.skip('no C compiler')
    exe = tmp_path / 'test_quant_division'
    base = [cc, '-O2', '-ffp-contract=off', str(SRC), '-lm', '-o', str(exe)]
    build = subprocess.run(base[:3] + ['-fopenmp'] + base[3:], capture_output=True, text=True)
    if build.returncode != 0:  # no OpenMP: the same check on one thread
        build = subprocess.run(base, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=600)
    assert run.returncode == 0, run.stdout + run.stderr
    assert 'division ok' in run.stdout
    assert 'fp16: 1007713280 pairs, 0 mismatches' in run.stdout
