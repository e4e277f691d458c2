"""Host-compiled bounds test of the kernels' index guards (CPU, no GPU).

tests/native/test_bounds.cpp includes localmoe35ba3b_amd/csrc/bounds.hpp -
the header the HIP kernels use to clamp expert ids, route positions and
tile-table rows before they form addresses - builds it with g++ under
AddressSanitizer and UndefinedBehaviorSanitizer, and feeds every guard
garbage (NaN / infinite / signed-zero / denormal logits, duplicated and
out-of-range ids, unwritten workspace words, malformed tile rows), checking
each resulting address against the buffer it indexes.
"""
import pathlib
import shutil
import subprocess

import pytest

ROOT = pathlib.Path(__file__).resolve().parents[1]
SRC = ROOT / 'tests' / 'native' / 'test_bounds.cpp'
CSRC = ROOT / 'localmoe35ba3b_amd' / 'csrc'


def test_index_guards_keep_every_address_in_bounds(tmp_path):
    gxx = shutil.which('g++')
    if gxx is None:
        pytest.skip('g++ not available')
    exe = tmp_path / 'test_bounds'
    cmd = [gxx, '-std=c++17', '-O1', '-g', '-fsanitize=address,undefined',
           '-fno-sanitize-recover=all', '-I', str(CSRC), str(SRC), '-o', str(exe)]
    build = subprocess.run(cmd, capture_output=True, text=True)
    assert build.returncode == 0, build.stderr
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=300)
    assert run.returncode == 0, run.stdout + run.stderr
    assert 'bounds ok' in run.stdout
