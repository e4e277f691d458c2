"""Shared pytest setup: the `gpu` marker, device fixture and tolerance helpers.

Tolerance used by every floating-point comparison (stated once here):
  norm-wise   ||a - b||_2 <= tol * ||b||_2
  elementwise |a - b| <= tol * |b| + tol * rms(b)   (rms(b) is the atol floor)
with tol = 2e-2 for bf16 outputs and 1e-3 for fp32 outputs.  Integer, index
and routing results are compared bit for bit.
"""
import pathlib
import sys

import numpy as np
import pytest
import torch

ROOT = pathlib.Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

BF16_TOL = 2e-2
FP32_TOL = 1e-3


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: runs HIP kernels on an MI355X (gfx950)')


@pytest.fixture(scope='session')
def dev():
    if not torch.cuda.is_available():
        pytest.skip('no HIP device')
    return torch.device('cuda:0')


def assert_close(a, b, tol=BF16_TOL, what=''):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    diff = np.abs(a - b)
    nb = np.linalg.norm(b)
    rel = np.linalg.norm(a - b) / max(nb, 1e-30)
    rms = nb / np.sqrt(max(b.size, 1))
    bad = diff > tol * np.abs(b) + tol * rms
    assert rel <= tol, f'{what}: norm-wise relative error {rel:.3e} > {tol}'
    assert not bad.any(), (f'{what}: {int(bad.sum())} elements outside tolerance, '
                           f'max diff {diff.max():.3e}')


def seeded(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g
