"""bench.py's command line on the CPU: the benchmark measures one GPU and
refuses a several-GPU run before it touches a device."""
import os
import subprocess
import sys

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_bench_refuses_several_gpus():
    r = subprocess.run([sys.executable, os.path.join(ROOT, 'bench.py'), '--gpus', '2'],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 2
    assert 'measures one GPU' in r.stderr
    assert r.stdout.strip() == ''  # no JSON line
