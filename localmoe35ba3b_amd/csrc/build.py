"""Builds liblocalmoe35ba3b.so for gfx950 with hipcc.

Each HIP source is compiled to an object in parallel, then linked into one
shared library placed next to the Python package so that it travels with the
source tree.  Run as a script or call build(); both rebuild unconditionally.
"""
import concurrent.futures
import os
import pathlib
import shutil
import subprocess
import sys

CSRC = pathlib.Path(__file__).resolve().parent
PKG = CSRC.parent
INCLUDE = PKG.parent / 'include'
LIB = PKG / 'liblocalmoe35ba3b.so'
SOURCES = sorted(CSRC.glob('*.hip'))
ARCH = os.environ.get('LM_OFFLOAD_ARCH', 'gfx950')

# -ffp-contract=off: the reference epilogues are unfused (enable_fp_fusion=
# False); fused multiply-adds are written explicitly where wanted.
# -packed-fp32-ops disabled: packed fp32 VALU forms are avoided on this target.
COMMON = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', '-ffp-contract=off',
          '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
          '-Wno-unused-command-line-argument']
# Per-source flags.  moe.hip: kernel-argument preloading of each kernel's
# leading scalar arguments (up to 6) into SGPRs at launch; the decode kernels
# take the pointers their first loads need as such arguments.  The compiler
# emits a prologue that loads them normally for firmware without preloading.
# The VGPR form of the MFMA instructions: the prefill router adds each MFMA
# result to an fp32 sum on the VALU, which reads VGPR results directly
# instead of copying them out of AGPRs (the router is moe.hip's only MFMA
# user).  gemm.hip keeps the default flags: its register-streamed GEMMs
# already hold their accumulators in VGPRs, and the same two flags there
# left the prefill unchanged.
EXTRA = {'moe.hip': ['-mllvm', '-amdgpu-kernarg-preload-count=6',
                     '-mllvm', '-amdgpu-mfma-vgpr-form=1']}


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found; the HIP extension cannot be built')
    return path


def _compile(src, obj):
    cmd = [hipcc(), *COMMON, *EXTRA.get(src.name, []), '-I', str(INCLUDE), '-c', str(src), '-o',
           str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature"
    err = '\n'.join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode:
        raise RuntimeError(f'hipcc failed on {src.name}:\n{err}')
    return err


def build(verbose=False):
    out = CSRC / '_build'
    out.mkdir(exist_ok=True)
    objs = [out / (s.stem + '.o') for s in SOURCES]
    workers = min(len(SOURCES), int(os.environ.get('MAX_JOBS', os.cpu_count() or 4)), 8)
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        for msg in pool.map(_compile, SOURCES, objs):
            if msg.strip() and verbose:
                print(msg, file=sys.stderr)
    tmp = LIB.with_suffix('.so.tmp')
    cmd = [hipcc(), '-shared', f'--offload-arch={ARCH}', '-fPIC', *map(str, objs), '-o', str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode:
        raise RuntimeError('link failed:\n' + proc.stderr)
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose=True))
