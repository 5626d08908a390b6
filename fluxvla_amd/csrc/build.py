"""Compile the gfx950 kernels into fluxvla_amd/libfluxvla_amd.so.

Each ``*.hip`` source becomes one object (built in parallel), then hipcc links
the shared library in-tree so it travels with the repository snapshot.

    python -m fluxvla_amd.csrc.build            # or build() from Python
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.dirname(HERE)
OUT = os.path.join(PKG, 'libfluxvla_amd.so')
OBJ_DIR = os.path.join(HERE, '_build')
SOURCES = ['norm.hip', 'gemm.hip', 'attention.hip', 'misc.hip', 'preprocess.hip',
           'backward.hip']
ARCH = 'gfx950'

HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
FLAGS = [
    f'--offload-arch={ARCH}',
    '-O3',
    '-fPIC',
    '-std=c++17',
    # packed fp32 VALU ops stay off: hipcc emits no v_pk_*_f32 then.
    '-Xclang',
    '-target-feature',
    '-Xclang',
    '-packed-fp32-ops',
    '-Wno-unused-command-line-argument',
]


def _compile(src):
    obj = os.path.join(OBJ_DIR, src.replace('.hip', '.o'))
    cmd = [HIPCC, *FLAGS, '-c', os.path.join(HERE, src), '-o', obj]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src}:\n{res.stderr}')
    return obj


def build(verbose=False):
    """Compile every source and link the library.  Returns its path."""
    os.makedirs(OBJ_DIR, exist_ok=True)
    workers = min(len(SOURCES), int(os.environ.get('MAX_JOBS', '8')))
    with concurrent.futures.ThreadPoolExecutor(workers) as ex:
        objs = list(ex.map(_compile, SOURCES))
    tmp = OUT + '.tmp'
    cmd = [HIPCC, f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs, '-o',
           tmp]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr}')
    os.replace(tmp, OUT)
    if verbose:
        print(f'built {OUT}')
    return OUT


if __name__ == '__main__':
    build(verbose=True)
    sys.exit(0)
