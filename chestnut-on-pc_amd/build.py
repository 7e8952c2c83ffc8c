"""Builds chestnut/libchestnut.so from csrc/ with hipcc for gfx950.

    python chestnut-on-pc_amd/build.py [-j N]

Objects go to chestnut-on-pc_amd/_build/ (git-ignored); the shared library
is written in-tree next to the Python package so it travels with the
repository snapshot.  Always recompiles (no timestamp cache).
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
BUILD = os.path.join(HERE, '_build')
LIB = os.path.join(HERE, 'chestnut', 'libchestnut.so')
HIPCC = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
ARCH = 'gfx950'

COMMON = ['-O3', '-std=c++17', '-fPIC', f'--offload-arch={ARCH}', '-Wall', '-Wno-unused-function',
          '-Wno-unused-variable']
# Packed-FP32 VALU ops are disabled for all device code.
DEVICE_ONLY = ['-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops']


def sources():
    return sorted(f for f in os.listdir(CSRC) if f.endswith(('.hip', '.cpp')))


def compile_one(src):
    obj = os.path.join(BUILD, src + '.o')
    cmd = [HIPCC] + COMMON + DEVICE_ONLY + ['-c', os.path.join(CSRC, src), '-o', obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    noise = "'-packed-fp32-ops' is not a recognized feature for this target (ignoring feature)"
    msg = '\n'.join(l for l in (r.stdout + r.stderr).splitlines() if noise not in l)
    return src, r.returncode, msg, obj


def build(jobs=8, verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    srcs = sources()
    with ThreadPoolExecutor(max_workers=max(1, jobs)) as ex:
        results = list(ex.map(compile_one, srcs))
    failed = [(s, m) for s, rc, m, _ in results if rc != 0]
    for s, rc, m, _ in results:
        if m.strip() and (verbose or rc != 0):
            print(f'--- {s}\n{m}', file=sys.stderr)
    if failed:
        raise RuntimeError('hipcc failed for: ' + ', '.join(s for s, _ in failed))
    tmp = LIB + '.tmp'
    cmd = [HIPCC, '-shared', '-fPIC', f'--offload-arch={ARCH}', '-o', tmp] + [o for _, _, _, o in results]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('link failed:\n' + r.stdout + r.stderr)
    os.replace(tmp, LIB)
    return LIB


VENDOR = os.path.join(HERE, 'vendor_compare')


def build_vendor_compare():
    """The config-1 comparison against hipBLASLt (vendor_compare/), linked
    against the built library; run it from anywhere."""
    src = os.path.join(VENDOR, 'config1_hipblaslt.cpp')
    exe = os.path.join(VENDOR, 'config1_hipblaslt')
    inc = os.path.join(os.path.dirname(HERE), 'include')
    libdir = os.path.dirname(LIB)
    cmd = [HIPCC] + COMMON + DEVICE_ONLY + ['-I', inc, src, '-o', exe, '-L', libdir, '-lchestnut', '-lhipblaslt',
                                            f'-Wl,-rpath,{libdir}', "-Wl,-rpath,$ORIGIN/../chestnut"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError('vendor comparison build failed:\n' + r.stdout + r.stderr)
    return exe


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('-j', type=int, default=8)
    ap.add_argument('-v', action='store_true')
    ap.add_argument('--vendor-compare', action='store_true',
                    help='also build vendor_compare/config1_hipblaslt (needs the library built first)')
    a = ap.parse_args()
    print(build(a.j, a.v))
    if a.vendor_compare:
        print(build_vendor_compare())
