"""Builds libsvhip.so (all HIP sources under csrc/) for gfx950 with hipcc, in-tree next to this file.

    python -m streamvoxel_amd.build            # or streamvoxel_amd.build.build()
    python -m streamvoxel_amd.build --trace    # also the wave-timeline library (libsvhip_trace.so)
    python -m streamvoxel_amd.build --microbench   # also microbench/xattn_chain (the attention half taken apart)
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
LIB = os.path.join(HERE, 'libsvhip.so')
ARCH = os.environ.get('SVHIP_ARCH', 'gfx950')

SOURCES = ['api.hip', 'entropy.hip', 'select.hip', 'xattn.hip', 'xattn_f32.hip', 'producer.hip', 'norm.hip', 'embed.hip',
           'sample.hip']

FLAGS = [
    '-O3', '-std=c++17', '-fPIC', '-shared', f'--offload-arch={ARCH}',
    # Packed fp32 VALU forms are kept out of the generated code.
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wall', '-Wno-unused-function', '-Wno-unused-variable',
]


def hipcc():
    path = shutil.which('hipcc') or '/opt/rocm/bin/hipcc'
    if not os.path.exists(path):
        raise RuntimeError('hipcc not found; the ROCm toolchain is required to build libsvhip')
    return path


TRACE_LIB = os.path.join(HERE, 'libsvhip_trace.so')


def build_trace(verbose=False):
    """The wave-timeline build of the library (cross attention compiled with -DSVHIP_XATTN_TRACE, every other
    source the product's objects): libsvhip_trace.so, for streamvoxel_amd.xattn_trace only. Needs `build()` first."""
    objdir = os.path.join(HERE, '_build')
    obj = os.path.join(objdir, 'xattn_trace.o')
    cmd = [hipcc(), *[f for f in FLAGS if f != '-shared'], '-DSVHIP_XATTN_TRACE', '-c', os.path.join(CSRC, 'xattn.hip'),
           '-o', obj]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError('hipcc failed (trace build):\n' + res.stdout.decode(errors='replace'))
    objects = [os.path.join(objdir, src.replace('.hip', '.o')) for src in SOURCES if src != 'xattn.hip'] + [obj]
    tmp = TRACE_LIB + '.tmp'
    res = subprocess.run([hipcc(), *FLAGS, *objects, '-o', tmp], stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError('link failed (trace build):\n' + res.stdout.decode(errors='replace'))
    os.replace(tmp, TRACE_LIB)
    return TRACE_LIB


MICROBENCH = os.path.join(HERE, 'microbench', 'xattn_chain')
TR16_PROBE = os.path.join(HERE, 'microbench', 'tr16_probe')


def build_microbench():
    """The standalone programs under microbench/ (no library): xattn_chain.hip, the cross-attention half's
    instructions with its dependencies, one ingredient at a time; tr16_probe.hip, the lane layout of the LDS
    transpose load the kernel reads row-major V with."""
    flags = [f for f in FLAGS if f not in ('-shared', '-fPIC')]
    for prog in (MICROBENCH, TR16_PROBE):
        res = subprocess.run([hipcc(), *flags, prog + '.hip', '-o', prog], stdout=subprocess.PIPE,
                             stderr=subprocess.STDOUT)
        if res.returncode != 0:
            raise RuntimeError('hipcc failed (microbench):\n' + res.stdout.decode(errors='replace'))
    return MICROBENCH


def build(verbose=False, jobs=4):
    """Compile each source to an object in parallel, then link the shared library. Returns the library path."""
    objdir = os.path.join(HERE, '_build')
    os.makedirs(objdir, exist_ok=True)
    procs = []
    objects = []
    for src in SOURCES:
        obj = os.path.join(objdir, src.replace('.hip', '.o'))
        objects.append(obj)
        cmd = [hipcc(), *[f for f in FLAGS if f != '-shared'], '-c', os.path.join(CSRC, src), '-o', obj]
        if verbose:
            print(' '.join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)))
    failed = []
    for src, proc in procs:
        out, _ = proc.communicate()
        text = out.decode(errors='replace')
        text = '\n'.join(line for line in text.splitlines() if 'packed-fp32-ops' not in line)
        if proc.returncode != 0:
            failed.append((src, text))
        elif verbose and text.strip():
            print(text)
    if failed:
        raise RuntimeError('hipcc failed:\n' + '\n'.join(f'--- {s}\n{t}' for s, t in failed))
    tmp = LIB + '.tmp'
    cmd = [hipcc(), *FLAGS, *objects, '-o', tmp]
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT)
    if res.returncode != 0:
        raise RuntimeError('link failed:\n' + res.stdout.decode(errors='replace'))
    os.replace(tmp, LIB)
    return LIB


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
    if '--trace' in sys.argv:
        print(build_trace())
    if '--microbench' in sys.argv:
        print(build_microbench())
