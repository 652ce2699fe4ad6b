"""Build recipe for the HIP library ``brainstate_amd/_lib/libbsamd.so`` (gfx950 only).

Run as ``python -m brainstate_amd.build``.  Cross-compiles with hipcc; no GPU needed.
Flags that matter for results:
  * ``-ffp-contract=off`` -- hipcc fuses a*b+c into FMA by default for device code; the
    fused neuron updates must be the exact sequence of rounded operations they spell.
  * ``-Xclang -target-feature -Xclang -packed-fp32-ops`` -- no packed fp32 instructions.
Scheduling only (no effect on results): the persistent runner (network.hip) is built with the
"max-memory-clause" machine scheduler, which keeps its loads together: 1M-neuron COBA-LIF
7.22 -> 7.17 us per step, COBA-HH 9.13 -> 9.09, same rasters, measured alternately on one box
(the default, max-ilp and iterative-ilp schedulers measured 7.22, 7.20 and 7.74).
"""
import os
import shutil
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
LIBDIR = os.path.join(HERE, '_lib')
LIB = os.path.join(LIBDIR, 'libbsamd.so')
SOURCES = ['runtime.hip', 'compact.hip', 'event_sparse.hip', 'event_bucket.hip', 'event_dense.hip',
           'event_dense_packed.hip', 'neuron.hip', 'network.hip', 'delay.hip', 'conn.hip']
ARCH = 'gfx950'


def hipcc():
    for cand in (os.environ.get('HIPCC'), '/opt/rocm/bin/hipcc', shutil.which('hipcc')):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError('hipcc not found (set HIPCC or install ROCm)')


def flags():
    return ['-O3', f'--offload-arch={ARCH}', '-std=c++17', '-fPIC', '-ffp-contract=off',
            '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
            '-Wno-unused-command-line-argument', '-fvisibility=hidden']


# per-source additions to flags()
SOURCE_FLAGS = {'network.hip': ['-mllvm', '-amdgpu-sched-strategy=max-memory-clause']}


def build(verbose=False, jobs=8):
    os.makedirs(LIBDIR, exist_ok=True)
    cc = hipcc()
    objs = []
    procs = []
    for src in SOURCES:
        obj = os.path.join(LIBDIR, src.replace('.hip', '.o'))
        cmd = [cc, *flags(), *SOURCE_FLAGS.get(src, []), '-c', os.path.join(CSRC, src), '-o', obj]
        if verbose:
            print(' '.join(cmd), flush=True)
        procs.append((src, subprocess.Popen(cmd, stdout=subprocess.PIPE,
                                            stderr=subprocess.STDOUT)))
        objs.append(obj)
        if len(procs) >= jobs:
            _wait(procs.pop(0))
    for p in procs:
        _wait(p)
    tmp = LIB + '.tmp'
    cmd = [cc, f'--offload-arch={ARCH}', '-shared', '-fPIC', *objs, '-o', tmp]
    if verbose:
        print(' '.join(cmd), flush=True)
    subprocess.run(cmd, check=True)
    os.replace(tmp, LIB)
    for o in objs:
        os.remove(o)
    return LIB


def _wait(item):
    src, p = item
    out, _ = p.communicate()
    if p.returncode != 0:
        sys.stderr.write(out.decode(errors='replace'))
        raise RuntimeError(f'hipcc failed on {src}')
    text = out.decode(errors='replace').strip()
    if text:
        # hipcc's host pass warns about the device-only packed-fp32 feature: harmless.
        lines = [ln for ln in text.splitlines() if 'packed-fp32-ops' not in ln]
        if lines:
            sys.stderr.write('\n'.join(lines) + '\n')


if __name__ == '__main__':
    print(build(verbose='-v' in sys.argv))
