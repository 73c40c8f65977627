"""Build the gfx950 shared library libodie_amd.so from odie_amd/csrc/*.hip.

Every translation unit is compiled with hipcc for gfx950 only, with fp contraction off
(fp32 multiply-adds round exactly as written; fused operations are explicit) and with
packed-fp32 instructions disabled.  Objects go to odie_amd/_build/, the library next to
this file so that it travels with the source tree.
"""
from concurrent.futures import ThreadPoolExecutor
import os
from pathlib import Path
import subprocess

PACKAGE = Path(__file__).resolve().parent
SOURCES = PACKAGE / 'csrc'
BUILD = PACKAGE / '_build'
LIBRARY = PACKAGE / 'libodie_amd.so'
ARCH = 'gfx950'

FLAGS = ['--offload-arch=' + ARCH, '-O3', '-std=c++17', '-fPIC', '-ffp-contract=off',
         '-munsafe-fp-atomics', '-fvisibility=hidden',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
         '-I' + str(PACKAGE.parent / 'include')]


# Per-source additions.  mlp.hip: MFMA results in VGPRs, so the layer outputs feed the fp16
# conversions without an AGPR-to-VGPR copy per value.
EXTRA = {'mlp.hip': ['-mllvm', '-amdgpu-mfma-vgpr-form']}


def hipcc():
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    return str(Path(rocm) / 'bin' / 'hipcc')


def _compile(source):
    target = BUILD / (source.stem + '.o')
    command = [hipcc(), *FLAGS, *EXTRA.get(source.name, []), '-c', str(source), '-o', str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError('hipcc failed for %s:\n%s' % (source.name, result.stderr[-6000:]))
    return target


def build(verbose=False):
    """Compile every .hip source (always) and link libodie_amd.so."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(SOURCES.glob('*.hip'))
    jobs = min(len(sources), int(os.environ.get('MAX_JOBS', os.cpu_count() or 4)), 8)
    with ThreadPoolExecutor(max_workers=max(jobs, 1)) as pool:
        objects = list(pool.map(_compile, sources))
    temporary = LIBRARY.with_suffix('.so.tmp')
    command = [hipcc(), '--offload-arch=' + ARCH, '-shared', '-fPIC', *map(str, objects), '-o', str(temporary)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError('link failed:\n' + result.stderr[-6000:])
    os.replace(temporary, LIBRARY)
    if verbose:
        print('built', LIBRARY)
    return LIBRARY


if __name__ == '__main__':
    build(verbose=True)
