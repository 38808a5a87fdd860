"""Compile the HIP extension (gfx950 only) into qwen3_dspark_amd/_build/.

The shared library is built in-tree so that it travels with the source tree;
there is no JIT path and no CPU build of the kernels.
"""
import os
import subprocess
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, 'csrc')
BUILD_DIR = os.path.join(HERE, '_build')
LIB_NAME = 'libdspark_amd.so'
LIB_PATH = os.path.join(BUILD_DIR, LIB_NAME)
# Profiling build of the same sources with per-workgroup phase stamps in the
# draft kernel (DSPARK_TIMELINE); loaded instead of LIB_PATH only when the
# DSPARK_AMD_TIMELINE environment variable is set (bench.py --timeline).
TIMELINE_LIB_PATH = os.path.join(BUILD_DIR, 'libdspark_amd_timeline.so')
SOURCES = ('attn.hip', 'kv.hip', 'layout.hip', 'prologue.hip', 'project.hip', 'sample.hip', 'measure.hip',
           'errors.cpp')
ARCH = 'gfx950'
# Packed FP32 VALU ops are disabled for all device code.
FLAGS = ('--offload-arch=' + ARCH, '-O3', '-std=c++17', '-shared', '-fPIC',
         '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops')


def hipcc():
    path = os.environ.get('HIPCC', '/opt/rocm/bin/hipcc')
    if not os.path.exists(path):
        raise RuntimeError(f'hipcc not found at {path}')
    return path


def build(verbose=False, timeline=False):
    """Compile every source into LIB_PATH (or, with timeline, the profiling
    build into TIMELINE_LIB_PATH), atomically replaced."""
    os.makedirs(BUILD_DIR, exist_ok=True)
    target = TIMELINE_LIB_PATH if timeline else LIB_PATH
    fd, tmp = tempfile.mkstemp(prefix=os.path.basename(target) + '.', suffix='.tmp', dir=BUILD_DIR)
    os.close(fd)
    extra = ['-DDSPARK_TIMELINE'] if timeline else []
    cmd = [hipcc(), *FLAGS, *extra, *(os.path.join(CSRC, s) for s in SOURCES), '-o', tmp]
    try:
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError('hipcc failed:\n' + proc.stderr[-8000:])
        if verbose and proc.stderr:
            print(proc.stderr)
        os.replace(tmp, target)
    finally:
        if os.path.exists(tmp):
            os.unlink(tmp)
    return target


if __name__ == '__main__':
    print(build(verbose=True))
