"""Ahead-of-time build of libdeep_gemm_amd.so for gfx950.

Compiles every ``csrc/*.hip`` translation unit with hipcc in parallel and links them into
``deep_gemm/libdeep_gemm_amd.so`` (in-tree, so the library travels with the source tree).
Usage: ``python deepgemm-ascend_amd/build.py [-j N]``.
"""
import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent
CSRC = ROOT / 'csrc'
OUT_DIR = ROOT / '_build'
LIB = ROOT / 'deep_gemm' / 'libdeep_gemm_amd.so'
ARCH = os.environ.get('DG_OFFLOAD_ARCH', 'gfx950')


def hipcc() -> str:
    for cand in (os.environ.get('HIPCC'), '/opt/rocm/bin/hipcc', shutil.which('hipcc')):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError('hipcc not found (set HIPCC)')


COMMON_FLAGS = [
    f'--offload-arch={ARCH}', '-O3', '-std=c++20', '-fPIC',
    # packed fp32 VALU ops are kept off: hipcc must not form v_pk_{add,mul,fma}_f32
    '-Xclang', '-target-feature', '-Xclang', '-packed-fp32-ops',
    '-Wno-unused-command-line-argument', '-Wno-pass-failed',
]


def _compile(src: Path, obj: Path, verbose: bool) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, '-c', str(src), '-o', str(obj)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'hipcc failed for {src.name}:\n{res.stderr[-6000:]}')


def build(jobs: int = 0, verbose: bool = False) -> Path:
    OUT_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob('*.hip'))
    objs = [OUT_DIR / (s.stem + '.o') for s in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 4)))
    with cf.ThreadPoolExecutor(max_workers=jobs) as ex:
        futs = [ex.submit(_compile, s, o, verbose) for s, o in zip(sources, objs)]
        for f in futs:
            f.result()
    tmp = LIB.with_suffix('.so.tmp')
    # -z defs: a kernel whose host stub was silently dropped fails here, not at load time
    cmd = [hipcc(), f'--offload-arch={ARCH}', '-shared', '-fPIC', '-Wl,-z,defs', *map(str, objs), '-lhiprtc', '-o', str(tmp)]
    if verbose:
        print(' '.join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f'link failed:\n{res.stderr[-4000:]}')
    os.replace(tmp, LIB)
    return LIB


EXT_NAME = 'deep_gemm_C'
EXT = ROOT / 'deep_gemm' / f'{EXT_NAME}.so'


def build_ext(verbose: bool = False) -> Path:
    """The C++ host-path extension (csrc/torch_ext.cpp), built with torch's extension builder into
    ``deep_gemm/deep_gemm_C.so``.  It links no HIP code: the Python layer hands it the loaded
    library's entry points."""
    import torch.utils.cpp_extension as ce
    bdir = OUT_DIR / 'ext'
    bdir.mkdir(parents=True, exist_ok=True)
    ce.load(name=EXT_NAME, sources=[str(CSRC / 'torch_ext.cpp')], build_directory=str(bdir),
            extra_cflags=['-O2', '-std=c++17'], extra_include_paths=[str(ROOT.parent / 'include')],
            with_cuda=False, verbose=verbose, is_python_module=True)
    built = bdir / f'{EXT_NAME}.so'
    tmp = EXT.with_suffix('.so.tmp')
    shutil.copyfile(built, tmp)
    os.replace(tmp, EXT)
    return EXT


if __name__ == '__main__':
    ap = argparse.ArgumentParser()
    ap.add_argument('-j', type=int, default=0)
    ap.add_argument('-v', action='store_true')
    args = ap.parse_args()
    print(build(args.j, args.v))
    print(build_ext(args.v))
    sys.exit(0)
