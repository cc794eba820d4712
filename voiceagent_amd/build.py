"""Compile the HIP attention kernels and the C ABI into one shared library.

``build_native()`` runs ``hipcc --offload-arch=gfx950`` on every ``csrc/*.hip``
file (in parallel, one object per file) and links them into
``voiceagent_amd/lib/libvoiceagent_attn.so``, the drop-in library.  The
bench-only diagnostics in ``csrc/bench/*.hip`` (include/voiceagent_bench.h)
link into ``voiceagent_amd/lib/libvoiceagent_bench.so``.  ``csrc/host/
fast_calls.cpp``, host C++ with no GPU code, builds with g++ into the
``_fast_calls`` module beside them (the wrappers' fast path).  It always
recompiles; the GPU box loads the libraries built here and never compiles.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sysconfig
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC_DIR = PACKAGE_DIR / "csrc"
LIB_DIR = PACKAGE_DIR / "lib"
INCLUDE_DIR = PACKAGE_DIR.parent / "include"
OBJ_DIR = PACKAGE_DIR / "_build"
LIB_NAME = "libvoiceagent_attn.so"
LIB_PATH = LIB_DIR / LIB_NAME
BENCH_LIB_PATH = LIB_DIR / "libvoiceagent_bench.so"
# Host fast path of ops.paged_decode / ops.varlen_attention (csrc/host/*.cpp,
# plain C++ against torch's headers; no GPU code).
FAST_MODULE = "_fast_calls"
FAST_PATH = LIB_DIR / (FAST_MODULE + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))
OFFLOAD_ARCH = "gfx950"

# Packed-fp32 VALU ops are disabled for every HIP object: ordinary float code
# is compiled to scalar v_fma/v_mul/v_add.
HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-variable",
    "-Wno-unused-function",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


# Per-source extra flags.  The decode translation units keep matrix-core
# accumulators in ordinary VGPRs: the online-softmax rescale of the output
# accumulators is VALU work, and AGPR accumulators would be copied out and
# back on every tile.
EXTRA_FLAGS = {
    "paged_decode_bf16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
    "paged_decode_f16.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=true"],
}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found; the HIP kernels cannot be built")
    return path


def _compile(hipcc: str, src: Path, obj: Path) -> tuple[Path, str]:
    cmd = [hipcc, *HIPCC_FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    log = "\n".join(
        line for line in (proc.stdout + proc.stderr).splitlines() if noise not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{log}")
    return obj, log


def _link(hipcc: str, objects: list[Path], target: Path) -> None:
    tmp = target.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", "-Wl,--no-undefined",
           "-o", str(tmp)]
    cmd += [str(o) for o in objects]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of {target.name} failed:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, target)


def _build_fast_calls() -> None:
    """g++ build of the host fast-path module against torch's C++ headers."""
    from torch.utils import cpp_extension

    src = CSRC_DIR / "host" / "fast_calls.cpp"
    cxx = shutil.which("g++") or "c++"
    abi = int(bool(getattr(__import__("torch")._C, "_GLIBCXX_USE_CXX11_ABI", True)))
    tmp = FAST_PATH.with_suffix(".so.tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-w",
           f"-D_GLIBCXX_USE_CXX11_ABI={abi}", f"-DTORCH_EXTENSION_NAME={FAST_MODULE}",
           "-DTORCH_API_INCLUDE_EXTENSION_H", f"-I{INCLUDE_DIR}"]
    cmd += [f"-I{p}" for p in cpp_extension.include_paths()]
    cmd += [f"-I{sysconfig.get_paths()['include']}", str(src), "-o", str(tmp)]
    cmd += [f"-L{p}" for p in cpp_extension.library_paths()]
    cmd += ["-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed on {src.name}:\n{proc.stdout}{proc.stderr}")
    os.replace(tmp, FAST_PATH)


def build_native(verbose: bool = False) -> Path:
    """Compile every HIP source and link both shared libraries; returns the
    drop-in library's path."""
    hipcc = _hipcc()
    sources = sorted(CSRC_DIR.glob("*.hip"))
    bench_sources = sorted((CSRC_DIR / "bench").glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    every = sources + bench_sources
    jobs = max(1, min(len(every), int(os.environ.get("MAX_JOBS", os.cpu_count() or 4))))
    objects: dict[Path, Path] = {}
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        fast = pool.submit(_build_fast_calls)
        futures = {
            src: pool.submit(_compile, hipcc, src,
                             OBJ_DIR / (("bench_" if src in bench_sources else "") + src.stem + ".o"))
            for src in every
        }
        for src, fut in futures.items():
            obj, log = fut.result()
            objects[src] = obj
            if verbose and log.strip():
                print(log)
        fast.result()
    _link(hipcc, [objects[s] for s in sources], LIB_PATH)
    _link(hipcc, [objects[s] for s in bench_sources], BENCH_LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} and {BENCH_LIB_PATH.name}")
    return LIB_PATH


if __name__ == "__main__":
    build_native(verbose=True)
