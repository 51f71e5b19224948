"""Build libkvrepair.so (gfx950 HIP kernels + C ABI) in-tree with hipcc, and the
host-side CPython extensions _kvr_walk (the executor's module-tree walk, C) with
gcc and _kvr_layout (a cache's per-layer K/V layout and addresses, C++ on torch's
tensor headers) with g++.

The library links the HIP runtime by SONAME (libamdhip64.so.7). It must be
loaded after ``import torch`` so that the dynamic linker binds it to the
runtime torch already loaded, and both share streams and device memory.
"""

from __future__ import annotations

import os
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_ROOT.parent
CSRC = PACKAGE_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
OUTPUT = PACKAGE_ROOT / "kv_cache_repair_amd" / "libkvrepair.so"
WALK_SOURCE = CSRC / "kvr_module_walk.c"
WALK_OUTPUT = PACKAGE_ROOT / "kv_cache_repair_amd" / ("_kvr_walk" + sysconfig.get_config_var("EXT_SUFFIX"))
LAYOUT_SOURCE = CSRC / "kvr_tensor_layout.cpp"
LAYOUT_OUTPUT = PACKAGE_ROOT / "kv_cache_repair_amd" / ("_kvr_layout" + sysconfig.get_config_var("EXT_SUFFIX"))
SOURCES = ("kvr_common.hip", "kvr_rotate.hip", "kvr_scatter.hip", "kvr_fresh.hip", "kvr_layer.hip", "kvr_gemm.hip", "kvr_attention.hip", "kvr_decoder.hip", "kvr_writeback.hip", "kvr_inputs.hip", "kvr_scoring.hip")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled: hipcc still vectorises ordinary
# float code into them otherwise.
HIP_FLAGS = (
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
)


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def _defines() -> list[str]:
    """-D options from the environment: KVR_ATTN_SCRATCH_MB sizes the static
    device array of kvr_packed_causal_attention_noalloc (MiB, default 128),
    which every GPU the library's code object loads on holds."""
    mb = os.environ.get("KVR_ATTN_SCRATCH_MB")
    if mb is None:
        return []
    if not mb.isdigit() or not 1 <= int(mb) <= 4096:
        raise ValueError("KVR_ATTN_SCRATCH_MB must be an integer number of MiB in [1, 4096]")
    return [f"-DKVR_ATTN_SCRATCH_MB={int(mb)}"]


def build_walk(verbose: bool = False) -> Path:
    """Compile the _kvr_walk CPython extension (host C, this interpreter's
    headers) next to the package's modules; returns its path."""
    tmp = WALK_OUTPUT.with_name(WALK_OUTPUT.name + ".tmp")
    cmd = [os.environ.get("CC", "gcc"), "-O2", "-shared", "-fPIC", "-Wall", "-Werror",
           f"-I{sysconfig.get_paths()['include']}", str(WALK_SOURCE), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    result = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError("gcc failed for _kvr_walk:\n" + result.stdout)
    os.replace(tmp, WALK_OUTPUT)
    return WALK_OUTPUT


def build_layout(verbose: bool = False) -> subprocess.Popen:
    """Start compiling the _kvr_layout extension (C++ against the installed
    torch's headers and libraries, its C++ ABI); returns the running compiler,
    whose output replaces LAYOUT_OUTPUT once finish_layout() sees it succeed."""
    import torch

    root = Path(torch.__file__).resolve().parent
    lib = root / "lib"
    cmd = [os.environ.get("CXX", "g++"), "-O2", "-shared", "-fPIC", "-std=c++17", "-Wall", "-Werror",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           f"-I{root / 'include'}", f"-I{root / 'include' / 'torch' / 'csrc' / 'api' / 'include'}",
           f"-I{sysconfig.get_paths()['include']}", str(LAYOUT_SOURCE),
           "-o", str(LAYOUT_OUTPUT.with_name(LAYOUT_OUTPUT.name + ".tmp")),
           f"-L{lib}", "-lc10", "-ltorch_cpu", "-ltorch_python", f"-Wl,-rpath,{lib}"]
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)


def finish_layout(proc: subprocess.Popen) -> Path:
    out, _ = proc.communicate()
    if proc.returncode != 0:
        raise RuntimeError("g++ failed for _kvr_layout:\n" + out)
    os.replace(LAYOUT_OUTPUT.with_name(LAYOUT_OUTPUT.name + ".tmp"), LAYOUT_OUTPUT)
    return LAYOUT_OUTPUT


def build(verbose: bool = False, jobs: int = 4) -> Path:
    """Compile the host extensions and every HIP source and link the shared
    library; returns the library's path."""
    build_walk(verbose)
    layout = build_layout(verbose)  # compiles while the HIP sources do
    build_dir = PACKAGE_ROOT / "_build"
    defines = _defines()
    build_dir.mkdir(exist_ok=True)
    objects, procs = [], []
    for name in SOURCES:
        obj = build_dir / (Path(name).stem + ".o")
        cmd = [hipcc(), *HIP_FLAGS, *defines, f"-I{INCLUDE}", f"-I{CSRC}", "-c", str(CSRC / name), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((name, subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)))
        objects.append(obj)
        while len([p for _, p in procs if p.poll() is None]) >= jobs:
            procs[0][1].wait()
    failed = []
    for name, proc in procs:
        out, _ = proc.communicate()
        out = "\n".join(line for line in (out or "").splitlines() if "packed-fp32-ops" not in line)
        if proc.returncode != 0:
            failed.append((name, out))
        elif verbose and out.strip():
            print(out)
    if failed:
        raise RuntimeError("hipcc failed:\n" + "\n".join(f"--- {n}\n{o}" for n, o in failed))
    tmp = OUTPUT.with_suffix(".so.tmp")
    link = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    if verbose:
        print(" ".join(link), flush=True)
    result = subprocess.run(link, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    if result.returncode != 0:
        raise RuntimeError("hipcc link failed:\n" + result.stdout)
    os.replace(tmp, OUTPUT)
    finish_layout(layout)
    return OUTPUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
