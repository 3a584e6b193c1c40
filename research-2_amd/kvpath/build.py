"""Build recipe for libkvpath.so: every HIP source under csrc/ compiled for gfx950 and linked
in-tree next to this file (kvpath/libkvpath.so), where `kvpath._lib` loads it; then
libkvpath_torch.so, the torch.ops.kvpath registrations over its C ABI (csrc/kvpath_torch.cpp).

    python research-2_amd/kvpath/build.py     # or via __graft_entry__.build()

The recipe imports nothing of the kvpath package (whose import loads the libraries it builds):
__graft_entry__ loads this file by path, and the ISA scan next to it the same way.

Each source is also compiled to gfx950 assembly with the same flags, and the assembly is scanned
(kvpath.isa_scan) for any instruction that touches a register an inline-asm load may still be
writing; a report refuses the link. (The attention kernels issue loads the compiler does not
track; a register copied or reused before its wait once faulted the GPU.)

hipcc cross-compiles without a GPU, so this runs anywhere ROCm is installed.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE.parent / "csrc"
BUILD_DIR = PACKAGE / "_build"
LIBRARY = PACKAGE / "libkvpath.so"
TORCH_OPS = PACKAGE / "libkvpath_torch.so"
TORCH_OPS_SOURCE = CSRC / "kvpath_torch.cpp"
ARCH = "gfx950"

# Every device compile: packed-fp32 instructions off (hipcc alone may emit them; the host pass
# warns that the feature is unknown to x86, which is harmless), O3, PIC for the shared object.
HIP_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(path).exists():
        raise RuntimeError("hipcc not found: ROCm is required to build libkvpath.so")
    return path


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIP_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {src.name}:\n{proc.stderr}")
    return obj


def assemble(src: Path, out: Path | None = None) -> Path:
    """The gfx950 assembly of one source, with the library's own flags."""
    out = out or BUILD_DIR / (src.stem + ".s")
    cmd = [hipcc(), *HIP_FLAGS, "--cuda-device-only", "-S", str(src), "-o", str(out)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc -S failed on {src.name}:\n{proc.stderr}")
    return out


class IsaHazardError(RuntimeError):
    """The assembly has an instruction that touches an outstanding inline-asm load's register."""


def _isa_scan():
    """kvpath/isa_scan.py, loaded by path (no package import)."""
    import importlib.util

    name = "kvpath_isa_scan"
    if name not in sys.modules:
        spec = importlib.util.spec_from_file_location(name, PACKAGE / "isa_scan.py")
        module = importlib.util.module_from_spec(spec)
        sys.modules[name] = module  # its dataclasses resolve their module through sys.modules
        spec.loader.exec_module(module)
    return sys.modules[name]


def refuse_hazards(assembly: dict[str, str]) -> None:
    """Scan each source's assembly ({name: text}); raise IsaHazardError on any report."""
    isa_scan = _isa_scan()

    found = {}
    for name, text in assembly.items():
        for kernel, reports in isa_scan.scan(text).items():
            if reports:
                found[f"{name}:{kernel}"] = reports
    if found:
        lines = [f"{k}: {len(v)} report(s), first: {v[0]}" for k, v in found.items()]
        raise IsaHazardError("inline-asm load destinations touched before their wait; "
                             "not linking libkvpath.so:\n" + "\n".join(lines))


def build_torch_ops(verbose: bool = False) -> Path:
    """libkvpath_torch.so: the torch.ops.kvpath registrations (csrc/kvpath_torch.cpp), host C++
    against this interpreter's torch headers and libraries, linked to libkvpath.so beside it (its
    rpath is its own directory, so the loader reuses the libkvpath.so ctypes loads)."""
    import torch
    from torch.utils import cpp_extension

    includes = cpp_extension.include_paths()
    if "/opt/rocm/include" not in includes:
        includes.append("/opt/rocm/include")
    libdir = cpp_extension.library_paths()[0]
    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    tmp = TORCH_OPS.with_suffix(".so.tmp")
    cmd = ["g++", "-O2", "-std=c++17", "-fPIC", "-shared", f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
           "-D__HIP_PLATFORM_AMD__", "-DUSE_ROCM", "-Wall", "-Wno-unused-function",
           *[f"-I{d}" for d in includes], str(TORCH_OPS_SOURCE), "-o", str(tmp),
           f"-L{PACKAGE}", "-l:libkvpath.so", f"-L{libdir}", "-lc10", "-lc10_hip", "-ltorch_cpu",
           "-ltorch", "-Wl,-rpath,$ORIGIN", f"-Wl,-rpath,{libdir}"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"build of {TORCH_OPS.name} failed:\n{proc.stderr[-6000:]}")
    os.replace(tmp, TORCH_OPS)
    if verbose:
        print(f"built {TORCH_OPS}", flush=True)
    return TORCH_OPS


def build(verbose: bool = False) -> Path:
    """Compile every csrc/*.hip, scan its assembly, and link libkvpath.so. Always recompiles (it
    is the build check)."""
    BUILD_DIR.mkdir(exist_ok=True)
    srcs = sources()
    assert srcs, f"no HIP sources under {CSRC}"
    workers = min(2 * len(srcs), max(1, (os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(workers) as pool:
        objs_f = [pool.submit(_compile, src) for src in srcs]
        asm_f = [pool.submit(assemble, src) for src in srcs]
        objs = [f.result() for f in objs_f]
        asms = [f.result() for f in asm_f]
    refuse_hazards({path.name: path.read_text() for path in asms})
    if verbose:
        print(f"scanned the assembly of {len(asms)} sources: no outstanding-load hazards",
              flush=True)
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link of libkvpath.so failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY} from {len(srcs)} sources", flush=True)
    build_torch_ops(verbose)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
