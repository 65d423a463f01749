"""Build the gfx950 HIP library ``cast_amd/_lib/librcsa.so``.

Every ``csrc/*.hip`` file is compiled to an object with hipcc for gfx950 and
linked into one shared library that exports the C ABI of ``include/rcsa.h``.
Run ``python -m cast_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG / "csrc"
LIBDIR = PKG / "_lib"
LIBNAME = "librcsa.so"
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    if path.exists():
        return str(path)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # keep the compiler from emitting packed-fp32 VALU ops
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
]


# Per-source flags.  The attention kernels are scheduled for instruction-level
# parallelism (interleaved A/B on one MI355X: int8 attention 1.4%, bf16 1.7%,
# the gathered int8 layer call 3.5% faster); the gathered bf16 kernel, 4.5%
# slower that way, sits in a source of its own with the default scheduler, as
# does the int8 kernel of three workgroups per compute unit (15% slower with
# the ILP scheduler).  The bf16 kernels of three workgroups per compute unit
# with gathered sources or validity bytes fit their 168 VGPRs without spills
# only under the memory-clause scheduler.
FILE_FLAGS = {
    "sparse_attn.hip": ["-mllvm", "-amdgpu-sched-strategy=max-ilp"],
    "sparse_attn_bf16_cu3.hip": ["-mllvm", "-amdgpu-sched-strategy=max-memory-clause"],
}


def _compile(src: Path, obj: Path) -> None:
    cmd = [hipcc(), *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []),
           "-Rpass-analysis=kernel-resource-usage", "-c", str(src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    lines = [line for line in res.stderr.splitlines()
             if "packed-fp32-ops" not in line]  # host pass does not know the feature
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n" + "\n".join(lines))
    _check_resources(src, lines)
    other = [line for line in lines if "remark:" not in line and line.strip()
             and not line.lstrip().startswith(("|", "^", "In file included from"))
             and not line.lstrip()[:1].isdigit()]
    if other:
        print("\n".join(other), file=sys.stderr)
    _check_stubs(obj)


def _check_resources(src: Path, lines: list[str]) -> None:
    """Fail if a kernel spills or uses scratch memory: the hot kernels are
    written to live in registers and LDS, and a silent fall-back to scratch
    (e.g. an un-inlined lambda) costs an order of magnitude."""
    kernel = None
    bad = []
    for line in lines:
        if "Function Name:" in line:
            kernel = line.split("Function Name:")[1].split()[0]
        elif "ScratchSize [bytes/lane]:" in line or "VGPRs Spill:" in line:
            val = int(line.split(":")[-1].split()[0])
            if val:
                bad.append(f"{kernel}: {line.split('remark:')[1].split('[')[0].strip()}")
    if bad:
        raise RuntimeError(f"{src.name}: kernels spill or use scratch:\n  " + "\n  ".join(bad))


def _check_stubs(obj: Path) -> None:
    """Fail if the host pass left a kernel launch stub undefined.

    hipcc can drop a template kernel's host stub without any diagnostic
    (the library then links but fails to load with an undefined
    ``__device_stub__`` symbol); catch that at build time.
    """
    nm = shutil.which("nm")
    if nm is None:
        return
    res = subprocess.run([nm, str(obj)], capture_output=True, text=True)
    missing = [line.split()[-1] for line in res.stdout.splitlines()
               if " U " in line and "__device_stub__" in line]
    if missing:
        raise RuntimeError(f"{obj.name}: host pass left kernel stubs undefined: "
                           f"{missing[:4]}{' ...' if len(missing) > 4 else ''}")


def build(verbose: bool = True) -> Path:
    """Compile every kernel source and link ``_lib/librcsa.so``; return its path."""
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir = PKG / "_build"
    objdir.mkdir(exist_ok=True)
    LIBDIR.mkdir(exist_ok=True)
    objs = [objdir / (s.stem + ".o") for s in sources]
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda so: _compile(*so), zip(sources, objs)))
    out = LIBDIR / LIBNAME
    tmp = LIBDIR / (LIBNAME + ".tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    try:
        ext = build_torch_ops()
    except RuntimeError as e:  # the C ABI library stands; only the torch ops are missing
        raise RuntimeError(f"{out} is built (the C ABI is usable through ctypes), but the "
                           f"torch extension {TORCH_OPS} is not:\n{e}") from None
    if verbose:
        print(f"built {out} from {len(sources)} sources and {ext.name}")
    return out


TORCH_OPS = "librcsa_torch.so"


def build_torch_ops() -> Path:
    """Compile ``csrc/torch_ops.cpp`` (the PyTorch-ROCm extension: torch custom
    ops over the C ABI) into ``_lib/librcsa_torch.so`` against this torch."""
    import torch
    import torch.utils.cpp_extension as ce

    src = CSRC / "torch_ops.cpp"
    out = LIBDIR / TORCH_OPS
    tmp = LIBDIR / (TORCH_OPS + ".tmp")
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    libdirs = ce.library_paths()
    cmd = [shutil.which("g++") or "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
           "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
           f"-D_GLIBCXX_USE_CXX11_ABI={int(torch._C._GLIBCXX_USE_CXX11_ABI)}",
           *[f"-I{p}" for p in ce.include_paths()], f"-I{rocm}/include",
           str(src), "-o", str(tmp),
           *[f"-L{p}" for p in libdirs], "-lc10", "-lc10_hip", "-ltorch", "-ltorch_cpu",
           f"-L{rocm}/lib", "-lamdhip64", "-ldl",
           *[f"-Wl,-rpath,{p}" for p in libdirs], f"-Wl,-rpath,{rocm}/lib"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"torch_ops.cpp failed:\n{res.stderr[-4000:]}")
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    build()
