"""Build the gfx950 shared library ``intent_amd/_lib/libintent_amd.so`` with hipcc.

Each ``csrc/*.hip`` translation unit is compiled for gfx950 only and linked
into one shared object with a plain C ABI (declared in ``include/intent_amd.h``).
Usage: ``python -m intent_amd.build`` (or ``build()`` from Python).
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBDIR = PACKAGE / "_lib"
LIBRARY = LIBDIR / "libintent_amd.so"
OBJDIR = PACKAGE.parent / "_build" / "intent_amd"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    # Packed fp32 VALU ops are kept out of generated code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # The first 16 kernarg dwords arrive preloaded in SGPRs: no scalar load
    # round trip before a kernel's first address is known (measured ~0.3 us
    # per launch on the decode GEMV).
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    candidate = Path(rocm) / "bin" / "hipcc"
    if candidate.exists():
        return str(candidate)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found; the gfx950 library cannot be built")
    return found


def _compile(source: Path, objdir: Path = OBJDIR, extra_flags=()) -> Path:
    obj = objdir / (source.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, *extra_flags, "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{proc.stdout}\n{proc.stderr}")
    return obj


def check_objects(objects, workdir: Path) -> None:
    """Run the code-object checks (``codeobj_check``) over the device code of
    every object; every kernel named in ``UNTRACKED_DMA_KERNELS`` must be
    among them, with its LDS DMA, when its source file is."""
    from .codeobj_check import UNTRACKED_DMA_KERNELS, check_binary

    seen = set()
    for obj in objects:
        if not _has_device_code(obj):
            continue
        for rep in check_binary(obj, workdir):
            for k in UNTRACKED_DMA_KERNELS:
                if k in rep.name and rep.dma:
                    seen.add(k)
    if any(Path(o).stem == "moe" for o in objects):
        missing = set(UNTRACKED_DMA_KERNELS) - seen
        if missing:
            raise RuntimeError(f"code-object check: no LDS DMA found in {sorted(missing)}; update UNTRACKED_DMA_KERNELS")


def _has_device_code(obj: Path) -> bool:
    from .codeobj_check import _tool

    proc = subprocess.run([_tool("llvm-readelf"), "-S", str(obj)], capture_output=True, text=True)
    return ".hip_fatbin" in proc.stdout


def build(verbose: bool = False, *, sources=None, extra_flags=(), library: Path = LIBRARY,
          objdir: Path = OBJDIR) -> Path:
    """Compile every HIP source (or ``sources``), check the device code
    (``check_objects``) and link the shared library; returns its path."""
    objdir = Path(objdir)
    library = Path(library)
    objdir.mkdir(parents=True, exist_ok=True)
    library.parent.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip")) if sources is None else [Path(s) for s in sources]
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, objdir, tuple(extra_flags)), sources))
    check_objects(objects, objdir / "codeobj")
    tmp = library.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stdout}\n{proc.stderr}")
    os.replace(tmp, library)
    if verbose:
        print(f"built {library}")
    return library


def build_host_sanitized(out_dir: Path) -> Path:
    """The library with its host code (argument checks, dispatch, launch set-up)
    compiled with AddressSanitizer, into out_dir/libintent_amd.so; the device
    code is built as usual (-Xarch_host keeps the sanitizer off the gfx950
    pass). Loaded under the sanitizer runtime through INTENT_AMD_LIBRARY."""
    out_dir = Path(out_dir)
    out_dir.mkdir(parents=True, exist_ok=True)
    flags = [f for f in HIPCC_FLAGS if f not in ("-O3", "-Wall")] + [
        "-O1", "-Xarch_host", "-fsanitize=address", "-Xarch_host", "-fno-omit-frame-pointer"]

    def one(source: Path) -> Path:
        obj = out_dir / (source.stem + ".o")
        proc = subprocess.run([hipcc(), *flags, "-c", str(source), "-o", str(obj)], capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"hipcc (host ASan) failed for {source.name}:\n{proc.stderr}")
        return obj

    sources = sorted(CSRC.glob("*.hip"))
    with ThreadPoolExecutor(max_workers=min(len(sources), os.cpu_count() or 1)) as pool:
        objects = list(pool.map(one, sources))
    lib = out_dir / "libintent_amd.so"
    proc = subprocess.run([hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-fsanitize=address", "-o", str(lib),
                           *map(str, objects)], capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link (host ASan) failed:\n{proc.stderr}")
    return lib


# Measurement-only builds (INTENT_ABLATE in csrc/mfma_pipe.h): name -> bit mask.
ABLATIONS = {"no_loads": 1, "no_loads_no_lds_writes": 3, "no_epilogue_stores": 4, "fp4_no_decode": 8}
ABLATION_DIR = LIBRARY.parent / "ablation"


def ablation_library(name: str) -> Path:
    return ABLATION_DIR / f"libintent_amd_{name}.so"


def build_ablations(verbose: bool = False) -> list:
    """The libraries `bench.py --probe ablation` times beside the product one (never
    loaded by the package itself)."""
    out = []
    for name, mask in ABLATIONS.items():
        out.append(build(verbose, extra_flags=[f"-DINTENT_ABLATE={mask}"], library=ablation_library(name),
                         objdir=OBJDIR.parent / f"obj_ablate_{name}"))
    return out


if __name__ == "__main__":
    if "--ablations" in sys.argv[1:]:
        build_ablations(verbose=True)
    else:
        build(verbose=True)
    sys.exit(0)
