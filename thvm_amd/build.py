"""Build libthvm_hip.so in-tree: C host layer with gcc, gfx950 kernels with
hipcc, linked by hipcc.  Run as ``python -m thvm_amd.build`` or through
``__graft_entry__.build()``.  Always recompiles (the build check) unless
``incremental=True`` (``python -m thvm_amd.build --incremental``): then a
unit is rebuilt when its source, or any header under csrc/ or include/, is
newer than its object."""
from __future__ import annotations

import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OBJ = PKG / "_build"
LIB = PKG / "lib" / "libthvm_hip.so"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

C_SOURCES = ["hip_backend.c", "hip_custom.c", "decoder.c", "render.c", "tune.c", "serve.c", "loader.c"]
# (source, object stem, extra flags): the GEMV kernel instances are one unit
# per (weight type, x type) so the twelve compile in parallel
GEMV_UNITS = [("kernels/gemv_inst.hip", f"gemv_inst_{w}_{x}",
               [f"-DGEMV_WT={w}", f"-DGEMV_XD={x}", f"-DGEMV_PICK=gemv_pick_{w}_{x}"])
              for w in range(4) for x in range(3)] + \
             [("kernels/gemv_inst.hip", f"gemv_inst_{w}_3",   # summed x (norm = 3): bf16 / fp8 weights
               [f"-DGEMV_WT={w}", "-DGEMV_XD=3", f"-DGEMV_PICK=gemv_pick_{w}_3"]) for w in (2, 3)]
HIP_SOURCES = ["kernels/gemv.hip", "kernels/gemm.hip", "kernels/rowops.hip", "kernels/attn.hip",
               "kernels/mla.hip", "kernels/moe.hip", "kernels/step.hip", "kernels/step_m1.hip",
               "kernels/step_m2.hip", "kernels/step_m4.hip"]

CFLAGS = ["-std=c11", "-O2", "-fPIC", "-Wall", "-Wextra", "-Wno-unused-parameter",
          "-fvisibility=hidden", "-D__HIP_PLATFORM_AMD__",
          f"-I{ROCM}/include", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
HIPFLAGS = ["--offload-arch=gfx950", "-O3", "-fPIC", "-std=c++17", "-fvisibility=hidden",
            "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
            "-Wno-unused-command-line-argument",
            f"-I{ROOT / 'include'}", f"-I{CSRC}"]


def _run(cmd: list[str]) -> None:
    r = subprocess.run(cmd, capture_output=True, text=True)
    out = "\n".join(l for l in (r.stdout + r.stderr).splitlines()
                    if "packed-fp32-ops" not in l and "is not a recognized feature" not in l)
    if r.returncode != 0:
        raise RuntimeError(f"build failed: {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def _stale(src: Path, obj: Path, headers_mtime: float) -> bool:
    if not obj.exists():
        return True
    t = obj.stat().st_mtime
    return src.stat().st_mtime > t or headers_mtime > t


VARIANTS = {
    # the measurement build: kernels with the phase-clock marks compiled in
    # (bench.py --phase-clock loads it); the product library has none
    "pclk": ("_build_pclk", "libthvm_hip_pclk.so", ["-DTHVM_PCLK"]),
}


def build(verbose: bool = True, incremental: bool = False, variant: str | None = None) -> Path:
    obj_dir, lib, hipflags = OBJ, LIB, HIPFLAGS
    if variant:
        d, name, extra = VARIANTS[variant]
        obj_dir, lib, hipflags = PKG / d, PKG / "lib" / name, HIPFLAGS + extra
    return _build(obj_dir, lib, hipflags, verbose, incremental)


def _build(OBJ: Path, LIB: Path, HIPFLAGS: list, verbose: bool, incremental: bool) -> Path:
    OBJ.mkdir(exist_ok=True)
    LIB.parent.mkdir(exist_ok=True)
    hdr = max(p.stat().st_mtime for d in (CSRC, ROOT / "include") for p in d.rglob("*.h"))
    jobs = []
    for s in C_SOURCES:
        o = OBJ / (Path(s).stem + ".o")
        if not incremental or _stale(CSRC / s, o, hdr):
            jobs.append(["gcc", *CFLAGS, "-c", str(CSRC / s), "-o", str(o)])
    units = [(s, Path(s).stem, []) for s in HIP_SOURCES] + GEMV_UNITS
    for s, stem, extra in units:
        o = OBJ / (stem + ".hip.o")
        if not incremental or _stale(CSRC / s, o, hdr):
            jobs.append([f"{ROCM}/bin/hipcc", *HIPFLAGS, *extra, "-c", str(CSRC / s), "-o", str(o)])
    jobs.sort(key=lambda j: "gemv_inst" not in " ".join(j))    # the long units first
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "8"))))
    with cf.ThreadPoolExecutor(max_workers=workers) as ex:
        list(ex.map(_run, jobs))
    objs = [str(OBJ / (Path(s).stem + ".o")) for s in C_SOURCES] + \
           [str(OBJ / (stem + ".hip.o")) for _, stem, _ in units]
    tmp = LIB.with_suffix(".so.tmp")
    _run([f"{ROCM}/bin/hipcc", "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *objs,
          f"-L{ROCM}/lib", "-lamdhip64", "-lhiprtc", "-lm", f"-Wl,-rpath,{ROCM}/lib"])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", file=sys.stderr)
    return LIB


if __name__ == "__main__":
    v = sys.argv[sys.argv.index("--variant") + 1] if "--variant" in sys.argv else None
    build(incremental="--incremental" in sys.argv[1:], variant=v)
