"""Builds the gfx950 device layer in-tree.

    python -m nert_amd.build            # incremental
    python -m nert_amd.build --force    # rebuild everything

Outputs (git-ignored, shipped with the tree to the GPU box):
    nert_amd/lib/libnert_hip.so      C-ABI kernels + runtime + nert::HipDevice()
    nert_amd/lib/libnert_core.so     the NERT host library a seam user links
    nert_amd/lib/libnert_seamrun.so  (nert_amd/host/): Model on HipDevice()

The seam rows compile against NERT's public headers and its header-only form
helpers (include/nert/*.hpp, src/{softmax_form,reduce_axes,axes_form}.hpp of
olibartfast/nert), found under $NERT_REF (default /root/reference); nothing of
NERT is copied into this repository. The oracle side (oracle/Makefile) and the
test harnesses are built by `build_all()`.
"""

from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import subprocess
import sys
from pathlib import Path

ROOT = Path(__file__).resolve().parent.parent
PKG = ROOT / "nert_amd"
CSRC = PKG / "csrc"
OBJ = PKG / "_build" / "obj"
LIB = PKG / "lib"
NERT_REF = Path(os.environ.get("NERT_REF", "/root/reference"))
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# Packed-FP32 instructions are disabled for all device code: hipcc -O3 forms
# them from ordinary float code and some of their forms have been unreliable
# on these boxes. The host pass warns that it does not know the feature.
COMMON_FLAGS = [
    "-std=c++17",
    "-O3",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # MFMA accumulators in ordinary VGPRs: otherwise, in kernels of 256 threads
    # or fewer, the backend keeps them in AGPRs and copies all of them to
    # VGPRs and back on every K-loop iteration (v_accvgpr_read/write, 16 per
    # 32x32 block per iteration); with this form no kernel here gains a spill.
    "-mllvm", "-amdgpu-mfma-vgpr-form=1",
    "-Wall",
    "-Wno-unused-command-line-argument",
    "-Wno-unknown-warning-option",
    "-include", "cstddef",
]


def _sources() -> list[Path]:
    files = sorted(CSRC.glob("*.hip")) + sorted((CSRC / "device").glob("*.cpp"))
    return files


def _headers() -> list[Path]:
    hs = list(CSRC.rglob("*.hpp")) + list((ROOT / "include").glob("*.h")) + list((ROOT / "include").glob("*.hpp"))
    return hs


def _include_flags() -> list[str]:
    inc = NERT_REF / "include"
    src = NERT_REF / "src"
    if not (inc / "nert" / "device.hpp").exists():
        raise RuntimeError(
            f"NERT headers not found under {NERT_REF} (set NERT_REF to a checkout of olibartfast/nert)")
    return [f"-I{inc}", f"-I{src}", f"-I{ROOT / 'include'}"]


def _compile(src: Path, force: bool, newest_header: float) -> Path:
    rel = src.relative_to(CSRC)
    obj = OBJ / rel.with_suffix(".o")
    obj.parent.mkdir(parents=True, exist_ok=True)
    if not force and obj.exists():
        mtime = obj.stat().st_mtime
        if mtime > src.stat().st_mtime and mtime > newest_header:
            return obj
    lang = ["-x", "hip"] if src.suffix == ".hip" else []
    cmd = [HIPCC, *COMMON_FLAGS, *_include_flags(), *lang, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"compile failed: {src}\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
    return obj


def build_device_layer(force: bool = False, jobs: int | None = None) -> Path:
    """Compiles every HIP/C++ source under nert_amd/csrc and links libnert_hip.so."""
    LIB.mkdir(parents=True, exist_ok=True)
    # A change of the compile flags (this file) rebuilds every object too.
    newest_header = max([h.stat().st_mtime for h in _headers()] + [Path(__file__).stat().st_mtime])
    sources = _sources()
    jobs = jobs or min(8, os.cpu_count() or 4)
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(s, force, newest_header), sources))
    out = LIB / "libnert_hip.so"
    newest_obj = max(o.stat().st_mtime for o in objs)
    if force or not out.exists() or out.stat().st_mtime < newest_obj:
        tmp = out.with_suffix(".so.tmp")
        cmd = [HIPCC, "-shared", f"--offload-arch={ARCH}", "-fPIC", "-o", str(tmp), *map(str, objs)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed\n{' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}")
        os.replace(tmp, out)
    return out


def build_oracle(force: bool = False) -> None:
    """Builds oracle/_ref (the reference CPU library and its C shim)."""
    args = ["make", "-C", str(ROOT / "oracle"), "-j8"]
    if force:
        args.insert(1, "-B")
    if not (NERT_REF / "src" / "executor.cpp").exists():
        return  # the reference is absent (GPU box): use the prebuilt oracle/_ref
    subprocess.run(args, check=True, capture_output=True, text=True)


def build_host(force: bool = False) -> None:
    """Builds the NERT host side a seam user links (nert_amd/host/Makefile):
    nert_amd/lib/libnert_core.so and the drop-in C-ABI libnert_seamrun.so."""
    if not (NERT_REF / "src" / "executor.cpp").exists():
        return  # the reference is absent (GPU box): use the prebuilt libraries
    args = ["make", "-C", str(PKG / "host"), "-j8"]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, capture_output=True, text=True)


def build_tests(force: bool = False) -> None:
    """Builds the C++ test harness libraries under tests/_build."""
    mk = ROOT / "tests" / "cpp" / "Makefile"
    if not mk.exists():
        return
    args = ["make", "-C", str(mk.parent), "-j8"]
    if force:
        args.insert(1, "-B")
    subprocess.run(args, check=True, capture_output=True, text=True)


def build_all(force: bool = False) -> None:
    build_device_layer(force=force)
    build_host(force=force)
    build_oracle(force=force)
    build_tests(force=force)


def main(argv: list[str] | None = None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("--only", choices=["device", "host", "oracle", "tests", "all"], default="all")
    a = ap.parse_args(argv)
    try:
        if a.only in ("device", "all"):
            print(build_device_layer(force=a.force))
        if a.only in ("host", "all"):
            build_host(force=a.force)
        if a.only in ("oracle", "all"):
            build_oracle(force=a.force)
        if a.only in ("tests", "all"):
            build_tests(force=a.force)
    except (RuntimeError, subprocess.CalledProcessError) as e:
        msg = str(e)
        if isinstance(e, subprocess.CalledProcessError):
            msg += "\n" + (e.stdout or "") + (e.stderr or "")
        print(msg, file=sys.stderr)
        return 1
    return 0


if __name__ == "__main__":
    sys.exit(main())
