"""Build libqwen_hip.so for gfx950 from csrc/*.hip.

Each translation unit is compiled by hipcc in parallel into _build/, then linked
into qwen_triton/_lib/libqwen_hip.so (in-tree, so it travels with the source
snapshot to the GPU box). Usage:

    python qwen-triton_amd/build.py [--force] [--jobs N]
"""
from __future__ import annotations

import argparse
import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PKG_ROOT / "_build"
LIB_DIR = PKG_ROOT / "qwen_triton" / "_lib"
LIB_PATH = LIB_DIR / "libqwen_hip.so"

ARCH = "gfx950"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    # Never emit packed-FP32 VALU ops (v_pk_{add,mul,fma}_f32) on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-result",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-file additions. Attention keeps its MFMA accumulators in VGPRs (with no
# AGPR copies around the online-softmax rescale, the forward fits two waves per
# SIMD) and assumes NaN-free scores, so max() needs no NaN canonicalisation.
FILE_FLAGS = {
    "qh_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form", "-fno-honor-nans"],
}


def _sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def _headers() -> list[Path]:
    return sorted(CSRC.glob("*.h")) + sorted(INCLUDE.glob("*.h"))


def _compile(src: Path, force: bool) -> tuple[Path, str]:
    obj = BUILD_DIR / (src.stem + ".o")
    newest_dep = max([src.stat().st_mtime, Path(__file__).stat().st_mtime] + [h.stat().st_mtime for h in _headers()])
    if not force and obj.exists() and obj.stat().st_mtime >= newest_dep:
        return obj, ""
    cmd = [HIPCC, *COMMON_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")
    # hipcc's host pass warns about the device-only target feature; drop that noise.
    noise = "is not a recognized feature for this target"
    msgs = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    return obj, msgs


def build(force: bool = False, jobs: int | None = None, verbose: bool = False) -> Path:
    if shutil.which(HIPCC) is None and not Path(HIPCC).exists():
        raise RuntimeError(f"hipcc not found at {HIPCC}")
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    srcs = _sources()
    jobs = jobs or min(len(srcs), max(1, min(16, os.cpu_count() or 4)))
    objs: list[Path] = []
    with cf.ThreadPoolExecutor(max_workers=jobs) as pool:
        futs = {pool.submit(_compile, s, force): s for s in srcs}
        for fut in cf.as_completed(futs):
            obj, msgs = fut.result()
            objs.append(obj)
            if verbose and msgs:
                print(msgs, file=sys.stderr)
    objs.sort()
    relink = force or not LIB_PATH.exists() or any(o.stat().st_mtime > LIB_PATH.stat().st_mtime for o in objs)
    if relink:
        tmp = LIB_PATH.with_suffix(".so.tmp")
        cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr}")
        os.replace(tmp, LIB_PATH)
    return LIB_PATH


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--force", action="store_true")
    ap.add_argument("--jobs", type=int, default=None)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    path = build(force=args.force, jobs=args.jobs, verbose=args.verbose)
    print(path)


if __name__ == "__main__":
    main()
