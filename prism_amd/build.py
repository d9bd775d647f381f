"""Build libprism_kv.so (the gfx950 HIP kernels behind include/prism_kv.h) in-tree.

Usage: python -m prism_amd.build   (or prism_amd.build.build() from Python).

Every .hip file under prism_amd/csrc is compiled by hipcc for gfx950 into one object each (in
parallel), then linked into prism_amd/libprism_kv.so.  The .so is what the ctypes loader
(prism_amd/_lib.py) opens; it is git-ignored but travels with the source tree to a GPU host.
Two more libraries come out of the same run: libpkv_probe.so (the streaming-read probe of
bench.py --workload peak) and libprism_kv_stamps.so (the kernels with decode_lean_kernel's
timeline stamps, for bench.py --workload tile-stamps).
"""
from __future__ import annotations

import concurrent.futures as cf
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libprism_kv.so"
LIB_PATH = PKG_DIR / LIB_NAME
PROBE_LIB_PATH = PKG_DIR / "libpkv_probe.so"
# the same library with decode_lean_kernel's timeline stamps (-DPKV_TILE_STAMPS): only
# bench.py --workload tile-stamps loads it
STAMPS_LIB_PATH = PKG_DIR / "libprism_kv_stamps.so"
STAMPS_SOURCE = "pkv_attention.hip"
BUILD_DIR = PKG_DIR / "_build"
ARCH = "gfx950"

# -packed-fp32-ops off: hipcc must not emit packed FP32 arithmetic (v_pk_fma_f32 and friends)
# from ordinary float code; the host pass prints a harmless "not a recognized feature" warning.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # keep MFMA accumulators in ordinary VGPRs: the online-softmax rescale touches them from
    # VALU code, and AGPR homes cost a copy back after every tile (and an occupancy step)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    # start every loop on a 64-byte instruction-cache line: the speculative-verify decode loop
    # (about 2.7 KB of code per tile) ran 68.8 us per config-5 call when an unrelated prologue
    # edit happened to move it off that alignment and 65.6 us on it; prefill and decode are
    # unchanged or a little faster
    "-falign-loops=64",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: cannot build libprism_kv.so")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "is not a recognized feature for this target" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = False, extra_flags: list[str] | None = None) -> Path:
    """Compile every csrc/*.hip for gfx950 and link libprism_kv.so.  Always rebuilds.

    extra_flags (or the whitespace-separated PKV_HIPCC_FLAGS environment variable) are appended
    to every compile, e.g. -DPKV_DECODE_DEPTH=1 to build a tuning variant."""
    hipcc = _hipcc()
    extra = list(extra_flags or []) + os.environ.get("PKV_HIPCC_FLAGS", "").split()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objs = [BUILD_DIR / (s.stem + ".o") for s in sources]
    cmds = [[hipcc, *HIPCC_FLAGS, *extra, "-c", str(s), "-o", str(o)] for s, o in zip(sources, objs)]
    stamps_obj = BUILD_DIR / (Path(STAMPS_SOURCE).stem + "_stamps.o")
    cmds.insert(1, [hipcc, *HIPCC_FLAGS, *extra, "-DPKV_TILE_STAMPS", "-c", str(CSRC / STAMPS_SOURCE), "-o",
                    str(stamps_obj)])
    workers = min(len(cmds), max(1, (os.cpu_count() or 2) // 2), 8)
    with cf.ThreadPoolExecutor(workers) as ex:
        for cmd, fut in zip(cmds, [ex.submit(_run, c) for c in cmds]):
            if verbose:
                print(" ".join(cmd))
            fut.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH}")
    stamps_objs = [stamps_obj if o.name == Path(STAMPS_SOURCE).stem + ".o" else o for o in objs]
    tmp = STAMPS_LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, stamps_objs)])
    os.replace(tmp, STAMPS_LIB_PATH)
    if verbose:
        print(f"built {STAMPS_LIB_PATH}")
    # the bandwidth probe bench.py --workload peak runs: its own library, outside the paged-KV ABI
    probe_src = PKG_DIR / "csrc_probe" / "pkv_probe.hip"
    probe_tmp = PROBE_LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, *HIPCC_FLAGS, *extra, "-shared", "-o", str(probe_tmp), str(probe_src)])
    os.replace(probe_tmp, PROBE_LIB_PATH)
    if verbose:
        print(f"built {PROBE_LIB_PATH}")
    return LIB_PATH


if __name__ == "__main__":
    build(verbose=True)
