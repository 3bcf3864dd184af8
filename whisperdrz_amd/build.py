"""Build libwdrz_attn.so in-tree with hipcc for gfx950.

Usage: python -m whisperdrz_amd.build [--debug]

The library is a plain shared object (no torch / pybind dependency); the Python side loads it
with ctypes. Every build also links libwdrz_attn_debug.so: the same kernel objects with the C-ABI
layer compiled with WDRZ_DEBUG_CHECKS, which copies the device metadata of a call (slot ids,
cache lengths) to the host and rejects out-of-range rows before launching (synchronous, so not
for graph capture; selected with WDRZ_DEBUG=1). ``--debug`` compiles everything with -O1 -g, for
host-side debugging.
"""
from __future__ import annotations

import hashlib
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libwdrz_attn.so"
LIB_PATH = PKG_DIR / LIB_NAME
DEBUG_LIB_PATH = PKG_DIR / "libwdrz_attn_debug.so"
SOURCES = ["attn_kvcache.hip", "attn_dense.hip", "attn_dense_f32.hip", "dtw_prep.hip", "dtw_qk.hip", "logmel.hip", "decode_ops.hip", "kv_fill.hip", "kv_noalloc.hip", "linear.hip", "wdrz_capi.cpp"]
ARCH = "gfx950"


def source_hash() -> str:
    """Hash of everything the library is built from: the kernel and C-ABI sources, the public
    header and this build script (flags). Stamped into the library (wdrz_build_id) so that a
    library built from other sources is refused at load time."""
    h = hashlib.sha256()
    files = sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp", ".h", ".inc", ".py"))
    files += sorted((PKG_DIR.parent / "include").glob("*.h"))
    files.append(Path(__file__).resolve())
    for f in files:
        h.update(f.name.encode())
        h.update(b"\0")
        h.update(f.read_bytes())
        h.update(b"\0")
    return h.hexdigest()[:16]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (ROCm toolchain required to build libwdrz_attn.so)")


def build_library(debug: bool = False, verbose: bool = False) -> Path:
    """Compile every source for gfx950 and link libwdrz_attn.so next to this file."""
    out_dir = PKG_DIR / "_build"
    out_dir.mkdir(exist_ok=True)
    # the encoder kernel's hand-scheduled loop is generated (rewritten only when it changes)
    gen = subprocess.run([sys.executable, str(CSRC / "gen_dense_loop.py")], capture_output=True, text=True)
    if gen.returncode != 0:
        raise RuntimeError(f"gen_dense_loop.py failed:\n{gen.stderr}")
    opt = ["-O1", "-g"] if debug else ["-O3"]
    common = [
        f"--offload-arch={ARCH}",
        "-fPIC",
        "-std=c++17",
        "-Wall",
        "-Wno-unused-function",
        *opt,
    ]
    # Packed-fp32 instructions are disabled for all device code (they have returned wrong
    # results on these boxes); the flag is device-only, hipcc's host pass merely warns.
    device_flags = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]
    # Per-file device flags. The kernels assume no NaN inputs (masking uses -inf): without
    # this, every fmaxf on a computed score pays an extra canonicalising max.
    per_file = {
        "attn_dense.hip": ["-fno-honor-nans"],
        "attn_kvcache.hip": ["-fno-honor-nans"],
        "dtw_prep.hip": ["-fno-honor-nans"],  # NaN outputs are written explicitly, never computed
        "dtw_qk.hip": ["-fno-honor-nans"],
    }
    objs, cmds = [], []
    build_id = f'-DWDRZ_BUILD_ID="{source_hash()}"'
    for src in SOURCES:
        obj = out_dir / (src + ".o")
        cmd = [hipcc(), *common, "-c", str(CSRC / src), "-o", str(obj)]
        if src == "wdrz_capi.cpp":
            cmd.append(build_id)
        if src.endswith(".hip"):
            cmd[1:1] = ["-x", "hip"]
            cmd += device_flags + per_file.get(src, [])
        if verbose:
            print(" ".join(cmd), flush=True)
        cmds.append((src, cmd))
        objs.append(str(obj))
    # the sources compile independently: run the compilers side by side
    jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        for (src, _), proc in zip(cmds, pool.map(lambda c: subprocess.run(c[1], capture_output=True, text=True), cmds)):
            if proc.returncode != 0:
                raise RuntimeError(f"hipcc failed for {src}:\n{proc.stderr}")
    # the host-checked twin: the C-ABI layer again, with WDRZ_DEBUG_CHECKS
    capi_dbg = out_dir / "wdrz_capi.debug.o"
    cmd = [hipcc(), *common, "-DWDRZ_DEBUG_CHECKS", build_id, "-c", str(CSRC / "wdrz_capi.cpp"), "-o", str(capi_dbg)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for wdrz_capi.cpp (debug checks):\n{proc.stderr}")
    objs_dbg = [str(capi_dbg) if o.endswith("wdrz_capi.cpp.o") else o for o in objs]
    for target, parts in ((LIB_PATH, objs), (DEBUG_LIB_PATH, objs_dbg)):
        tmp = out_dir / (target.name + ".tmp")
        cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *parts, "-o", str(tmp)]
        proc = subprocess.run(cmd, capture_output=True, text=True)
        if proc.returncode != 0:
            raise RuntimeError(f"link failed:\n{proc.stderr}")
        os.replace(tmp, target)
    return LIB_PATH


if __name__ == "__main__":
    p = build_library(debug="--debug" in sys.argv, verbose=True)
    print(p)
