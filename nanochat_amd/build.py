"""Build libnc_kv.so (the gfx950 HIP kernels + C ABI) in-tree with hipcc.

    python -m nanochat_amd.build            # compile every source, link the .so

The library lands next to this file (nanochat_amd/libnc_kv.so) so it travels
with the repository snapshot; nothing is installed or cached elsewhere.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
INCLUDE = REPO_DIR / "include"
LIB_NAME = "libnc_kv.so"
LIB_PATH = PKG_DIR / LIB_NAME
# measurement tooling for bench.py (read-bandwidth ceilings); not part of the KV-cache library
PROBE_SOURCE = "probe.hip"
PROBE_PATH = PKG_DIR / "libnc_probe.so"
OBJ_DIR = PKG_DIR / "_build"
ARCH = "gfx950"

SOURCES = ["nc_kv_abi.hip", "kv_copy.hip", "attn_decode.hip", "attn_decode_bf16.hip", "attn_decode_f16.hip",
           "attn_decode_f32.hip", "attn_chunk.hip", "linear_small_m.hip",
           "sample.hip"]

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    # Keep the compiler from forming packed-fp32 VALU ops (v_pk_*_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wno-unused-command-line-argument",
]

# Per-source flags.  The MFMA chunk kernel keeps its accumulators in VGPRs
# (the MFMA forms that read and write VGPRs): with the compiler's default
# AGPR accumulators every key tile copied the 32 output values to VGPRs and
# back for the softmax rescale, and the kernel held 2 waves per SIMD instead
# of 3.
SOURCE_FLAGS = {
    "attn_chunk.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
    "linear_small_m.hip": ("-mllvm", "-amdgpu-mfma-vgpr-form"),
}


def _hipcc() -> str:
    path = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not os.path.exists(path):
        raise RuntimeError("hipcc not found: the ROCm toolchain is required to build libnc_kv.so")
    return path


def _compile(src: str, obj_dir: Path, extra: tuple) -> Path:
    obj = obj_dir / (Path(src).stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src, ()), *extra, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
           str(CSRC / src), "-o", str(obj)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{res.stderr}")
    return obj


def build(verbose: bool = True, defines: dict | None = None, out: Path | None = None) -> Path:
    """Compile all kernels for gfx950 and link nanochat_amd/libnc_kv.so.

    `defines` (e.g. {"NC_DECODE_WAVES": 8}) and `out` build a tuning variant
    of the library at another path, leaving the in-tree build alone.
    """
    out = Path(out) if out is not None else LIB_PATH
    extra = tuple(f"-D{k}={v}" for k, v in sorted((defines or {}).items()))
    obj_dir = OBJ_DIR if not extra else OBJ_DIR / ("v_" + "_".join(f"{k}{v}" for k, v in sorted(defines.items())))
    obj_dir.mkdir(parents=True, exist_ok=True)
    workers = min(len(SOURCES), os.cpu_count() or 2, 8)
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, obj_dir, extra), SOURCES))
    tmp = out.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objs)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, out)
    if verbose:
        print(f"built {out}", flush=True)
    if not extra and out == LIB_PATH:
        build_probe(verbose)
    return out


def build_probe(verbose: bool = True) -> Path:
    """Compile bench.py's read-bandwidth probes into nanochat_amd/libnc_probe.so."""
    OBJ_DIR.mkdir(parents=True, exist_ok=True)
    obj = _compile(PROBE_SOURCE, OBJ_DIR, ())
    tmp = PROBE_PATH.with_suffix(".so.tmp")
    res = subprocess.run([_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), str(obj)],
                         capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, PROBE_PATH)
    if verbose:
        print(f"built {PROBE_PATH}", flush=True)
    return PROBE_PATH


if __name__ == "__main__":
    build()
    sys.exit(0)
