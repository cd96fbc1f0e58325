"""Ahead-of-time build of the native parts of the backend.

* ``libnkipy_hip.so``  -- the C-ABI runtime (``csrc/runtime.cpp``), host code
  linked against the HIP runtime.
* ``<name>.hsaco``     -- one gfx950 code object per ``csrc/kernels/*.hip``,
  loaded at run time with ``hipModuleLoad``.

Everything is written into ``nkipy_amd/lib/`` inside the source tree, so a
copy of the tree carries its built artefacts.  ``hipcc`` cross-compiles for
gfx950 without a GPU present.
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
KERNEL_DIR = CSRC / "kernels"
LIB_DIR = PKG_DIR / "lib"
REPO_DIR = PKG_DIR.parent
INCLUDE_DIR = REPO_DIR / "include"

ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))
HIPCC = str(ROCM / "bin" / "hipcc")
ARCH = os.environ.get("NKIPY_GPU_ARCH", "gfx950")

# Packed-fp32 VALU forms are disabled for all device code: the compiler may
# otherwise form v_pk_* fp32 instructions from ordinary float code.
NO_PACKED_FP32 = ["-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"]

RUNTIME_LIB = LIB_DIR / "libnkipy_hip.so"


def _run(cmd):
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            "build step failed:\n  " + " ".join(cmd) + "\n" + proc.stdout + proc.stderr
        )
    return proc


def build_runtime() -> Path:
    """The C-ABI library: the runtime core (host code) plus the compute entry
    points, whose gfx950 kernels are compiled into the library."""
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    tmp = RUNTIME_LIB.with_suffix(".so.tmp")
    cmd = [
        HIPCC,
        "-O3",
        "-fPIC",
        "-shared",
        "-std=c++17",
        f"--offload-arch={ARCH}",
        *NO_PACKED_FP32,
        f"-I{INCLUDE_DIR}",
        f"-I{KERNEL_DIR}",
        str(CSRC / "runtime.cpp"),
        str(CSRC / "entry.hip"),
        "-o",
        str(tmp),
    ]
    _run(cmd)
    os.replace(tmp, RUNTIME_LIB)
    return RUNTIME_LIB


def kernel_sources():
    return sorted(KERNEL_DIR.glob("*.hip"))


def hsaco_path(name: str) -> Path:
    return LIB_DIR / f"{name}.hsaco"


def build_kernel(src: Path) -> Path:
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    out = hsaco_path(src.stem)
    tmp = out.with_suffix(".hsaco.tmp")
    cmd = [
        HIPCC,
        "--genco",
        "--no-gpu-bundle-output",
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        *NO_PACKED_FP32,
        f"-I{KERNEL_DIR}",
        str(src),
        "-o",
        str(tmp),
    ]
    _run(cmd)
    os.replace(tmp, out)
    write_manifest(out)
    return out


def read_kernel_metadata(hsaco: Path) -> dict:
    """Kernel name -> {kernarg_size, vgpr, agpr, sgpr, lds, spills} from the
    code object's AMDGPU metadata note (read with llvm-readelf)."""
    readelf = str(ROCM / "llvm" / "bin" / "llvm-readelf")
    txt = _run([readelf, "--notes", str(hsaco)]).stdout
    kernels = {}
    cur = {}
    arg = {}
    keys = {
        ".kernarg_segment_size": "kernarg_size",
        ".vgpr_count": "vgpr",
        ".agpr_count": "agpr",
        ".sgpr_count": "sgpr",
        ".group_segment_fixed_size": "lds",
        ".vgpr_spill_count": "vgpr_spill",
        ".sgpr_spill_count": "sgpr_spill",
        ".max_flat_workgroup_size": "max_block",
        ".private_segment_fixed_size": "scratch",
    }
    for line in txt.splitlines():
        line = line.strip().lstrip("- ").strip()
        if ":" not in line:
            continue
        k, _, v = line.partition(":")
        k, v = k.strip(), v.strip()
        # explicit (non-hidden) argument bytes: what the caller packs
        if k in (".offset", ".size"):
            arg[k] = int(v)
        elif k == ".value_kind":
            if not v.startswith("hidden_") and ".offset" in arg and ".size" in arg:
                cur["explicit_size"] = max(cur.get("explicit_size", 0), arg[".offset"] + arg[".size"])
            if v.startswith("hidden_"):
                cur["hidden_args"] = True
            arg = {}
        elif k in keys:
            try:
                cur[keys[k]] = int(v)
            except ValueError:
                pass
        elif k == ".name" and not v.endswith(".kd"):
            cur["name"] = v
        # Keys are emitted in sorted order; .wavefront_size closes an entry.
        if k == ".wavefront_size" and "name" in cur:
            cur.setdefault("explicit_size", 0)
            kernels[cur.pop("name")] = cur
            cur = {}
    return kernels


def write_manifest(hsaco: Path) -> Path:
    meta = read_kernel_metadata(hsaco)
    out = hsaco.with_suffix(".json")
    out.write_text(json.dumps(meta, indent=1, sort_keys=True))
    return out


def build_all(verbose: bool = False, jobs: int = 8) -> list:
    """Compile the runtime library and every kernel source.  Always rebuilds."""
    srcs = kernel_sources()
    with ThreadPoolExecutor(max_workers=max(1, min(jobs, len(srcs) + 1))) as ex:
        futs = [ex.submit(build_runtime)] + [ex.submit(build_kernel, s) for s in srcs]
        outs = [f.result() for f in futs]
    if verbose:
        for o in outs:
            print(f"built {o.relative_to(REPO_DIR)}", file=sys.stderr)
    return outs


def is_built() -> bool:
    if not RUNTIME_LIB.exists():
        return False
    return all(hsaco_path(s.stem).exists() for s in kernel_sources())


if __name__ == "__main__":
    build_all(verbose=True)
