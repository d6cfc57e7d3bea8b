"""Build ``libqxt_gfx950.so`` (the HIP kernels + C ABI) in-tree with hipcc.

Usage: ``python qpu-xla-triton_amd/build.py`` (or ``__graft_entry__.build()``).
Sources are compiled in parallel to objects under ``_build/`` and linked into
``qpu_xla_amd/libqxt_gfx950.so`` next to the Python package that loads it.
"""

from __future__ import annotations

import concurrent.futures
import hashlib
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent
REPO_ROOT = PKG_ROOT.parent
CSRC = PKG_ROOT / "csrc"
BUILD_DIR = PKG_ROOT / "_build"
LIBRARY = PKG_ROOT / "qpu_xla_amd" / "libqxt_gfx950.so"
ARCH = "gfx950"

# -ffp-contract=off: no multiply-add fusion, so fp32 results match NumPy's separately
#   rounded operations bit for bit.
# -fhip-fp32-correctly-rounded-divide-sqrt: '/' is IEEE division (quantiser parity).
# -packed-fp32-ops: keep the compiler from emitting packed fp32 VALU instructions.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-ffp-contract=off",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-source additions.  The prefill kernel and the four-row decode tiles
# convert every matrix-core result with VALU instructions, so their MFMAs
# write VGPRs directly (no accumulator-register copies); the W8A8 GEMM keeps
# its 256 accumulators in AGPRs.
SOURCE_FLAGS = {
    "qxt_q4_0_tiled.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
    "qxt_q4_0.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found: the gfx950 library cannot be built")
    return found


def source_hash() -> str:
    """SHA-256 over every kernel source and public header, in name order.

    Compiled in as ``QXT_Q4_0_SOURCE_HASH`` and returned by
    ``qxt_llama_q4_0_source_hash()``: the value a prepared linear's
    ``expected_source_hash`` must carry.
    """
    digest = hashlib.sha256()
    files = sorted([*CSRC.glob("*.hip"), *CSRC.glob("*.h"), *(REPO_ROOT / "include").glob("*.h")], key=lambda f: f.name)
    for path in files:
        digest.update(path.name.encode())
        digest.update(b"\0")
        digest.update(path.read_bytes())
    return digest.hexdigest()


def _compile(source: Path, defines: tuple[str, ...] = ()) -> Path:
    obj = BUILD_DIR / (source.stem + ".o")
    cmd = [_hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(source.name, []), *defines, "-I", str(REPO_ROOT / "include"),
           "-I", str(CSRC), "-c", str(source), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{proc.stderr}")
    noise = "is not a recognized feature for this target"
    warnings = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if warnings.strip():
        print(warnings, file=sys.stderr)
    return obj


def build(verbose: bool = True) -> Path:
    """Compile every ``csrc/*.hip`` for gfx950 and link the shared library."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    defines = (f'-DQXT_Q4_0_SOURCE_HASH="{source_hash()}"',)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        objects = list(pool.map(lambda src: _compile(src, defines), sources))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [_hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY.relative_to(REPO_ROOT)} from {len(sources)} sources")
    return LIBRARY


if __name__ == "__main__":
    build()
