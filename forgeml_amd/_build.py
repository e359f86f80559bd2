"""Build the gfx950 kernel library ``forgeml_amd/libforgeml_hip.so`` with hipcc.

Each ``csrc/*.hip`` translation unit is compiled to an object in parallel and
the objects are linked into one shared library next to this file, so the
built library travels with the source tree.  The library links against the
HIP runtime by soname (``libamdhip64.so.7``); at run time it binds to the one
PyTorch-ROCm has already loaded (see ``forgeml_amd._native``).

Run ``python -m forgeml_amd._build`` to rebuild.
"""

from __future__ import annotations

import hashlib
import json
import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
INCLUDE = REPO_ROOT / "include"
BUILD_DIR = PACKAGE_DIR / "_build"
LIBRARY = PACKAGE_DIR / "libforgeml_hip.so"

OFFLOAD_ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-mcode-object-version=5",
    # Packed fp32 VALU ops (v_pk_*_f32) are kept out of every kernel.
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the gfx950 kernels cannot be built")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(
            f"command failed ({proc.returncode}): {' '.join(cmd)}\n{proc.stdout}\n{proc.stderr}"
        )
    # hipcc's host pass does not know the packed-fp32 feature and says so;
    # anything else is worth showing.
    noise = "is not a recognized feature for this target"
    lines = [ln for ln in proc.stderr.splitlines() if ln.strip() and noise not in ln]
    if lines:
        print("\n".join(lines), file=sys.stderr)


def build(jobs: int | None = None) -> Path:
    """Compile every HIP source under csrc/ and link libforgeml_hip.so."""
    compiler = hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    include_flags = [f"-I{INCLUDE}", f"-I{CSRC}"]
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = jobs or min(len(sources), max(1, (os.cpu_count() or 2)))
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        futures = [
            pool.submit(_run, [compiler, *HIPCC_FLAGS, *include_flags, "-c", str(src), "-o", str(obj)])
            for src, obj in zip(sources, objects)
        ]
        for f in futures:
            f.result()
    tmp = LIBRARY.with_suffix(".so.tmp")
    _run([compiler, *HIPCC_FLAGS, "-shared", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, LIBRARY)
    _write_build_info(sources)
    return LIBRARY


BUILD_INFO = PACKAGE_DIR / "_build_info.json"


def _write_build_info(sources) -> None:
    """Provenance of the built library, read by measurement.environment where
    the tree has no git metadata: the commit it was built at and a hash of
    every kernel source and header it was built from."""
    digest = hashlib.sha256()
    for path in sorted([*sources, *CSRC.glob("*.hpp"), *INCLUDE.glob("*.h")]):
        digest.update(path.name.encode())
        digest.update(path.read_bytes())
    info = {"sources_sha256": digest.hexdigest(), "hipcc_flags": HIPCC_FLAGS}
    try:
        info["git_commit"] = subprocess.check_output(["git", "rev-parse", "HEAD"], cwd=REPO_ROOT, text=True,
                                                     stderr=subprocess.DEVNULL).strip()
        info["git_dirty"] = bool(subprocess.check_output(["git", "status", "--porcelain", "--", "forgeml_amd/csrc",
                                                          "include"], cwd=REPO_ROOT, text=True,
                                                         stderr=subprocess.DEVNULL).strip())
    except (OSError, subprocess.CalledProcessError):
        info["git_commit"] = None
    BUILD_INFO.write_text(json.dumps(info, indent=1) + "\n")


if __name__ == "__main__":
    path = build()
    print(path)
