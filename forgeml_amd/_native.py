"""ctypes binding of ``libforgeml_hip.so`` (the C ABI in include/forgeml_hip.h).

The library is loaded after ``torch`` so that its ``libamdhip64.so.7``
dependency resolves, by soname, to the HIP runtime PyTorch-ROCm already
mapped: device pointers and ``hipStream_t`` handles from torch are then valid
in the library.  Loading refuses to continue if two HIP runtimes end up
mapped in the process.  There is no fallback: if the library is missing or
does not load, every GPU call raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

from forgeml_amd.ir import GraphError

LIBRARY_PATH = Path(__file__).resolve().parent / "libforgeml_hip.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "forgeml_hip.h"

ABI_VERSION = 5

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
ACT_NONE, ACT_GELU_ERF, ACT_GELU_TANH, ACT_RELU = 0, 1, 2, 3
OK, EINVAL, ECONFIG, EHIP, EWORKSPACE = 0, -1, -2, -3, -4
CONFIG_AUTO = -1
CONFIG_INFO_FIELDS = 8

# Exported symbols and their ctypes signatures (restype, argtypes).
_I64, _I32, _P = ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p
SIGNATURES: dict[str, tuple] = {
    "forgeml_hip_gemm": (
        ctypes.c_int,
        [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _I32, _I32, _P, _I64, _P],
    ),
    "forgeml_hip_gemm_add": (
        ctypes.c_int,
        [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _P, _I64, _I64, _I64, _I32, _I32, _I32, _P, _I64,
         _P],
    ),
    "forgeml_hip_gemm_noalloc": (
        ctypes.c_int,
        [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I64, _I32, _I32, _I32, _P],
    ),
    "forgeml_hip_noalloc_scratch_bytes": (_I64, []),
    "forgeml_hip_layer_norm": (ctypes.c_int, [_P, _I64, _P, _P, _P, _I64, _I64, ctypes.c_float, _I32, _P]),
    "forgeml_hip_attention": (
        ctypes.c_int,
        [_P, ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64), _P, ctypes.POINTER(_I64),
         _I64, _I64, _I64, _I64, _I64, _I32, ctypes.c_float, _I32, _P],
    ),
    "forgeml_hip_gemm_plan": (
        ctypes.c_int,
        [_P, _I64, _I64, _P, _I64, _I64, _I64, _I64, _I64, _I32, _I32, ctypes.POINTER(_I64)],
    ),
    "forgeml_hip_gemm_workspace_size": (_I64, [_I64, _I64, _I64, _I32, _I32]),
    "forgeml_hip_select_config": (ctypes.c_int, [_I64, _I64, _I64, _I32]),
    "forgeml_hip_num_configs": (ctypes.c_int, []),
    "forgeml_hip_config_info": (ctypes.c_int, [_I32, ctypes.POINTER(_I32)]),
    "forgeml_hip_last_error": (ctypes.c_char_p, []),
    "forgeml_hip_abi_version": (ctypes.c_int, []),
}


class NativeLibraryError(GraphError):
    """The gfx950 kernel library is missing, stale or failed to load."""


_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def hip_runtimes_mapped() -> list[str]:
    """Distinct libamdhip64 files mapped into this process."""
    try:
        with open("/proc/self/maps") as fh:
            return sorted({line.split()[-1] for line in fh if "libamdhip64" in line})
    except OSError:
        return []


def load() -> ctypes.CDLL:
    """Load (once) and return the kernel library; raises NativeLibraryError."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        import torch  # noqa: F401  (maps torch's HIP runtime before the library needs one)

        if not LIBRARY_PATH.exists():
            raise NativeLibraryError(
                f"{LIBRARY_PATH.name} is not built; run `python -m forgeml_amd._build` (hipcc, gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(LIBRARY_PATH), mode=ctypes.RTLD_LOCAL)
        except OSError as e:
            raise NativeLibraryError(f"cannot load {LIBRARY_PATH}: {e}") from e
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name, None)
            if fn is None:
                raise NativeLibraryError(f"{LIBRARY_PATH.name} does not export {name}; rebuild it")
            fn.restype = restype
            fn.argtypes = argtypes
        version = lib.forgeml_hip_abi_version()
        if version != ABI_VERSION:
            raise NativeLibraryError(f"library ABI {version} != expected {ABI_VERSION}; rebuild it")
        runtimes = hip_runtimes_mapped()
        if len(runtimes) > 1:
            raise NativeLibraryError(f"more than one HIP runtime is mapped: {runtimes}")
        _lib = lib
        return lib


def last_error() -> str:
    lib = load()
    msg = lib.forgeml_hip_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def config_table() -> list[tuple[int, ...]]:
    """The library's tile table as tuples of CONFIG_INFO_FIELDS ints."""
    lib = load()
    out = []
    buf = (ctypes.c_int32 * CONFIG_INFO_FIELDS)()
    for i in range(lib.forgeml_hip_num_configs()):
        rc = lib.forgeml_hip_config_info(i, buf)
        if rc != OK:
            raise NativeLibraryError(f"config_info({i}) failed: {last_error()}")
        out.append(tuple(buf))
    return out
