"""ctypes binding of ``libmoe_hip.so`` (the C ABI declared in ``include/moe_hip.h``).

The library is built in-tree (``make -C cuda-moe-engine_amd/csrc``) and loaded
after torch so both share one HIP runtime. There is no fallback: if the
library is missing or fails to load, every HIP operator raises.
"""

from __future__ import annotations

import ctypes
import os
from functools import lru_cache
from pathlib import Path

LIBRARY_NAME = "libmoe_hip.so"
ABI_VERSION = 8

DTYPE_F32 = 0
DTYPE_F16 = 1
DTYPE_BF16 = 2

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int

# name -> (restype, argtypes); mirrors include/moe_hip.h
_SIGNATURES = {
    "moe_abi_version": (_int, []),
    "moe_status_string": (ctypes.c_char_p, [_int]),
    "moe_last_error": (ctypes.c_char_p, []),
    "moe_topk_route": (_int, [_c_void_p] * 5 + [_i64, _i64, _i64, _c_void_p]),
    "moe_router_scratch_bytes": (_i64, [_i64, _i64]),
    "moe_router_fused": (_int, [_c_void_p] * 8 + [_i64] * 5 + [_c_void_p]),
    "moe_router_split": (_int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _c_void_p]),
    "moe_router_rank_tile": (_i64, [_i64, _i64]),
    "moe_router_fused_ranked": (_int, [_c_void_p] * 8 + [_i64] * 5 + [_c_void_p, _c_void_p, _i64, _c_void_p]),
    "moe_dispatch_scratch_bytes": (_i64, [_i64, _i64, _i64]),
    "moe_dispatch": (
        _int,
        [_c_void_p, _int] + [_c_void_p] * 7 + [_i64] * 7 + [_int, _c_void_p],
    ),
    "moe_dispatch_noalloc": (
        _int,
        [_c_void_p, _int] + [_c_void_p] * 6 + [_i64] * 6 + [_int, _c_void_p],
    ),
    "moe_dispatch_ranked": (
        _int,
        [_c_void_p, _int] + [_c_void_p] * 8 + [_i64] * 8 + [_int, _c_void_p],
    ),
    "moe_dispatch_rows": (_int, [_c_void_p] * 7 + [_i64] * 6 + [_c_void_p]),
    "moe_dispatch_ranked_rows": (_int, [_c_void_p] * 8 + [_i64] * 7 + [_c_void_p]),
    "moe_combine": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _c_void_p] + [_i64] * 4 + [_c_void_p]),
    "moe_swiglu": (_int, [_c_void_p, _int, _c_void_p, _c_void_p, _i64, _i64, _c_void_p]),
    "moe_grouped_gemm": (_int, [_c_void_p] * 4 + [_i64] * 4 + [_c_void_p]),
    "moe_grouped_gateup_swiglu": (_int, [_c_void_p] * 4 + [_i64] * 4 + [_c_void_p]),
    "moe_grouped_gateup_swiglu_gathered": (_int, [_c_void_p, _c_void_p, _i64] + [_c_void_p] * 3 + [_i64] * 4
                                           + [_c_void_p]),
    "moe_grouped_gemm_strided": (_int, [_c_void_p, _c_void_p, _i64] + [_c_void_p] * 2 + [_i64] * 4 + [_c_void_p]),
    "moe_grouped_gateup_swiglu_strided": (_int, [_c_void_p, _c_void_p, _i64] + [_c_void_p] * 2 + [_i64] * 4
                                          + [_c_void_p]),
    "moe_grouped_gateup_swiglu_gathered_strided": (_int, [_c_void_p, _c_void_p, _i64, _c_void_p, _i64]
                                                   + [_c_void_p] * 2 + [_i64] * 4 + [_c_void_p]),
    "moe_set_gemm_workgroups": (_int, [_i64]),
}

EXPORTED_SYMBOLS = tuple(_SIGNATURES)


def library_path() -> Path:
    override = os.environ.get("MOE_HIP_LIBRARY")
    if override:
        return Path(override)
    return Path(__file__).resolve().parent / LIBRARY_NAME


class HipLibraryError(RuntimeError):
    """The HIP library is missing, stale or failed to load."""


class MoeHipError(RuntimeError):
    """A C-ABI call returned a non-OK status."""


class _Library:
    def __init__(self, handle: ctypes.CDLL, path: Path):
        self.handle = handle
        self.path = path
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
            setattr(self, name, fn)

    def check(self, status: int, what: str) -> None:
        if status != 0:
            detail = self.moe_last_error().decode(errors="replace")
            kind = self.moe_status_string(status).decode(errors="replace")
            raise MoeHipError(f"{what}: {kind}: {detail}")


@lru_cache(maxsize=1)
def load_library(require_symbols_only: bool = False) -> _Library:
    """Load the prebuilt library; raises HipLibraryError when it is absent.

    Importing torch first makes the library bind to torch's HIP runtime (same
    soname), so torch streams and device pointers are valid in both.
    """
    import torch  # noqa: F401  (load order: torch's libamdhip64 first)

    path = library_path()
    if not path.is_file():
        raise HipLibraryError(
            f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            " or `make -C cuda-moe-engine_amd/csrc`"
        )
    try:
        handle = ctypes.CDLL(str(path), mode=ctypes.RTLD_GLOBAL)
    except OSError as exc:  # pragma: no cover - depends on the box
        raise HipLibraryError(f"cannot load {path}: {exc}") from exc
    missing = [name for name in _SIGNATURES if not hasattr(handle, name)]
    if missing:
        raise HipLibraryError(f"{path} lacks symbols {missing}; rebuild it")
    lib = _Library(handle, path)
    version = lib.moe_abi_version()
    if version != ABI_VERSION:
        raise HipLibraryError(f"{path} has ABI version {version}, expected {ABI_VERSION}")
    return lib
