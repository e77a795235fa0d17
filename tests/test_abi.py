"""The C-ABI library loads and exports every entry point include/moe_hip.h declares.

Argument validation runs before any HIP call, so the error paths are checked
here without a GPU (no kernel is launched).
"""

import ctypes
import re
from pathlib import Path

import pytest
import torch

from moe_dispatch import _lib

# The validation tests pass stand-in addresses that are never dereferenced:
# every call is refused by its argument checks before any launch. Where a GPU
# is visible, a check that stopped refusing would launch a kernel on them, so
# those tests run only where no kernel can launch (the GPU tests use real
# buffers).
stand_in_addresses = pytest.mark.skipif(torch.cuda.is_available(),
                                        reason="stand-in addresses: run where no kernel can launch")

HEADER = Path(__file__).resolve().parents[1] / "include" / "moe_hip.h"


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(moe_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_table():
    assert declared_functions() == sorted(_lib.EXPORTED_SYMBOLS)


def _declarations():
    """name -> (return kind, [parameter kinds]) from the header, kinds being
    'p' (any pointer), 'i64' (int64_t) and 'i' (int)."""
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w \*]*?)\b(moe_[a-z0-9_]+)\s*\(([^)]*)\)\s*;", text):
        def kind(decl):
            decl = decl.strip()
            if "*" in decl:
                return "p"
            return "i64" if decl.startswith("int64_t") else "i"
        ret = ret.split("\n")[-1].strip()
        args = [] if params.strip() in ("", "void") else [kind(x) for x in params.split(",")]
        out[name] = (kind(ret + " x"), args)
    return out


def test_binding_table_matches_the_header_signatures():
    """Every ctypes signature has the header's parameter count and kinds, so a call
    with a wrong argument list fails in Python instead of reading garbage."""
    kinds = {ctypes.c_void_p: "p", ctypes.c_char_p: "p", ctypes.c_int64: "i64", ctypes.c_int: "i"}
    declared = _declarations()
    assert sorted(declared) == sorted(_lib.EXPORTED_SYMBOLS)
    for name, (restype, argtypes) in _lib._SIGNATURES.items():
        ret, params = declared[name]
        assert [kinds[t] for t in argtypes] == params, name
        assert kinds[restype] == ret, name


def test_library_exports_every_declared_symbol():
    lib = _lib.load_library()
    handle = ctypes.CDLL(str(lib.path))
    for name in declared_functions():
        assert hasattr(handle, name), name
    assert lib.moe_abi_version() == _lib.ABI_VERSION


def test_status_strings():
    lib = _lib.load_library()
    assert lib.moe_status_string(0) == b"ok"
    assert lib.moe_status_string(4) == b"workspace too small"
    assert lib.moe_status_string(99) == b"unknown status"


@stand_in_addresses
def test_validation_errors_without_launching():
    lib = _lib.load_library()
    assert lib.moe_topk_route(None, None, None, None, None, 5, 65, 2, None) == 2
    assert b"1..64" in lib.moe_last_error()
    assert lib.moe_topk_route(None, None, None, None, None, 5, 8, 9, None) == 2
    # Empty batches are valid no-ops.
    assert lib.moe_topk_route(None, None, None, None, None, 0, 8, 2, None) == 0
    assert lib.moe_combine(None, 2, None, None, None, 0, 64, 2, 0, None) == 0
    # Undersized packed workspace: T=10, K=2, E=8, a=8 needs 80 rows.
    need = lib.moe_dispatch_scratch_bytes(10, 8, 2)
    assert need > 0
    status = lib.moe_dispatch(1, 2, 1, 1, 1, 1, 1, 1, 1, need, 10, 64, 8, 2, 8, 79, 1, None)
    assert status == 4 and b"needs 80" in lib.moe_last_error()
    assert lib.moe_dispatch(1, 2, 1, 1, 1, 1, 1, 1, 1, 0, 10, 64, 8, 2, 8, 80, 1, None) == 4
    assert lib.moe_dispatch(1, 7, 1, 1, 1, 1, 1, 1, 1, need, 10, 64, 8, 2, 8, 80, 1, None) == 1
    assert lib.moe_grouped_gemm(1, 1, 1, 1, 16, 12, 64, 8, None) == 2
    assert lib.moe_grouped_gateup_swiglu(1, 1, 1, 1, 16, 64, 64, 65, None) == 2
    # One expert's weights of 4 GiB or more do not fit the kernels' 32-bit buffer ranges.
    assert lib.moe_grouped_gemm(1, 1, 1, 1, 16, 1 << 16, 1 << 15, 8, None) == 3
    assert b"4 GiB" in lib.moe_last_error()
    assert lib.moe_grouped_gateup_swiglu(1, 1, 1, 1, 16, 1 << 15, 1 << 15, 8, None) == 3
    assert lib.moe_grouped_gemm(1, 1, 1, 0, 0, 1 << 15, 1 << 15, 8, None) == 0  # 2 GiB: accepted (no rows)
    # hidden 12 is not a multiple of 8; then a scratch buffer below the split's size.
    assert lib.moe_router_fused(1, 1, 1, 1, 1, 1, None, 16, 1 << 20, 4, 12, 8, 2, None) == 2
    # Three bf16 planes (rounded up to 256 bytes), then the small-batch split's
    # fp32 partial logits: 4 token tiles x 16 slices x 16 tokens x 16 experts,
    # then the planes in fragment order: per 64 hidden, ceil(6E/16) fragments
    # of 1 KiB.
    partials = 4 * 16 * 16 * 16 * 4
    assert lib.moe_router_scratch_bytes(8, 64) == 3 * 8 * 64 * 2 + partials + 1 * 3 * 1024
    assert lib.moe_router_scratch_bytes(5, 72) == 2304 + partials + 2 * 2 * 1024  # 2160 rounded up
    assert lib.moe_router_scratch_bytes(17, 64) == 6656 + partials + 7 * 1024  # 6528 rounded up
    assert lib.moe_router_scratch_bytes(64, 4096) == 3 * 64 * 4096 * 2 + partials + 64 * 24 * 1024
    assert lib.moe_router_scratch_bytes(65, 64) == -1
    need = lib.moe_router_scratch_bytes(8, 64)
    assert lib.moe_router_fused(16, 16, 16, 16, 16, 16, None, 16, need - 1, 4, 64, 8, 2, None) == 4
    assert b"router scratch needs" in lib.moe_last_error()
    # The persistent GEMM's workgroup bound (scheduling only; no launch here).
    assert lib.moe_set_gemm_workgroups(-1) == 1
    assert lib.moe_set_gemm_workgroups(1 << 40) == 1
    assert lib.moe_set_gemm_workgroups(16) == 0 and lib.moe_set_gemm_workgroups(0) == 0


@stand_in_addresses
def test_ranked_route_arguments_are_checked_without_launching():
    lib = _lib.load_library()
    # Tile size: 16 tokens for E <= 16, 32 above; none past 4096 table entries or for no tokens.
    assert lib.moe_router_rank_tile(4096, 8) == 16 and lib.moe_router_rank_tile(4096, 16) == 16
    assert lib.moe_router_rank_tile(100, 64) == 32 and lib.moe_router_rank_tile(2048, 64) == 32
    assert lib.moe_router_rank_tile(2049, 64) == 0 and lib.moe_router_rank_tile(8192, 64) == 0
    assert lib.moe_router_rank_tile(0, 8) == 0
    assert lib.moe_router_rank_tile(10, 65) == -1 and lib.moe_router_rank_tile(-1, 8) == -1
    need = lib.moe_router_scratch_bytes(8, 64)
    # Router: 100 tokens, E=8 -> 7 tiles x 8 counts x 4 bytes = 224 bytes.
    args = (16, 16, 16, 16, 16, 16, None, 16, need, 100, 64, 8, 2)
    assert lib.moe_router_fused_ranked(*args, 16, 16, 223, None) == 4
    assert b"224" in lib.moe_last_error()
    assert lib.moe_router_fused_ranked(*args, None, 16, 224, None) == 1
    assert lib.moe_router_fused_ranked(*args, 18, 16, 224, None) == 1  # ranks not 4-byte aligned
    big = (16, 16, 16, 16, 16, 16, None, 16, lib.moe_router_scratch_bytes(64, 64), 8192, 64, 64, 6)
    assert lib.moe_router_fused_ranked(*big, 16, 16, 1 << 30, None) == 2  # no ranked route for this shape
    # Dispatch: the tile must be the route's; then the table size.
    d = (16, 2, 16, 16, 16, 16, 16, 16, 16, 16)
    tail = (100, 64, 8, 2, 1, 200, 1, None)
    assert lib.moe_dispatch_ranked(*d, 224, 32, *tail) == 1
    assert b"not the ranked route's tile" in lib.moe_last_error()
    assert lib.moe_dispatch_ranked(*d, 223, 16, *tail) == 4
    assert lib.moe_dispatch_ranked(16, 2, 16, 16, 16, 16, 16, 16, None, 16, 224, 16, *tail) == 1
    assert lib.moe_dispatch_ranked(*d, 224, 16, 100, 64, 8, 2, 1, 199, 1, None) == 4  # packed rows


@stand_in_addresses
def test_misaligned_pointers_are_rejected_without_launching():
    """Addresses the kernels cannot access as they must are refused before any launch.

    The GEMMs and the fused router read their operands with 16-byte (direct-to-LDS)
    loads, so a view starting mid-vector is an error there; the transport kernels
    take narrower accesses instead, and only an address that is not a multiple of
    the element size is an error.
    """
    lib = _lib.load_library()
    A = 1 << 20  # 16-byte aligned stand-in addresses (never dereferenced)
    assert lib.moe_grouped_gemm(A + 2, A, A, A, 16, 64, 64, 1, None) == 1
    assert b"16-byte aligned" in lib.moe_last_error()
    assert lib.moe_grouped_gemm(A, A + 8, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gemm(A, A, A + 8, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gemm(A, A, A, A + 2, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gateup_swiglu(A + 8, A, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gateup_swiglu(A, A, A + 4, A, 16, 64, 64, 1, None) == 1
    need = lib.moe_router_scratch_bytes(8, 64)
    assert lib.moe_router_fused(A + 2, A, A, A, A, A, None, A, need, 4, 64, 8, 2, None) == 1
    assert b"16-byte aligned" in lib.moe_last_error()
    assert lib.moe_router_fused(A, A, A, A, A + 4, A, None, A, need, 4, 64, 8, 2, None) == 1  # ids64
    assert lib.moe_topk_route(A, A, A, A + 4, A, 4, 8, 2, None) == 1
    assert lib.moe_topk_route(A + 2, A, A, A, A, 4, 8, 2, None) == 1
    scratch = lib.moe_dispatch_scratch_bytes(10, 8, 2)
    # bf16 rows at an odd address; then an index buffer off its 4-byte grid
    assert lib.moe_dispatch(A + 1, 2, A, A, A, A, A, A, A, scratch, 10, 64, 8, 2, 8, 80, 1, None) == 1
    assert b"element size" in lib.moe_last_error()
    assert lib.moe_dispatch(A, 2, A, A, A, A + 2, A, A, A, scratch, 10, 64, 8, 2, 1, 20, 1, None) == 1
    assert lib.moe_dispatch(A, 0, A, A, A + 2, A, A, A, A, scratch, 10, 64, 8, 2, 1, 20, 1, None) == 1
    assert lib.moe_combine(A, 0, A, A, A + 2, 4, 64, 2, 8, None) == 1  # fp32 output at +2
    assert lib.moe_combine(A, 2, A + 1, A, A, 4, 64, 2, 8, None) == 1  # inverse
    assert lib.moe_swiglu(A + 1, 2, A, A, 4, 64, None) == 1


def test_strided_gemm_arguments_are_checked_without_launching():
    """The row stride of the _strided entry points: at least the row length, a
    multiple of 8, and one expert's rows * stride within 4 GiB."""
    lib = _lib.load_library()
    A = 1 << 20  # 16-byte aligned stand-in addresses (never dereferenced)
    # a, b, stride, c, offsets, rows, n, k, E
    assert lib.moe_grouped_gemm_strided(A, A, 56, A, A, 16, 64, 64, 1, None) == 2
    assert b"row stride" in lib.moe_last_error()
    assert lib.moe_grouped_gemm_strided(A, A, 68, A, A, 16, 64, 64, 1, None) == 2
    assert lib.moe_grouped_gemm_strided(A, A, 1 << 22, A, A, 16, 1024, 64, 1, None) == 3
    assert b"4 GiB" in lib.moe_last_error()
    assert lib.moe_grouped_gemm_strided(A, A + 8, 72, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gemm_strided(A, A, 72, A, A, 0, 64, 64, 1, None) == 0  # no rows
    # a, gate_up, stride, act, offsets, rows, H, I, E
    assert lib.moe_grouped_gateup_swiglu_strided(A, A, 60, A, A, 16, 64, 64, 1, None) == 2
    assert lib.moe_grouped_gateup_swiglu_strided(A, A, 1 << 16, A, A, 16, 64, 1 << 15, 1, None) == 3
    assert lib.moe_grouped_gateup_swiglu_strided(A, A, 128, A, A, 0, 64, 64, 1, None) == 0
    # x, row_src, x_rows, gate_up, stride, act, offsets, rows, H, I, E
    assert lib.moe_grouped_gateup_swiglu_gathered_strided(A, A, 16, A, 63, A, A, 16, 64, 64, 1, None) == 2
    assert lib.moe_grouped_gateup_swiglu_gathered_strided(A, A, 16, A, 128, A, A, 0, 64, 64, 1, None) == 0


def test_error_surfaces_as_runtime_error():
    lib = _lib.load_library()
    with pytest.raises(_lib.MoeHipError, match="1..64"):
        lib.check(lib.moe_topk_route(None, None, None, None, None, 5, 65, 2, None), "topk")


@stand_in_addresses
def test_row_table_entry_points_check_their_arguments_without_launching():
    """moe_dispatch_rows, moe_dispatch_ranked_rows and the gathered gate/up GEMM
    refuse bad shapes, sizes and pointers before any launch (stand-in addresses,
    never dereferenced)."""
    lib = _lib.load_library()
    A = 1 << 20
    scratch = lib.moe_dispatch_scratch_bytes(10, 8, 2)
    # ids, counts, offsets, slots, inverse, row_src, scratch, bytes, T, E, K, a, rows
    assert lib.moe_dispatch_rows(A, A, A, A, A, A, A, scratch, 10, 8, 2, 8, 79, None) == 4  # rows < capacity (80)
    assert b"row table" in lib.moe_last_error()
    assert lib.moe_dispatch_rows(A, A, A, A, A, A, A, scratch, 10, 65, 2, 1, 20, None) == 2  # experts
    assert lib.moe_dispatch_rows(A, A, A, A, A, None, A, scratch, 10, 8, 2, 1, 20, None) == 1  # null table
    assert lib.moe_dispatch_rows(A, A, A, A, A, A + 2, A, scratch, 10, 8, 2, 1, 20, None) == 1  # misaligned
    assert lib.moe_dispatch_rows(A, A, A, A, A, A, A, scratch - 4, 10, 8, 2, 1, 20, None) == 4  # scratch
    # ranked: the tile must be the route's, then the table size
    r = (A, A, A, A, A, A, A, A)
    assert lib.moe_dispatch_ranked_rows(*r, 224, 32, 100, 8, 2, 1, 200, None) == 1
    assert b"not the ranked route's tile" in lib.moe_last_error()
    assert lib.moe_dispatch_ranked_rows(*r, 223, 16, 100, 8, 2, 1, 200, None) == 4
    # gathered gate/up: x, row_src, x_rows, gate_up, act, offsets, rows, H, I, E
    assert lib.moe_grouped_gateup_swiglu_gathered(A, A, 16, A, A, A, 16, 96, 64, 1, None) == 2
    assert b"multiple of 64" in lib.moe_last_error()
    assert lib.moe_grouped_gateup_swiglu_gathered(A, A, 1 << 18, A, A, A, 16, 4096, 64, 1, None) == 3  # 2 GiB
    assert lib.moe_grouped_gateup_swiglu_gathered(A + 8, A, 16, A, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gateup_swiglu_gathered(A, A + 2, 16, A, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gateup_swiglu_gathered(A, None, 16, A, A, A, 16, 64, 64, 1, None) == 1
    assert lib.moe_grouped_gateup_swiglu_gathered(A, A, 16, A, A, A, 0, 64, 64, 1, None) == 0  # no rows
