"""The C ABI library: it loads, exports every function ``include/ayaka_hip.h`` declares,
and refuses bad arguments on the host (no kernel is launched here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from ayaka_amd.hip import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "ayaka_hip.h"


def declared() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return re.findall(r"\b(ayk_\w+)\s*\(", text)


def test_every_declared_function_is_exported_and_bound() -> None:
    names = declared()
    assert len(names) == 21
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), name
    assert sorted(names) == sorted(_lib.EXPORTS)
    assert lib.ayk_abi_version() == _lib.ABI_VERSION


def test_multi_row_tile_capacity_matches_the_host() -> None:
    from ayaka_amd.hip import attention as hip_attention

    lib = _lib.lib()
    for head_dim, pairs in hip_attention.PREFILL_PAIRS.items():
        assert lib.ayk_paged_prefill_tile_pairs(head_dim) == pairs
    assert lib.ayk_paged_prefill_tile_pairs(96) == 0


def test_workspace_size() -> None:
    lib = _lib.lib()
    assert lib.ayk_paged_attention_v2_workspace_bytes(64, 32, 128, 8) == 64 * 32 * 8 * (128 + 2) * 4
    assert lib.ayk_paged_attention_v2_workspace_bytes(0, 32, 128, 8) == 0


def _v1(lib: ctypes.CDLL, **kw: object) -> int:
    args = dict(out=1, q=1, k=1, v=1, table=1, stride=4, lengths=1, ror=None, pos=None, n_rows=1,
                heads=8, kv_heads=2, head_dim=128, num_blocks=10, block_size=16, max_blocks=4,
                layout=0, dtype=1, kv_dtype=1, scale=ctypes.c_float(1.0), k_scale=1.0, v_scale=1.0, flags=0,
                stream=None)
    args.update(kw)
    return lib.ayk_paged_attention_v1(*args.values())


@pytest.mark.parametrize(
    "changes,code,message",
    [
        ({"head_dim": 96}, 2, b"head_dim 96"),
        ({"dtype": 5}, 2, b"dtype 5"),
        ({"kv_dtype": 0}, 2, b"kv_dtype 0"),
        ({"kv_dtype": 2, "flags": 1}, 2, b"16-bit caches only"),
        ({"layout": 3}, 2, b"layout 3"),
        ({"heads": 6, "kv_heads": 4}, 1, b"not a positive multiple"),
        ({"block_size": 0}, 2, b"block_size 0 is not in [1, 65536]"),
        ({"max_blocks": 1 << 24, "stride": 1 << 24}, 2, b"exceeds 2^24"),
        ({"ror": 1}, 1, b"together"),
        ({"q": None}, 1, b"null"),
        ({"stride": 2}, 1, b"table_stride"),
        ({"flags": 3}, 1, b"exclude each other"),
        ({"flags": 1024}, 1, b"unknown flags"),
        ({"flags": 32 | 64}, 1, b"at most one AYK_FLAG_WAVES"),
        ({"flags": 1 | 128}, 2, b"does not split a context"),
    ],
)
def test_bad_arguments_are_refused_without_a_launch(changes: dict, code: int, message: bytes) -> None:
    lib = _lib.lib()
    assert _v1(lib, **changes) == code
    assert message in lib.ayk_last_error()


def test_v2_and_store_refusals() -> None:
    lib = _lib.lib()
    base = [1, 1, 1, 1, 1, 4, 1, None, None, 1, 8, 2, 128, 10, 16, 4, 0, 1, 1, ctypes.c_float(1.0), 1.0, 1.0]
    assert lib.ayk_paged_attention_v2(*base, 100, 4, None, 0, None, 1, 1 << 20, None, 0, None) == 1
    assert b"multiple of 64" in lib.ayk_last_error()
    assert lib.ayk_paged_attention_v2(*base, 512, 4, None, 0, None, 1, 16, None, 0, None) == 4
    assert b"workspace" in lib.ayk_last_error()
    assert lib.ayk_paged_attention_v2(*base, 512, 4, None, 3, None, 1, 1 << 20, None, 0, None) == 1
    assert b"work items" in lib.ayk_last_error()
    assert lib.ayk_paged_attention_v2(*base, 512, 4, None, 0, None, 16, 1 << 20, None, 8 | 16, None) == 1
    assert b"exclude each other" in lib.ayk_last_error()
    assert lib.ayk_paged_attention_v2(*base, 512, 4, None, 0, 1, 16, 1 << 20, None, 0, None) == 1
    assert b"staged parameters need a work list" in lib.ayk_last_error()
    # the multi-row entry: tiles of the full capacity (128 at head_dim 128), a half or a
    # quarter; a partition size that is not a multiple of 64; the partitions' workspace
    def prefill(tile_pairs: int, size: int = 0, workspace: int = 0) -> int:
        return lib.ayk_paged_prefill(1, 1, 1, 1, 1, 4, 1, 1, 1, 1, 2, tile_pairs, 3, 8, 2, 128, 10, 16, 4, 0, 1, 1,
                                     ctypes.c_float(1.0), 1.0, 1.0, size, 1, workspace, None)
    assert prefill(100) == 1 and b"tile_pairs 100 is not 128, 64 or 32" in lib.ayk_last_error()
    assert prefill(16) == 1
    # the window entry: positions required; more than 16 query heads per key/value head; a
    # partition size that is not a multiple of 64
    def windows(heads: int, positions: object = 1, size: int = 0) -> int:
        return lib.ayk_paged_attention_windows(1, 1, 1, 1, 1, 4, 1, 1, positions, 1, 2, 3, heads, 1, 128, 10, 16, 4,
                                               0, 1, 1, ctypes.c_float(1.0), 1.0, 1.0, size, None, 0, None)
    assert windows(8, positions=None) == 1 and b"positions are required" in lib.ayk_last_error()
    assert windows(32) == 2 and b"exceed a window's 16 columns" in lib.ayk_last_error()
    assert windows(8, size=96) == 1 and b"multiple of 64" in lib.ayk_last_error()
    assert prefill(32, size=96) == 1 and b"multiple of 64" in lib.ayk_last_error()
    assert prefill(64, size=64, workspace=16) == 4 and b"workspace" in lib.ayk_last_error()
    assert lib.ayk_reshape_and_cache(1, 1, 1, 1, 1, 3, 2, 64, 10, 16, 0, 3, None) == 2
    assert lib.ayk_reshape_and_cache_e4m3(1, 1, 1, 1, 1, 3, 2, 64, 10, 16, 0, 2, 1.0, 1.0, None) == 2
    assert b"src_dtype 2" in lib.ayk_last_error()
    assert lib.ayk_reshape_and_cache_e4m3(1, 1, 1, 1, 1, 0, 2, 64, 10, 16, 0, 1, 1.0, 1.0, None) == 0
    for k_scale, v_scale in ((0.0, 1.0), (1.0, -2.0), (float("inf"), 1.0), (1.0, float("nan"))):
        assert lib.ayk_reshape_and_cache_e4m3(1, 1, 1, 1, 1, 3, 2, 64, 10, 16, 0, 1, k_scale, v_scale, None) == 1
        assert b"positive and finite" in lib.ayk_last_error()
        assert _v1(lib, k_scale=k_scale, v_scale=v_scale) == 1 and b"positive and finite" in lib.ayk_last_error()
    assert lib.ayk_reshape_and_cache(1, 1, 1, 1, 1, 0, 2, 64, 10, 16, 0, 2, None) == 0
    assert lib.ayk_zero_blocks(1, 1, 1, 0, 2, 0, 64, None) == 1
