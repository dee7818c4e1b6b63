"""The C-ABI library loads without a GPU and exports every symbol include/peco_hip.h declares."""
import ctypes
import re
import subprocess
from pathlib import Path

from peco_amd import _native

HEADER = Path(__file__).resolve().parents[1] / "include" / "peco_hip.h"


def _declared():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(peco_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_reference_symbols():
    names = _declared()
    for ref in ("peco_assign_tokens_to_centers", "peco_recompute_cluster_centers", "peco_reorder_token_features",
                "peco_cluster_error_message", "peco_sparse_attention", "peco_attention_error_string"):
        assert ref in names


def test_library_exports_every_declared_symbol():
    if not _native.LIB_PATH.exists():
        _native.build_library()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_native.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    exported = set(re.findall(r" T (peco_\w+)", out))
    missing = [n for n in _declared() if n not in exported]
    assert not missing, f"declared but not exported: {missing}"
    assert set(_native.SIGNATURES) == set(_declared())


def test_library_loads_and_reports_status_strings_without_a_gpu():
    lib = _native.library()
    assert lib.peco_abi_version() == 5
    assert b"workspace" in lib.peco_cluster_error_message(20001)
    assert lib.peco_attention_error_string(0)
    # Size queries are host-only arithmetic.
    assert lib.peco_sparse_attention_workspace_size(24, 7006, 7006, 66, 258) <= 24 * (258 + 2 + 3 * (438 + 66))
    assert lib.peco_kmeans_workspace_size(24, 6750, 256, 128) > 0
    assert lib.peco_cluster_sort_workspace_size(24, 6750, 256) > 0


def test_invalid_arguments_are_rejected_before_any_launch():
    lib = _native.library()
    null = ctypes.c_void_p(0)
    assert lib.peco_reorder_token_features(null, null, null, 1, 4, 8, 3, 0, null) == 1
    assert lib.peco_sparse_attention(null, null, null, null, null, null, null, null, 1, 4, 4, 96, 1, 1, 1,
                                     null) == 1
    assert lib.peco_cluster_sort(null, 1, 4, 2, null, null, null, null, null, 0, null) == 1


def test_work_list_entries_reject_bad_arguments_and_size_the_buffer():
    lib = _native.library()
    null = ctypes.c_void_p(0)
    # 24 heads, 7006 rows, a 66 x 258 extended map: counters, counts, row lengths, items
    # (55 + 66 per head, 3 ints each), 16 queue counters, then 8-byte aligned segment rows of
    # 260 int2.
    head = 2 * 24 + 24 * 66 + 24 * (55 + 66) * 3 + 16
    head += head & 1
    assert lib.peco_select_work_size(24, 7006, 64, 256, 1) == head + 24 * 66 * 260 * 2
    assert lib.peco_select_work_size(0, 7006, 64, 256, 1) == 0
    assert lib.peco_select_work(null, null, null, null, 1, 4, 4, 128, 0.5, 0, 0, 0, 0, 16, 16, null, null, null,
                                null, 1 << 20, null) == 1
    assert lib.peco_sparse_attention_work(null, null, null, null, null, 0, null, null, 0, 0, null, 0, 1, 16, 16, 128,
                                          4, 4, 1, null) == 1


def test_base_offset_attention_rejects_bad_arguments():
    lib = _native.library()
    null = ctypes.c_void_p(0)
    args = [null, null, null, 4, null, null, null, null, null, null, null, null, null, 8, 4, null, null, null, null,
            null, 1 << 20, 1, 64, 64, 60, 128, 6, 10, 1, null]
    assert lib.peco_base_offset_attention(*args) == 1


def test_library_leaves_no_own_symbol_undefined():
    """A kernel whose host stub was not emitted leaves an undefined symbol that only fails at
    load time on the GPU host; catch it here."""
    if not _native.LIB_PATH.exists():
        _native.build_library()
    out = subprocess.run(["nm", "-D", "--undefined-only", str(_native.LIB_PATH)], capture_output=True, text=True,
                         check=True).stdout
    own = [line for line in out.splitlines() if "peco" in line]
    assert not own, f"undefined symbols of the library's own code: {own}"
