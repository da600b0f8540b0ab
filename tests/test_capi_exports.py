"""The C-ABI library loads and exports every symbol its header declares (CPU only)."""
import ctypes
import os

from mentat_amd import _lib


def test_library_is_built():
    assert os.path.exists(_lib.LIB_PATH), "run python -m mentat_amd.build first"


def test_exports_every_declared_symbol():
    lib = _lib.get_lib()
    declared = _lib.declared_symbols()
    assert declared, "no declarations parsed from include/mentat_capi.h"
    missing = [n for n in declared if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_every_declared_symbol_has_a_ctypes_signature():
    declared = set(_lib.declared_symbols())
    assert declared == set(_lib.SIGNATURES), (
        f"header-only: {sorted(declared - set(_lib.SIGNATURES))}, "
        f"binding-only: {sorted(set(_lib.SIGNATURES) - declared)}"
    )


def test_abi_version_and_pure_host_queries():
    lib = _lib.get_lib()
    assert lib.mentat_abi_version() >= 1
    # Pure host arithmetic: no device needed.
    assert lib.mentat_paged_decode_workspace_bytes(0, 0, 32, 8, 128, 16, 4096, 0, 0) == 0
    nb = lib.mentat_paged_decode_workspace_bytes(0, 64, 32, 8, 128, 16, 4096, 0, 256)
    assert nb == 262144 + 64 * 32 * 16 * (128 + 2) * 4  # reserved counters + partials
    # a window caps the attended span: 1024 tokens in chunks of 256 -> 4 chunks per sequence
    nw = lib.mentat_paged_decode_workspace_bytes(0, 64, 32, 8, 128, 16, 4096, 1024, 256)
    assert nw == 262144 + 64 * 32 * 4 * (128 + 2) * 4
    assert lib.mentat_paged_decode_workspace_bytes(0, 64, 32, 8, 128, 16, 4096, 8192, 256) == nb
    assert lib.mentat_paged_decode_workspace_bytes(0, 64, 32, 8, 128, 16, 4096, -1, 256) == 0
    assert lib.mentat_tree_decode_workspace_bytes(0, 32, 8, 128) == 0
    assert lib.mentat_tree_decode_workspace_bytes(10, 32, 8, 128) == 262144 + 10 * 4 * 130 * 4
    c = lib.mentat_paged_decode_auto_chunk(64, 8, 16, 4096)
    assert c % 16 == 0 and 16 <= c <= 4096
    assert isinstance(lib.mentat_paged_decode, ctypes._CFuncPtr)


def test_noalloc_entry_refuses_sizes_past_its_scratch():
    """The allocation-free decode checks its workspace need against the static
    scratch before touching the device (pure host arithmetic on the reference
    layout: 64 x 32 heads x 4096 chunks of partials are far past 8 MiB)."""
    lib = _lib.get_lib()
    need = lib.mentat_paged_decode_workspace_bytes(0, 64, 32, 8, 128, 16, 65536, 0, 16)
    assert need > 8388608
    st = lib.mentat_paged_decode_noalloc(0, None, None, None, None, 4096, None, None, None, 65536, None,
                                         64, 32, 8, 128, 16, 65536, 0, 0.088, 2, 16, None)
    assert st == _lib.MENTAT_ESPACE
    assert lib.mentat_paged_decode_noalloc(0, None, None, None, None, 1, None, None, None, 1, None,
                                           -1, 32, 8, 128, 16, 16, 0, 0.088, 2, 0, None) == _lib.MENTAT_EINVAL
    assert lib.mentat_paged_decode_noalloc(0, None, None, None, None, 1, None, None, None, 1, None,
                                           4, 32, 8, 128, 16, 16, -2, 0.088, 2, 0, None) == _lib.MENTAT_EINVAL
