"""The C-ABI boundary: struct layout and exported symbols (CPU only).

Sizes and offsets are the LP64 layout of the reference kvx_abi.h:73-188
(computed from the reference header with gcc); the library must export every
entry point that include/*.h declares and nothing else.
"""
import ctypes as C
import re
import subprocess

from kvx_amd import abi

from conftest import REPO

SIZES = {
    abi.Version: 16, abi.TensorDesc: 112, abi.PoolDesc: 32, abi.CacheDesc: 280,
    abi.BlockTable: 64, abi.SlotMapping: 32, abi.SeqLens: 24, abi.KvIoDesc: 248,
    abi.ScaleDesc: 104, abi.WriteDesc: 512, abi.GatherDesc: 352,
    abi.PoolBlocks: 24,  # kvx_ext.h
}

OFFSETS = [
    (abi.CacheDesc, "k", 24), (abi.CacheDesc, "v", 136), (abi.CacheDesc, "pool", 248),
    (abi.WriteDesc, "slots", 256), (abi.WriteDesc, "k_scale", 288),
    (abi.WriteDesc, "k_scale_desc", 304), (abi.GatherDesc, "block_table", 256),
    (abi.GatherDesc, "seq_lens", 320), (abi.GatherDesc, "max_seq_len", 344),
    (abi.TensorDesc, "shape", 24), (abi.TensorDesc, "stride", 64),
    (abi.TensorDesc, "data", 104),
    (abi.PoolBlocks, "primary", 8), (abi.PoolBlocks, "secondary", 16),
]


def test_struct_sizes():
    for cls, size in SIZES.items():
        assert C.sizeof(cls) == size, cls.__name__


def test_struct_offsets():
    for cls, field, off in OFFSETS:
        assert getattr(cls, field).offset == off, (cls.__name__, field)


def _declared_symbols():
    names = set()
    for h in (REPO / "include").glob("*.h"):
        text = h.read_text()
        names |= set(re.findall(r"KVX_API\s+kvx_status_t\s+(kvx_\w+)\s*\(", text))
    return names


def test_headers_declare_expected_entry_points():
    assert _declared_symbols() == set(abi.EXPORTED_SYMBOLS)


def test_library_exports_exactly_the_declared_symbols(kvx_lib):
    for name in _declared_symbols():
        assert hasattr(kvx_lib, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", str(abi.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = {l.split()[-1] for l in out.splitlines() if " T " in l}
    assert exported == _declared_symbols()


def test_version(kvx_lib):
    v = abi.Version()
    assert kvx_lib.kvx_get_version(C.byref(v)) == abi.Status.OK
    assert (v.size, v.abi_major, v.abi_minor, v.abi_patch) == (16, 1, 1, 0)
    assert kvx_lib.kvx_get_version(None) == abi.Status.INVALID_ARGUMENT


def test_header_compiles_as_c_and_matches_reference_layout(tmp_path):
    """A C11 translation unit including include/kvx_abi.h and kvx_ext.h
    compiles, with the sizes above asserted at compile time."""
    src = tmp_path / "layout.c"
    asserts = "\n".join(
        f"_Static_assert(sizeof({t}) == {n}, \"{t}\");"
        for t, n in [("kvx_tensor_desc_t", 112), ("kvx_cache_desc_t", 280),
                     ("kvx_write_desc_t", 512), ("kvx_gather_desc_t", 352),
                     ("kvx_scale_desc_t", 104), ("kvx_block_table_t", 64)])
    src.write_text('#include "kvx_paged_kv.h"\n#include "kvx_ext.h"\n' + asserts + "\n")
    subprocess.run(["gcc", "-std=c11", "-Wall", "-Werror", "-fsyntax-only",
                    f"-I{REPO / 'include'}", str(src)], check=True)
