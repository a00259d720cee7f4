"""ctypes mirror of the KVX C ABI and a loader for libkvx_amd.so.

The Structure classes reproduce include/kvx_abi.h field for field (reference
kvx_abi.h:26-188), so descriptors built here are byte-identical to those a C
caller builds.  The descriptor helpers mirror the helpers of the reference's
own tests (tests/kvx_abi_test.c:7-188, tests/kvx_kernel_test.cu:56-136): same
names, same canonical shapes and strides.

Data pointers are plain integers (device addresses for GPU buffers, e.g.
``tensor.data_ptr()`` of a torch CUDA tensor); nothing here allocates or
touches device memory.
"""
from __future__ import annotations

import ctypes as C
import enum
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libkvx_amd.so"

KVX_ABI_VERSION_MAJOR = 1
KVX_ABI_VERSION_MINOR = 1
KVX_MAX_TENSOR_DIMS = 5


class Status(enum.IntEnum):  # kvx_abi.h:26-33
    OK = 0
    INVALID_ARGUMENT = 1
    UNSUPPORTED = 2
    OUT_OF_RANGE = 3
    INCOMPATIBLE = 4
    INTERNAL_ERROR = 5


class DType(enum.IntEnum):  # kvx_abi.h:42-54
    INVALID = 0
    F16 = 1
    BF16 = 2
    F32 = 3
    F8_E4M3 = 4
    F8_E5M2 = 5
    S32 = 6
    S64 = 7
    U32 = 8
    U64 = 9
    U8 = 10


class Memory(enum.IntEnum):  # kvx_abi.h:56-61
    UNKNOWN = 0
    HOST = 1
    DEVICE = 2
    UNIFIED = 3


class Layout(enum.IntEnum):  # kvx_abi.h:63-69
    INVALID = 0
    BLOCK_NHD = 1
    BLOCK_HND = 2
    BLOCK_HND_PACKED = 3
    BLOCK_CUSTOM = 15


class TableFormat(enum.IntEnum):  # kvx_abi.h:103-108
    INVALID = 0
    PACKED = 1
    RAGGED = 2
    KV_OFFSETS = 3


TABLE_FLAG_KVCACHEINDEX = 1  # kvx_abi.h:110-113


class ScaleGranularity(enum.IntEnum):  # kvx_abi.h:154-160
    NONE = 0
    PER_TENSOR = 1
    PER_BLOCK = 2
    PER_HEAD = 3
    PER_BLOCK_HEAD = 4


DTYPE_SIZE = {DType.F16: 2, DType.BF16: 2, DType.F32: 4, DType.F8_E4M3: 1,
              DType.F8_E5M2: 1, DType.S32: 4, DType.S64: 8}

_i64x5 = C.c_int64 * KVX_MAX_TENSOR_DIMS


class Version(C.Structure):
    _fields_ = [("size", C.c_uint32), ("abi_major", C.c_uint32),
                ("abi_minor", C.c_uint32), ("abi_patch", C.c_uint32)]


class TensorDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_int), ("layout", C.c_int),
                ("memory", C.c_int), ("ndim", C.c_uint32), ("shape", _i64x5),
                ("stride", _i64x5), ("data", C.c_void_p)]


class PoolDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("memory", C.c_int),
                ("bytes_per_block", C.c_uint32), ("primary", C.c_void_p),
                ("secondary", C.c_void_p)]


class CacheDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("num_blocks", C.c_uint32),
                ("block_size", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32), ("k", TensorDesc), ("v", TensorDesc),
                ("pool", PoolDesc)]


class BlockTable(C.Structure):
    _fields_ = [("size", C.c_uint32), ("format", C.c_int),
                ("index_dtype", C.c_int), ("indptr_dtype", C.c_int),
                ("seq_count", C.c_uint32), ("beam_width", C.c_uint32),
                ("max_blocks_per_seq", C.c_uint32), ("indices", C.c_void_p),
                ("indptr", C.c_void_p), ("indices_count", C.c_uint32),
                ("indptr_count", C.c_uint32), ("flags", C.c_uint32)]


class SlotMapping(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_int),
                ("token_count", C.c_uint32), ("invalid_slot", C.c_int64),
                ("slots", C.c_void_p)]


class SeqLens(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_int),
                ("seq_count", C.c_uint32), ("lengths", C.c_void_p)]


class KvIoDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("key", TensorDesc), ("value", TensorDesc),
                ("num_tokens", C.c_uint32), ("num_kv_heads", C.c_uint32),
                ("head_dim", C.c_uint32)]


class ScaleDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("dtype", C.c_int), ("granularity", C.c_int),
                ("ndim", C.c_uint32), ("shape", _i64x5), ("stride", _i64x5),
                ("data", C.c_void_p)]


class PoolBlocks(C.Structure):  # kvx_ext.h: kvx_pool_blocks_t (no reference counterpart)
    _fields_ = [("size", C.c_uint32), ("reserved", C.c_uint32), ("primary", C.c_int64),
                ("secondary", C.c_int64)]


class WriteDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("io", KvIoDesc), ("slots", SlotMapping),
                ("k_scale", C.c_void_p), ("v_scale", C.c_void_p),
                ("k_scale_desc", ScaleDesc), ("v_scale_desc", ScaleDesc)]


class GatherDesc(C.Structure):
    _fields_ = [("size", C.c_uint32), ("io", KvIoDesc), ("block_table", BlockTable),
                ("seq_lens", SeqLens), ("max_seq_len", C.c_uint32)]


# Exported symbols and their argument lists (include/*.h).
_P = C.POINTER
_SIGS = {
    "kvx_get_version": [_P(Version)],
    "kvx_validate_cache_desc": [_P(CacheDesc)],
    "kvx_write_kv": [_P(CacheDesc), _P(WriteDesc), C.c_void_p],
    "kvx_gather_kv": [_P(CacheDesc), _P(GatherDesc), C.c_void_p],
    "kvx_launch_write_kv": [_P(CacheDesc), _P(WriteDesc), C.c_void_p],
    "kvx_launch_write_kv_prefill": [_P(CacheDesc), _P(WriteDesc), C.c_int32, C.c_void_p],
    "kvx_launch_gather_kv": [_P(CacheDesc), _P(GatherDesc), C.c_void_p],
    "kvx_launch_gather_kv_dequant": [_P(CacheDesc), _P(GatherDesc), _P(ScaleDesc),
                                     _P(ScaleDesc), C.c_void_p],
    "kvx_launch_gather_kv_pools": [_P(CacheDesc), _P(GatherDesc), _P(PoolBlocks), _P(ScaleDesc),
                                   _P(ScaleDesc), C.c_void_p],
}
for _t in ("f32", "f16", "bf16"):
    _SIGS[f"kvx_launch_write_kv_{_t}"] = [_P(CacheDesc), _P(WriteDesc), C.c_void_p]
    _SIGS[f"kvx_launch_write_kv_prefill_{_t}"] = [_P(CacheDesc), _P(WriteDesc),
                                                  C.c_int32, C.c_void_p]
    _SIGS[f"kvx_launch_gather_kv_{_t}"] = [_P(CacheDesc), _P(GatherDesc), C.c_void_p]

EXPORTED_SYMBOLS = tuple(sorted(_SIGS))

_LIB = None


def load(path: str | os.PathLike | None = None) -> C.CDLL:
    """Load libkvx_amd.so.  Raises if it has not been built: there is no
    fallback implementation."""
    global _LIB
    if path is None and _LIB is not None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(f"{p} is missing; build it with `python -m kvx_amd.build`")
    lib = C.CDLL(str(p))
    for name, args in _SIGS.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    if path is None:
        _LIB = lib
    return lib


def bind_like(lib: C.CDLL) -> C.CDLL:
    """Give another library with the same ABI (e.g. the compiled reference
    kvx_abi.c) the argument types of the functions it exports."""
    for name, args in _SIGS.items():
        fn = getattr(lib, name, None)
        if fn is not None:
            fn.argtypes = args
            fn.restype = C.c_int
    return lib


# ---------------------------------------------------------------------------
# Descriptor helpers (canonical strides, reference tests' conventions).

def _tensor(dtype, layout, memory, shape, stride, data) -> TensorDesc:
    t = TensorDesc()
    t.size = C.sizeof(TensorDesc)
    t.dtype = int(dtype)
    t.layout = int(layout)
    t.memory = int(memory)
    t.ndim = len(shape)
    for i, (n, s) in enumerate(zip(shape, stride)):
        t.shape[i] = int(n)
        t.stride[i] = int(s)
    t.data = data
    return t


def cache_tensor(layout, dtype, memory, num_blocks, block_size, heads, head_dim,
                 data, pack: int = 8) -> TensorDesc:
    """Canonical paged cache tensor (KVX_SPEC.md:50-75)."""
    layout = Layout(layout)
    if layout == Layout.BLOCK_NHD:
        shape = (num_blocks, block_size, heads, head_dim)
    elif layout == Layout.BLOCK_HND:
        shape = (num_blocks, heads, block_size, head_dim)
    elif layout == Layout.BLOCK_HND_PACKED:
        shape = (num_blocks, heads, head_dim // pack, block_size, pack)
    else:
        raise ValueError(layout)
    return _tensor(dtype, layout, memory, shape, contiguous_strides(shape), data)


def contiguous_strides(shape) -> tuple:
    st, acc = [], 1
    for n in reversed(shape):
        st.append(acc)
        acc *= int(n)
    return tuple(reversed(st))


def token_tensor(dtype, memory, num_tokens, heads, head_dim, data) -> TensorDesc:
    """[num_tokens, H, D] io tensor (tests/kvx_abi_test.c:54-71)."""
    shape = (num_tokens, heads, head_dim)
    return _tensor(dtype, Layout.BLOCK_CUSTOM, memory, shape, contiguous_strides(shape),
                   data)


def seq_tensor(dtype, memory, seq_count, max_seq_len, heads, head_dim, data) -> TensorDesc:
    """[seq_count, max_seq_len, H, D] io tensor (tests/kvx_abi_test.c:73-92)."""
    shape = (seq_count, max_seq_len, heads, head_dim)
    return _tensor(dtype, Layout.BLOCK_CUSTOM, memory, shape, contiguous_strides(shape),
                   data)


def cache_desc(num_blocks, block_size, heads, head_dim, k: TensorDesc,
               v: TensorDesc) -> CacheDesc:
    c = CacheDesc()
    c.size = C.sizeof(CacheDesc)
    c.num_blocks = num_blocks
    c.block_size = block_size
    c.num_kv_heads = heads
    c.head_dim = head_dim
    c.k = k
    c.v = v
    return c


def make_cache(layout, dtype, memory, num_blocks, block_size, heads, head_dim, k_data,
               v_data, pack: int = 8, v_layout=None) -> CacheDesc:
    """Cache descriptor with canonical K and V tensors; `v_layout` lets V use
    a different layout from K (accepted on the launch path)."""
    v_layout = layout if v_layout is None else v_layout
    k = cache_tensor(layout, dtype, memory, num_blocks, block_size, heads, head_dim,
                     k_data, pack)
    v = cache_tensor(v_layout, dtype, memory, num_blocks, block_size, heads, head_dim,
                     v_data, pack)
    return cache_desc(num_blocks, block_size, heads, head_dim, k, v)


def make_write(num_tokens, heads, head_dim, dtype, memory, key_data, value_data,
               slots_dtype, slots_data, k_scale=None, v_scale=None) -> WriteDesc:
    """Write descriptor (tests/kvx_abi_test.c:114-136)."""
    w = WriteDesc()
    w.size = C.sizeof(WriteDesc)
    w.io.size = C.sizeof(KvIoDesc)
    w.io.num_tokens = num_tokens
    w.io.num_kv_heads = heads
    w.io.head_dim = head_dim
    w.io.key = token_tensor(dtype, memory, num_tokens, heads, head_dim, key_data)
    w.io.value = token_tensor(dtype, memory, num_tokens, heads, head_dim, value_data)
    w.slots.size = C.sizeof(SlotMapping)
    w.slots.dtype = int(slots_dtype)
    w.slots.token_count = num_tokens
    w.slots.invalid_slot = -1
    w.slots.slots = slots_data
    w.k_scale = k_scale
    w.v_scale = v_scale
    return w


def scale_desc(data, dtype=DType.F32, granularity=ScaleGranularity.PER_TENSOR,
               shape=(1,), stride=None) -> ScaleDesc:
    """kvx_scale_desc_t.  Shapes this build accepts (strides in elements,
    contiguous by default): PER_TENSOR any; PER_HEAD [num_kv_heads];
    PER_BLOCK [num_blocks]; PER_BLOCK_HEAD [num_blocks, num_kv_heads]."""
    s = ScaleDesc()
    s.size = C.sizeof(ScaleDesc)
    s.dtype = int(dtype)
    s.granularity = int(granularity)
    shape = tuple(int(x) for x in shape)
    stride = contiguous_strides(shape) if stride is None else tuple(int(x) for x in stride)
    s.ndim = len(shape)
    for i, (n, st) in enumerate(zip(shape, stride)):
        s.shape[i] = n
        s.stride[i] = st
    s.data = data
    return s


def make_block_table_packed(seq_count, max_blocks_per_seq, index_dtype,
                            indices) -> BlockTable:
    """PACKED table (tests/kvx_abi_test.c:138-156)."""
    t = BlockTable()
    t.size = C.sizeof(BlockTable)
    t.format = int(TableFormat.PACKED)
    t.index_dtype = int(index_dtype)
    t.seq_count = seq_count
    t.beam_width = 1
    t.max_blocks_per_seq = max_blocks_per_seq
    t.indices = indices
    t.indices_count = seq_count * max_blocks_per_seq
    return t


def make_seq_lens(seq_count, dtype, lengths) -> SeqLens:
    s = SeqLens()
    s.size = C.sizeof(SeqLens)
    s.dtype = int(dtype)
    s.seq_count = seq_count
    s.lengths = lengths
    return s


def make_gather(seq_count, max_seq_len, heads, head_dim, dtype, memory, key_out,
                value_out, table: BlockTable, seq_lens: SeqLens) -> GatherDesc:
    """Gather descriptor (tests/kvx_abi_test.c:169-188)."""
    g = GatherDesc()
    g.size = C.sizeof(GatherDesc)
    g.io.size = C.sizeof(KvIoDesc)
    g.io.num_tokens = seq_count * max_seq_len
    g.io.num_kv_heads = heads
    g.io.head_dim = head_dim
    g.io.key = seq_tensor(dtype, memory, seq_count, max_seq_len, heads, head_dim,
                          key_out)
    g.io.value = seq_tensor(dtype, memory, seq_count, max_seq_len, heads, head_dim,
                            value_out)
    g.block_table = table
    g.seq_lens = seq_lens
    g.max_seq_len = max_seq_len
    return g


def ref(x):
    """ctypes pointer to a descriptor (None passes NULL)."""
    return None if x is None else C.byref(x)
