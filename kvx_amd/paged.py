"""Torch-facing host helpers over the KVX C ABI.

These build kvx_abi.h descriptors from torch tensors (shape, element strides,
data pointer, memory type) and call libkvx_amd.so through ctypes.  torch is
only the source of device memory and streams here; every byte is moved by the
library's HIP kernels.  There is no fallback: if libkvx_amd.so is missing,
``abi.load()`` raises.

The calls mirror the reference's launch API (kernels/kvx_paged_kv.h:11-21):
``write_kv`` -> kvx_launch_write_kv / kvx_launch_write_kv_prefill,
``gather_kv`` -> kvx_launch_gather_kv / kvx_launch_gather_kv_dequant, and
return the kvx_status_t as ``abi.Status``.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass

import torch

from . import abi
from .abi import DType, Layout, Memory, Status

_TORCH_DTYPE = {
    torch.float16: DType.F16,
    torch.bfloat16: DType.BF16,
    torch.float32: DType.F32,
    torch.float8_e4m3fn: DType.F8_E4M3,
    torch.float8_e5m2: DType.F8_E5M2,
    torch.int32: DType.S32,
    torch.int64: DType.S64,
}


def dtype_code(t: torch.Tensor | torch.dtype) -> DType:
    dt = t.dtype if isinstance(t, torch.Tensor) else t
    if dt not in _TORCH_DTYPE:
        raise ValueError(f"unsupported dtype {dt}")
    return _TORCH_DTYPE[dt]


def memory_of(t: torch.Tensor) -> Memory:
    return Memory.DEVICE if t.is_cuda else Memory.HOST


def tensor_desc(t: torch.Tensor, layout: Layout = Layout.BLOCK_CUSTOM,
                dtype: DType | None = None) -> abi.TensorDesc:
    """Descriptor of `t` as laid out in memory (its own shape and strides)."""
    d = abi.TensorDesc()
    d.size = C.sizeof(abi.TensorDesc)
    d.dtype = int(dtype if dtype is not None else dtype_code(t))
    d.layout = int(layout)
    d.memory = int(memory_of(t))
    d.ndim = t.dim()
    for i in range(t.dim()):
        d.shape[i] = t.shape[i]
        d.stride[i] = t.stride(i)
    d.data = t.data_ptr()
    return d


def cache_shape(layout: Layout, num_blocks: int, block_size: int, heads: int,
                head_dim: int, pack: int = 8) -> tuple:
    """Canonical shape of a cache tensor in `layout` (KVX_SPEC.md:50-56)."""
    layout = Layout(layout)
    if layout == Layout.BLOCK_NHD:
        return (num_blocks, block_size, heads, head_dim)
    if layout == Layout.BLOCK_HND:
        return (num_blocks, heads, block_size, head_dim)
    if layout == Layout.BLOCK_HND_PACKED:
        return (num_blocks, heads, head_dim // pack, block_size, pack)
    raise ValueError(layout)


@dataclass
class PagedCache:
    """K and V cache tensors and the kvx_cache_desc_t describing them."""

    key_cache: torch.Tensor
    value_cache: torch.Tensor
    k_layout: Layout
    v_layout: Layout
    num_blocks: int
    block_size: int
    heads: int
    head_dim: int

    def desc(self) -> abi.CacheDesc:
        k = tensor_desc(self.key_cache, self.k_layout)
        v = tensor_desc(self.value_cache, self.v_layout)
        return abi.cache_desc(self.num_blocks, self.block_size, self.heads,
                              self.head_dim, k, v)


def alloc_cache(num_blocks: int, block_size: int, heads: int, head_dim: int,
                dtype: torch.dtype, device, k_layout=Layout.BLOCK_NHD,
                v_layout=None, pack: int = 8) -> PagedCache:
    v_layout = k_layout if v_layout is None else v_layout
    k = torch.empty(cache_shape(k_layout, num_blocks, block_size, heads, head_dim, pack),
                    dtype=dtype, device=device)
    v = torch.empty(cache_shape(v_layout, num_blocks, block_size, heads, head_dim, pack),
                    dtype=dtype, device=device)
    return PagedCache(k, v, Layout(k_layout), Layout(v_layout), num_blocks, block_size,
                      heads, head_dim)


def custom_view(storage: torch.Tensor, order: str) -> torch.Tensor:
    """The logical CUSTOM view of a cache `storage` whose axes are named by
    `order`: a permutation of "bohd" (block, offset, head, dim) or "bohpx"
    (dim split as dim / x, x).  E.g. order "bhdo" is vLLM's value cache
    [num_blocks, H, D, block_size]."""
    logical = "bohpx" if len(order) == 5 else "bohd"
    if sorted(order) != sorted(logical):
        raise ValueError(f"order {order!r} is not a permutation of {logical!r}")
    return storage.permute([order.index(a) for a in logical])


def alloc_custom_cache(num_blocks: int, block_size: int, heads: int, head_dim: int,
                       dtype: torch.dtype, device, k_order: str = "bhdo",
                       v_order: str | None = None, x: int = 8) -> PagedCache:
    """K and V caches in KVX_LAYOUT_BLOCK_CUSTOM with storage axis orders
    k_order / v_order (see custom_view; 5-letter orders split dim by x)."""
    v_order = k_order if v_order is None else v_order

    def one(order):
        size = {"b": num_blocks, "o": block_size, "h": heads, "d": head_dim,
                "p": head_dim // x, "x": x}
        t = torch.empty([size[a] for a in order], dtype=dtype, device=device)
        return custom_view(t, order)

    return PagedCache(one(k_order), one(v_order), Layout.BLOCK_CUSTOM, Layout.BLOCK_CUSTOM,
                      num_blocks, block_size, heads, head_dim)


def alloc_block_pool(num_blocks: int, block_size: int, heads: int, head_dim: int,
                     dtype: torch.dtype, device, layout=Layout.BLOCK_NHD,
                     pack: int = 8) -> tuple[PagedCache, PagedCache]:
    """One pool of 2 * num_blocks single-tensor blocks in TensorRT-LLM's
    KVBlockArray pairing: the K block of logical block b is pool block 2b, its
    V block is 2b + 1.  Returns (pool, kv): `pool` describes all pool blocks
    (the cache for KV_OFFSETS gathers, whose OffsetsTable is
    ``pool_table``); `kv` views the same memory as K and V caches of
    num_blocks blocks for PACKED-table writes and gathers."""
    shape = cache_shape(layout, 2 * num_blocks, block_size, heads, head_dim, pack)
    mem = torch.empty(shape, dtype=dtype, device=device)
    layout = Layout(layout)
    pool = PagedCache(mem, mem, layout, layout, 2 * num_blocks, block_size, heads, head_dim)
    kv = PagedCache(mem[0::2], mem[1::2], layout, layout, num_blocks, block_size, heads,
                    head_dim)
    return pool, kv


def pool_table(pool: PagedCache, offsets: torch.Tensor,
               secondary: torch.Tensor | None = None) -> "OffsetsTable":
    """OffsetsTable over the memory of `pool` (see alloc_block_pool)."""
    mem = pool.key_cache
    return OffsetsTable(offsets, mem, secondary, mem.stride(0) * mem.element_size())


def _stream_handle(stream) -> int | None:
    if stream is None:
        return torch.cuda.current_stream().cuda_stream if torch.cuda.is_available() else None
    if isinstance(stream, torch.cuda.Stream):
        return stream.cuda_stream
    return int(stream)


@dataclass
class Scales:
    """FP8 scales of one tensor with a granularity: `values` is a float32
    device tensor of shape [1] (PER_TENSOR), [num_kv_heads] (PER_HEAD),
    [num_blocks] (PER_BLOCK, by physical block id) or [num_blocks,
    num_kv_heads] (PER_BLOCK_HEAD); its own strides are passed."""

    values: torch.Tensor
    granularity: abi.ScaleGranularity = abi.ScaleGranularity.PER_TENSOR


def scale_desc_of(scale) -> abi.ScaleDesc:
    """kvx_scale_desc_t for a one-element float32 tensor (per tensor) or a
    Scales."""
    if isinstance(scale, Scales):
        v = scale.values
        shape = tuple(v.shape) or (1,)
        stride = tuple(v.stride()) or (1,)
        return abi.scale_desc(v.data_ptr(), granularity=scale.granularity, shape=shape,
                              stride=stride)
    return abi.scale_desc(scale.data_ptr())


def build_write(cache: PagedCache, key: torch.Tensor, value: torch.Tensor,
                slot_mapping: torch.Tensor, k_scale=None, v_scale=None) -> abi.WriteDesc:
    """kvx_write_desc_t for [T, H, D] key/value rows and [T] slots.  FP8
    scales are one-element F32 device tensors, passed as PER_TENSOR scale
    descriptors."""
    T = key.shape[0]
    w = abi.WriteDesc()
    w.size = C.sizeof(abi.WriteDesc)
    w.io.size = C.sizeof(abi.KvIoDesc)
    w.io.key = tensor_desc(key)
    w.io.value = tensor_desc(value)
    w.io.num_tokens = T
    w.io.num_kv_heads = key.shape[1] if key.dim() == 3 else 0
    w.io.head_dim = key.shape[2] if key.dim() == 3 else 0
    w.slots.size = C.sizeof(abi.SlotMapping)
    w.slots.dtype = int(dtype_code(slot_mapping))
    w.slots.token_count = slot_mapping.numel()
    w.slots.invalid_slot = -1
    w.slots.slots = slot_mapping.data_ptr()
    if k_scale is not None:
        w.k_scale_desc = scale_desc_of(k_scale)
    if v_scale is not None:
        w.v_scale_desc = scale_desc_of(v_scale)
    return w


@dataclass
class RaggedTable:
    """RAGGED block table (KVX_SPEC.md:107-114): token t of sequence s is
    cached in block ``indices[indptr[s] + t]`` at offset ``t % block_size``,
    for t < indptr[s+1] - indptr[s]."""

    indices: torch.Tensor  # [total tokens] int32 / int64 block ids
    indptr: torch.Tensor   # [seq_count + 1] int32 / int64 prefix sums


@dataclass
class OffsetsTable:
    """KV_OFFSETS block table (KVX_SPEC.md:116-122, TensorRT-LLM's
    KVBlockArray): int32 ``offsets[s, 0, 0 (K) / 1 (V), j]`` are KVCacheIndex
    values; block j of sequence s lives at ``pool + (value & 0x7FFFFFFF) *
    bytes_per_block`` with bit 31 choosing the secondary pool.  The cache's K
    / V tensors give only the in-block layout."""

    offsets: torch.Tensor              # int32 [seq_count, 1, 2, max_blocks_per_seq]
    primary: torch.Tensor              # pool storage (its bytes)
    secondary: torch.Tensor | None
    bytes_per_block: int


def kv_cache_index(block: int, secondary: bool = False) -> int:
    """The int32 KVCacheIndex value for `block` in the primary or secondary
    pool (KV_CACHE_LAYOUTS.md:91-92)."""
    v = (int(block) & 0x7FFFFFFF) | (0x80000000 if secondary else 0)
    return v - (1 << 32) if v >= 0x80000000 else v


def _table_desc(table) -> abi.BlockTable:
    if isinstance(table, RaggedTable):
        t = abi.BlockTable()
        t.size = C.sizeof(abi.BlockTable)
        t.format = int(abi.TableFormat.RAGGED)
        t.index_dtype = int(dtype_code(table.indices))
        t.indptr_dtype = int(dtype_code(table.indptr))
        t.seq_count = table.indptr.numel() - 1
        t.beam_width = 1
        t.max_blocks_per_seq = 1  # not used by RAGGED; the ABI path requires > 0
        t.indices = table.indices.data_ptr()
        t.indptr = table.indptr.data_ptr()
        t.indices_count = table.indices.numel()
        t.indptr_count = table.indptr.numel()
        return t
    if isinstance(table, OffsetsTable):
        S, beam, two, mbps = table.offsets.shape
        if two != 2 or table.offsets.dtype != torch.int32:
            raise ValueError("KV_OFFSETS table is int32 [seq_count, beam, 2, max_blocks]")
        t = abi.BlockTable()
        t.size = C.sizeof(abi.BlockTable)
        t.format = int(abi.TableFormat.KV_OFFSETS)
        t.index_dtype = int(DType.S32)
        t.seq_count = S
        t.beam_width = beam
        t.max_blocks_per_seq = mbps
        t.indices = table.offsets.data_ptr()
        t.indices_count = table.offsets.numel()
        t.flags = abi.TABLE_FLAG_KVCACHEINDEX
        return t
    S, mbps = table.shape
    return abi.make_block_table_packed(S, mbps, dtype_code(table), table.data_ptr())


def gather_cache_desc(cache: PagedCache, block_table) -> abi.CacheDesc:
    """The cache descriptor of a gather; an OffsetsTable also fills its pool
    fields (kvx_pool_desc_t)."""
    cd = cache.desc()
    if isinstance(block_table, OffsetsTable):
        cd.pool.size = C.sizeof(abi.PoolDesc)
        cd.pool.memory = int(memory_of(block_table.primary))
        cd.pool.bytes_per_block = block_table.bytes_per_block
        cd.pool.primary = block_table.primary.data_ptr()
        cd.pool.secondary = (None if block_table.secondary is None
                             else block_table.secondary.data_ptr())
    return cd


def build_gather(key_out: torch.Tensor, value_out: torch.Tensor,
                 block_table, seq_lens: torch.Tensor,
                 max_seq_len: int) -> abi.GatherDesc:
    """kvx_gather_desc_t for [S, max_seq_len, H, D] outputs.  `block_table` is
    a [S, max_blocks_per_seq] tensor (PACKED), a RaggedTable or an
    OffsetsTable."""
    tb = _table_desc(block_table)
    S = tb.seq_count
    g = abi.GatherDesc()
    g.size = C.sizeof(abi.GatherDesc)
    g.io.size = C.sizeof(abi.KvIoDesc)
    g.io.key = tensor_desc(key_out)
    g.io.value = tensor_desc(value_out)
    g.io.num_tokens = S * max_seq_len
    g.io.num_kv_heads = key_out.shape[2]
    g.io.head_dim = key_out.shape[3]
    g.block_table = tb
    g.seq_lens = abi.make_seq_lens(seq_lens.numel(), dtype_code(seq_lens),
                                   seq_lens.data_ptr())
    g.max_seq_len = max_seq_len
    return g


def write_kv(cache: PagedCache, key: torch.Tensor, value: torch.Tensor,
             slot_mapping: torch.Tensor, *, tokens_per_seq: int | None = None,
             k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
             stream=None, entry: str = "launch") -> Status:
    """Scatter rows into the paged cache.  entry = "launch" (kvx_paged_kv.h)
    or "abi" (kvx_write_kv of kvx_abi.h)."""
    lib = abi.load()
    cd = cache.desc()
    wd = build_write(cache, key, value, slot_mapping, k_scale, v_scale)
    s = _stream_handle(stream)
    if entry == "abi":
        return Status(lib.kvx_write_kv(C.byref(cd), C.byref(wd), s))
    if tokens_per_seq is not None:
        return Status(lib.kvx_launch_write_kv_prefill(C.byref(cd), C.byref(wd),
                                                      tokens_per_seq, s))
    return Status(lib.kvx_launch_write_kv(C.byref(cd), C.byref(wd), s))


def gather_kv(cache: PagedCache, key_out: torch.Tensor, value_out: torch.Tensor,
              block_table, seq_lens: torch.Tensor, max_seq_len: int, *,
              k_scale: torch.Tensor | None = None, v_scale: torch.Tensor | None = None,
              stream=None, entry: str = "launch",
              pool_blocks: tuple[int, int] | None = None) -> Status:
    """Gather sequences into contiguous [S, max_seq_len, H, D] buffers.
    `block_table` is a PACKED [S, max_blocks_per_seq] tensor, a RaggedTable
    or an OffsetsTable (whose pool replaces the cache tensors' data).
    With k_scale/v_scale the FP8 cache is dequantized
    (kvx_launch_gather_kv_dequant).  pool_blocks = (primary, secondary)
    block counts go through kvx_launch_gather_kv_pools instead."""
    lib = abi.load()
    cd = gather_cache_desc(cache, block_table)
    gd = build_gather(key_out, value_out, block_table, seq_lens, max_seq_len)
    s = _stream_handle(stream)
    if entry == "abi":
        return Status(lib.kvx_gather_kv(C.byref(cd), C.byref(gd), s))
    if pool_blocks is not None:
        pb = abi.PoolBlocks(C.sizeof(abi.PoolBlocks), 0, pool_blocks[0], pool_blocks[1])
        ks = vs = None
        if k_scale is not None or v_scale is not None:
            ks, vs = C.byref(scale_desc_of(k_scale)), C.byref(scale_desc_of(v_scale))
        return Status(lib.kvx_launch_gather_kv_pools(C.byref(cd), C.byref(gd), C.byref(pb), ks,
                                                     vs, s))
    if k_scale is not None or v_scale is not None:
        ks = scale_desc_of(k_scale)
        vs = scale_desc_of(v_scale)
        return Status(lib.kvx_launch_gather_kv_dequant(C.byref(cd), C.byref(gd),
                                                       C.byref(ks), C.byref(vs), s))
    return Status(lib.kvx_launch_gather_kv(C.byref(cd), C.byref(gd), s))
