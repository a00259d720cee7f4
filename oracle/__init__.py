"""Python access to the CPU oracle (oracle/kvx_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker and the timed CPU baseline.  The
product (kvx_amd) never imports it.

Buffers are numpy arrays (C-contiguous, any element type: they are passed as
raw bytes).  Layout and dtype codes are the kvx_abi.h enum values.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

from . import build as _build

_LIB = None
_I64P = C.POINTER(C.c_int64)


class _ScaleT(C.Structure):
    _fields_ = [("p", C.c_void_p), ("s_block", C.c_int64), ("s_head", C.c_int64)]


class Scale:
    """FP8 scales of one tensor: the scale of (block b, head h) is
    values.flat[b * s_block + h * s_head].  A float is a per-tensor scale."""

    def __init__(self, values, s_block: int = 0, s_head: int = 0):
        self.values = np.ascontiguousarray(values, dtype=np.float32).reshape(-1)
        self.s_block = int(s_block)
        self.s_head = int(s_head)

    @classmethod
    def per_head(cls, values):
        return cls(values, 0, 1)

    @classmethod
    def per_block(cls, values):
        return cls(values, 1, 0)

    @classmethod
    def per_block_head(cls, values):
        v = np.asarray(values, dtype=np.float32)
        return cls(v, v.shape[1], 1)


def _scale_arg(x):
    """(keep-alive, pointer) for a float / Scale / None scale."""
    if x is None:
        return None, None
    if not isinstance(x, Scale):
        x = Scale([float(x)])
    st = _ScaleT(x.values.ctypes.data, x.s_block, x.s_head)
    return (x, st), C.pointer(st)


def lib() -> C.CDLL:
    global _LIB
    if _LIB is None:
        if not _build.ORACLE_LIB.exists():
            _build.build_oracle()
        L = C.CDLL(str(_build.ORACLE_LIB))
        vp, i32, i64, f32, i = C.c_void_p, C.c_int32, C.c_int64, C.c_float, C.c_int
        geom = [i, _I64P, i64]
        L.oracle_cache_offset.argtypes = [i, _I64P, i64, i64, i64, i64, i64]
        L.oracle_cache_offset.restype = i64
        sp = C.POINTER(_ScaleT)
        L.oracle_write_kv.argtypes = geom + geom + [vp, vp, vp, vp, vp, i, i64, i32, i32,
                                                    i32, i32, i, i, sp, sp]
        L.oracle_gather_kv.argtypes = geom + geom + [vp, vp, vp, vp, vp, vp, i, i32, i32,
                                                     i32, i32, i32, i32, i32, i, i, sp, sp]
        L.oracle_write_kv_fast.argtypes = geom + geom + [vp, vp, vp, vp, vp, i, i64, i32,
                                                         i32, i32, i32, i]
        L.oracle_write_kv_fast.restype = i
        L.oracle_gather_kv_fast.argtypes = geom + geom + [vp, vp, vp, vp, vp, vp, i, i32,
                                                          i32, i32, i32, i32, i32, i32, i]
        L.oracle_gather_kv_fast.restype = i
        L.oracle_write_kv_quant_fast.argtypes = geom + geom + [vp, vp, vp, vp, vp, i, i64,
                                                               i32, i32, i32, i32, i, i, f32,
                                                               f32]
        L.oracle_write_kv_quant_fast.restype = i
        L.oracle_gather_kv_dequant_fast.argtypes = geom + geom + [vp, vp, vp, vp, vp, vp, i,
                                                                  i32, i32, i32, i32, i32, i32,
                                                                  i32, i, i, f32, f32]
        L.oracle_gather_kv_dequant_fast.restype = i
        L.oracle_quantize_fp8_fast.argtypes = [vp, i, i64, f32, i, vp]
        L.oracle_dequantize_fp8_fast.argtypes = [vp, i64, f32, i, i, vp]
        L.oracle_set_threads.argtypes = [i]
        L.oracle_set_threads.restype = i
        L.oracle_gather_kv_ragged.argtypes = geom + geom + [vp, vp, vp, vp, vp, i, i64, vp, i,
                                                            vp, i, i32, i32, i32, i32, i32,
                                                            i32, i, i, sp, sp]
        L.oracle_gather_kv_offsets.argtypes = geom + geom + [vp, vp, i64, vp, vp, vp, vp, i,
                                                             i32, i32, i32, i32, i32, i32,
                                                             i32, i, i, sp, sp]
        L.oracle_f32_to_e4m3.argtypes = [f32]
        L.oracle_f32_to_e4m3.restype = C.c_uint8
        L.oracle_e4m3_to_f32.argtypes = [C.c_uint8]
        L.oracle_e4m3_to_f32.restype = f32
        L.oracle_f32_to_e5m2.argtypes = [f32]
        L.oracle_f32_to_e5m2.restype = C.c_uint8
        L.oracle_e5m2_to_f32.argtypes = [C.c_uint8]
        L.oracle_e5m2_to_f32.restype = f32
        L.oracle_f32_to_bf16.argtypes = [f32]
        L.oracle_f32_to_bf16.restype = C.c_uint16
        L.oracle_f32_to_f16.argtypes = [f32]
        L.oracle_f32_to_f16.restype = C.c_uint16
        L.oracle_f16_to_f32.argtypes = [C.c_uint16]
        L.oracle_f16_to_f32.restype = f32
        L.oracle_quantize_fp8.argtypes = [vp, i, i64, f32, i, vp]
        L.oracle_dequantize_fp8.argtypes = [vp, i64, f32, i, i, vp]
        _LIB = L
    return _LIB


def _ptr(a: np.ndarray) -> int:
    if not a.flags["C_CONTIGUOUS"]:
        raise ValueError("oracle buffers must be C-contiguous")
    return a.ctypes.data


def _strides(s) -> C.Array:
    arr = (C.c_int64 * 5)(*([int(x) for x in s] + [0] * (5 - len(s))))
    return arr


class Geometry:
    """Layout, element strides and pack of one cache tensor."""

    def __init__(self, layout: int, stride, pack: int = 1):
        self.layout = int(layout)
        self.stride = tuple(int(x) for x in stride)
        self.pack = int(pack)

    @classmethod
    def custom(cls, stride, head_dim: int, pack: int | None = None) -> "Geometry":
        """KVX_LAYOUT_BLOCK_CUSTOM: strides of the axes (block, offset, head,
        dim) or (block, offset, head, dim / pack, pack)."""
        st = tuple(int(x) for x in stride)
        if len(st) == 4:
            return cls(15, (st[0], st[1], st[2], 0, st[3]), head_dim)
        return cls(15, st, pack)

    def args(self):
        return [self.layout, C.cast(_strides(self.stride), _I64P), self.pack]


def cache_offset(g: Geometry, block, offset, head, dim) -> int:
    return lib().oracle_cache_offset(*g.args(), block, offset, head, dim)


def write_kv(gk: Geometry, gv: Geometry, key, value, key_cache, value_cache, slots,
             *, heads, head_dim, block_size, num_blocks, io_dtype, cache_dtype,
             k_scale=1.0, v_scale=1.0) -> None:
    """Element-wise write (kernels/kvx_paged_kv.cu:93-124), in place."""
    slots = np.ascontiguousarray(slots)
    kk, ks = _scale_arg(k_scale)
    vk, vs = _scale_arg(v_scale)
    lib().oracle_write_kv(*gk.args(), *gv.args(), _ptr(key), _ptr(value),
                          _ptr(key_cache), _ptr(value_cache), _ptr(slots),
                          int(slots.dtype == np.int64), int(slots.size), heads,
                          head_dim, block_size, num_blocks, int(io_dtype),
                          int(cache_dtype), ks, vs)


def gather_kv(gk: Geometry, gv: Geometry, key_cache, value_cache, key_out, value_out,
              block_table, seq_lens, *, seq_count, max_blocks_per_seq, max_seq_len,
              heads, head_dim, block_size, num_blocks, cache_dtype, io_dtype,
              k_scale=1.0, v_scale=1.0) -> None:
    """Element-wise gather (kernels/kvx_paged_kv.cu:226-267), in place."""
    block_table = np.ascontiguousarray(block_table)
    seq_lens = np.ascontiguousarray(seq_lens)
    if block_table.dtype != seq_lens.dtype:
        raise ValueError("block table and seq_lens share one index dtype")
    kk, ks = _scale_arg(k_scale)
    vk, vs = _scale_arg(v_scale)
    lib().oracle_gather_kv(*gk.args(), *gv.args(), _ptr(key_cache), _ptr(value_cache),
                           _ptr(key_out), _ptr(value_out), _ptr(block_table),
                           _ptr(seq_lens), int(block_table.dtype == np.int64),
                           seq_count, max_blocks_per_seq, max_seq_len, heads, head_dim,
                           block_size, num_blocks, int(cache_dtype), int(io_dtype), ks, vs)


def gather_kv_ragged(gk: Geometry, gv: Geometry, key_cache, value_cache, key_out, value_out,
                     indices, indptr, seq_lens, *, max_seq_len, heads, head_dim, block_size,
                     num_blocks, cache_dtype, io_dtype, k_scale=1.0, v_scale=1.0) -> None:
    """RAGGED-table gather (KVX_SPEC.md:107-114), in place."""
    indices = np.ascontiguousarray(indices)
    indptr = np.ascontiguousarray(indptr)
    seq_lens = np.ascontiguousarray(seq_lens)
    kk, ks = _scale_arg(k_scale)
    vk, vs = _scale_arg(v_scale)
    lib().oracle_gather_kv_ragged(*gk.args(), *gv.args(), _ptr(key_cache), _ptr(value_cache),
                                  _ptr(key_out), _ptr(value_out), _ptr(indices),
                                  int(indices.dtype == np.int64), int(indices.size),
                                  _ptr(indptr),
                                  int(indptr.dtype == np.int64), _ptr(seq_lens),
                                  int(seq_lens.dtype == np.int64), int(seq_lens.size),
                                  max_seq_len, heads, head_dim, block_size, num_blocks,
                                  int(cache_dtype), int(io_dtype), ks, vs)


def gather_kv_offsets(gk: Geometry, gv: Geometry, pool_primary, pool_secondary,
                      bytes_per_block, key_out, value_out, table, seq_lens, *,
                      max_blocks_per_seq, max_seq_len, heads, head_dim, block_size,
                      num_blocks, cache_dtype, io_dtype, k_scale=1.0, v_scale=1.0) -> None:
    """KV_OFFSETS-table gather (KVX_SPEC.md:116-122), in place.  `table` is
    int32 [seq_count, 1, 2, max_blocks_per_seq]; pool_secondary may be None."""
    table = np.ascontiguousarray(table, dtype=np.int32)
    seq_lens = np.ascontiguousarray(seq_lens)
    sec = None if pool_secondary is None else _ptr(pool_secondary)
    kk, ks = _scale_arg(k_scale)
    vk, vs = _scale_arg(v_scale)
    lib().oracle_gather_kv_offsets(*gk.args(), *gv.args(), _ptr(pool_primary), sec,
                                   int(bytes_per_block), _ptr(key_out), _ptr(value_out),
                                   _ptr(table), _ptr(seq_lens), int(seq_lens.dtype == np.int64),
                                   int(seq_lens.size), max_blocks_per_seq, max_seq_len, heads,
                                   head_dim, block_size, num_blocks, int(cache_dtype),
                                   int(io_dtype), ks, vs)


def write_kv_fast(gk: Geometry, gv: Geometry, key, value, key_cache, value_cache, slots,
                  *, heads, head_dim, block_size, num_blocks, elem_size) -> int:
    slots = np.ascontiguousarray(slots)
    return lib().oracle_write_kv_fast(*gk.args(), *gv.args(), _ptr(key), _ptr(value),
                                      _ptr(key_cache), _ptr(value_cache), _ptr(slots),
                                      int(slots.dtype == np.int64), int(slots.size),
                                      heads, head_dim, block_size, num_blocks, elem_size)


def gather_kv_fast(gk: Geometry, gv: Geometry, key_cache, value_cache, key_out,
                   value_out, block_table, seq_lens, *, seq_count, max_blocks_per_seq,
                   max_seq_len, heads, head_dim, block_size, num_blocks,
                   elem_size) -> int:
    return lib().oracle_gather_kv_fast(*gk.args(), *gv.args(), _ptr(key_cache),
                                       _ptr(value_cache), _ptr(key_out), _ptr(value_out),
                                       _ptr(block_table), _ptr(seq_lens),
                                       int(block_table.dtype == np.int64), seq_count,
                                       max_blocks_per_seq, max_seq_len, heads, head_dim,
                                       block_size, num_blocks, elem_size)


def write_kv_quant_fast(gk: Geometry, gv: Geometry, key, value, key_cache, value_cache,
                        slots, *, heads, head_dim, block_size, num_blocks, io_dtype,
                        cache_dtype, k_scale: float, v_scale: float) -> int:
    """Quantizing write of write_kv with per-tensor scales, OpenMP and
    table-driven casts (the timed CPU baseline of FP8 caches)."""
    slots = np.ascontiguousarray(slots)
    return lib().oracle_write_kv_quant_fast(*gk.args(), *gv.args(), _ptr(key), _ptr(value),
                                            _ptr(key_cache), _ptr(value_cache), _ptr(slots),
                                            int(slots.dtype == np.int64), int(slots.size),
                                            heads, head_dim, block_size, num_blocks,
                                            int(io_dtype), int(cache_dtype), float(k_scale),
                                            float(v_scale))


def gather_kv_dequant_fast(gk: Geometry, gv: Geometry, key_cache, value_cache, key_out,
                           value_out, block_table, seq_lens, *, seq_count,
                           max_blocks_per_seq, max_seq_len, heads, head_dim, block_size,
                           num_blocks, cache_dtype, io_dtype, k_scale: float,
                           v_scale: float) -> int:
    """Dequantizing gather of gather_kv with per-tensor scales, OpenMP and
    table-driven casts (the timed CPU baseline of FP8 caches)."""
    return lib().oracle_gather_kv_dequant_fast(
        *gk.args(), *gv.args(), _ptr(key_cache), _ptr(value_cache), _ptr(key_out),
        _ptr(value_out), _ptr(block_table), _ptr(seq_lens), int(block_table.dtype == np.int64),
        seq_count, max_blocks_per_seq, max_seq_len, heads, head_dim, block_size, num_blocks,
        int(cache_dtype), int(io_dtype), float(k_scale), float(v_scale))


def quantize_fp8_fast(x: np.ndarray, io_dtype: int, scale: float, fp8: int = 4) -> np.ndarray:
    """quantize_fp8 through the fast paths' table-driven cast."""
    x = np.ascontiguousarray(x)
    out = np.empty(x.size, np.uint8)
    lib().oracle_quantize_fp8_fast(_ptr(x), int(io_dtype), x.size, float(scale), int(fp8),
                                   _ptr(out))
    return out


def dequantize_fp8_fast(q: np.ndarray, scale: float, io_dtype: int, fp8: int = 4) -> np.ndarray:
    """dequantize_fp8 through the fast paths' table-driven cast."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(q.size, np.uint32 if int(io_dtype) == 3 else np.uint16)
    lib().oracle_dequantize_fp8_fast(_ptr(q), q.size, float(scale), int(fp8), int(io_dtype),
                                     _ptr(out))
    return out


def set_threads(n: int) -> int:
    """Threads of write_kv_fast / gather_kv_fast from now on; returns the
    previous count."""
    return lib().oracle_set_threads(int(n))


E4M3, E5M2 = 4, 5  # kvx_abi.h dtype codes of the FP8 formats


def quantize_fp8(x: np.ndarray, io_dtype: int, scale: float, fp8: int = E4M3) -> np.ndarray:
    """fp8(sat(x / scale)) of a raw io buffer (f32 / f16 / bf16 bits)."""
    x = np.ascontiguousarray(x)
    n = x.size
    out = np.empty(n, np.uint8)
    lib().oracle_quantize_fp8(_ptr(x), int(io_dtype), n, float(scale), int(fp8), _ptr(out))
    return out


def dequantize_fp8(q: np.ndarray, scale: float, io_dtype: int, fp8: int = E4M3) -> np.ndarray:
    """io(f32(q) * scale) as raw bits (uint32 for F32, uint16 otherwise)."""
    q = np.ascontiguousarray(q, dtype=np.uint8)
    out = np.empty(q.size, np.uint32 if int(io_dtype) == 3 else np.uint16)
    lib().oracle_dequantize_fp8(_ptr(q), q.size, float(scale), int(fp8), int(io_dtype),
                                _ptr(out))
    return out


def quantize_e4m3(x: np.ndarray, io_dtype: int, scale: float) -> np.ndarray:
    return quantize_fp8(x, io_dtype, scale, E4M3)


def dequantize_e4m3(q: np.ndarray, scale: float, io_dtype: int) -> np.ndarray:
    return dequantize_fp8(q, scale, io_dtype, E4M3)
