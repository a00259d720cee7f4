"""Helpers shared by the GPU parity tests: device buffers for a paged cache
(optionally padded, i.e. with non-canonical strides), and the calls that run
the same write / gather through libkvx_amd.so and through the CPU oracle."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from kvx_amd import paged
from kvx_amd.abi import DType, Layout, Status, contiguous_strides

TORCH_DT = {DType.F32: torch.float32, DType.F16: torch.float16,
            DType.BF16: torch.bfloat16, DType.F8_E4M3: torch.float8_e4m3fn,
            DType.F8_E5M2: torch.float8_e5m2}


class ScaleArg:
    """Indexed FP8 scales for a test: `values` (float32, [H], [nb] or
    [nb, H]) stored on the device with `stride` (elements; None =
    contiguous), handed to the library as a paged.Scales and to the oracle
    as an oracle.Scale with the same strides."""

    def __init__(self, granularity, values, stride=None, device="cuda"):
        from kvx_amd.abi import ScaleGranularity as SG

        self.granularity = SG(granularity)
        vals = np.asarray(values, dtype=np.float32)
        if stride is None:
            stride = contiguous_strides(vals.shape)
        stride = tuple(int(x) for x in stride)
        n = 1 + sum((d - 1) * st for d, st in zip(vals.shape, stride))
        host = torch.full((n,), float("nan"), dtype=torch.float32)  # gaps unused
        torch.as_strided(host, vals.shape, stride).copy_(torch.from_numpy(vals))
        self.dev = torch.as_strided(host.to(device), vals.shape, stride)
        flat = host.numpy()
        if self.granularity == SG.PER_HEAD:
            self.oracle = oracle.Scale(flat, 0, stride[0])
        elif self.granularity == SG.PER_BLOCK:
            self.oracle = oracle.Scale(flat, stride[0], 0)
        else:
            self.oracle = oracle.Scale(flat, stride[0], stride[1])

    def device(self):
        return paged.Scales(self.dev, self.granularity)


def _dev_scale(x, device):
    """(library scale, oracle scale) for None / float / ScaleArg."""
    if x is None:
        return None, 1.0
    if isinstance(x, ScaleArg):
        return x.device(), x.oracle
    return torch.tensor([x], dtype=torch.float32, device=device), x


def np_bytes(t: torch.Tensor) -> np.ndarray:
    """Host copy of a tensor's bytes (the tensor must be contiguous)."""
    return t.detach().contiguous().view(torch.uint8).cpu().numpy().reshape(-1).copy()


def random_fill(t: torch.Tensor, gen: torch.Generator) -> torch.Tensor:
    """Fill any tensor with random bytes (NaN/Inf patterns included)."""
    b = t.view(torch.uint8)
    b.copy_(torch.randint(0, 256, b.shape, dtype=torch.uint8, generator=gen,
                          device="cpu").to(b.device))
    return t


class CacheBuf:
    """A K or V cache tensor: `base` owns the storage, `view` is the shaped
    (possibly padded) tensor handed to the library."""

    def __init__(self, layout, dtype, nb, bs, H, D, pack, device, gen, pad_axis=None,
                 pad=3):
        self.layout = Layout(layout)
        self.pack = pack
        shape = paged.cache_shape(layout, nb, bs, H, D, pack)
        big = list(shape)
        if pad_axis is not None:
            big[pad_axis] += pad
        self.base = torch.empty(big, dtype=TORCH_DT[dtype], device=device)
        random_fill(self.base, gen)
        self.view = self.base[tuple(slice(0, n) for n in shape)]

    def geometry(self) -> oracle.Geometry:
        return oracle.Geometry(self.layout, self.view.stride(),
                               self.pack if self.layout == Layout.BLOCK_HND_PACKED else 1)


class CustomBuf:
    """A KVX_LAYOUT_BLOCK_CUSTOM cache tensor: storage with axes in `order` (a
    permutation of the logical axes b, o, h, d or b, o, h, p, x with
    p = d / x), its last storage axis padded by `pad` elements, and the
    logical view handed to the library."""

    def __init__(self, dtype, nb, bs, H, D, order, x=None, pad=0, gen=None, device="cuda"):
        sizes = {"b": nb, "o": bs, "h": H}
        if x is None:
            sizes["d"] = D
            logical = "bohd"
        else:
            sizes["p"], sizes["x"] = D // x, x
            logical = "bohpx"
        assert sorted(order) == sorted(logical)
        shape = [sizes[a] for a in order]
        shape[-1] += pad
        self.base = torch.empty(shape, dtype=TORCH_DT[dtype], device=device)
        random_fill(self.base, gen or torch.Generator().manual_seed(0))
        trimmed = self.base[..., : sizes[order[-1]]]
        self.view = trimmed.permute([order.index(a) for a in logical])
        self.x = x
        self.D = D

    def geometry(self) -> oracle.Geometry:
        return oracle.Geometry.custom(self.view.stride(), self.D, self.x)


def custom_cache(dtype, nb, bs, H, D, korder, vorder, kx=None, vx=None, gen=None, pad=0):
    """PagedCache of two CUSTOM tensors (K and V storage orders korder /
    vorder), with their CustomBufs."""
    k = CustomBuf(dtype, nb, bs, H, D, korder, kx, pad, gen)
    v = CustomBuf(dtype, nb, bs, H, D, vorder, vx, pad, gen)
    pc = paged.PagedCache(k.view, v.view, Layout.BLOCK_CUSTOM, Layout.BLOCK_CUSTOM, nb, bs, H, D)
    return pc, k, v


def make_cache(k_layout, v_layout, dtype, nb, bs, H, D, pack=8, device="cuda",
               gen=None, k_pad=None, v_pad=None):
    gen = gen or torch.Generator().manual_seed(0)
    k = CacheBuf(k_layout, dtype, nb, bs, H, D, pack, device, gen, k_pad)
    v = CacheBuf(v_layout, dtype, nb, bs, H, D, pack, device, gen, v_pad)
    pc = paged.PagedCache(k.view, v.view, k.layout, v.layout, nb, bs, H, D)
    return pc, k, v


def check_write(pc, kbuf, vbuf, key, value, slots, *, io_dtype, cache_dtype,
                tokens_per_seq=None, k_scale=None, v_scale=None, entry="launch",
                stream=None):
    """Run the write on the GPU and in the oracle from identical inputs and
    require bit-identical caches (touched and untouched bytes alike)."""
    kb0, vb0 = np_bytes(kbuf.base), np_bytes(vbuf.base)
    ks, k_or = _dev_scale(k_scale, key.device)
    vs, v_or = _dev_scale(v_scale, key.device)
    st = paged.write_kv(pc, key, value, slots, tokens_per_seq=tokens_per_seq,
                        k_scale=ks, v_scale=vs, entry=entry, stream=stream)
    assert st == Status.OK, st
    torch.cuda.synchronize()
    oracle.write_kv(kbuf.geometry(), vbuf.geometry(), np_bytes(key), np_bytes(value),
                    kb0, vb0, slots.cpu().numpy(), heads=pc.heads, head_dim=pc.head_dim,
                    block_size=pc.block_size, num_blocks=pc.num_blocks,
                    io_dtype=io_dtype, cache_dtype=cache_dtype, k_scale=k_or, v_scale=v_or)
    got_k, got_v = np_bytes(kbuf.base), np_bytes(vbuf.base)
    assert np.array_equal(got_k, kb0), _first_diff(got_k, kb0)
    assert np.array_equal(got_v, vb0), _first_diff(got_v, vb0)


def check_gather(pc, kbuf, vbuf, key_out, value_out, table, lens, max_seq_len, *,
                 cache_dtype, io_dtype, k_scale=None, v_scale=None, entry="launch",
                 stream=None):
    """Run the gather on the GPU and in the oracle from identical inputs (the
    outputs pre-filled with random bytes) and require bit-identical outputs."""
    ko0, vo0 = np_bytes(key_out), np_bytes(value_out)
    ks, k_or = _dev_scale(k_scale, key_out.device)
    vs, v_or = _dev_scale(v_scale, key_out.device)
    st = paged.gather_kv(pc, key_out, value_out, table, lens, max_seq_len, k_scale=ks,
                         v_scale=vs, entry=entry, stream=stream)
    assert st == Status.OK, st
    torch.cuda.synchronize()
    S, mbps = table.shape
    oracle.gather_kv(kbuf.geometry(), vbuf.geometry(), np_bytes(kbuf.base),
                     np_bytes(vbuf.base), ko0, vo0, table.cpu().numpy(), lens.cpu().numpy(),
                     seq_count=S, max_blocks_per_seq=mbps, max_seq_len=max_seq_len,
                     heads=pc.heads, head_dim=pc.head_dim, block_size=pc.block_size,
                     num_blocks=pc.num_blocks, cache_dtype=cache_dtype, io_dtype=io_dtype,
                     k_scale=k_or, v_scale=v_or)
    got_k, got_v = np_bytes(key_out), np_bytes(value_out)
    assert np.array_equal(got_k, ko0), _first_diff(got_k, ko0)
    assert np.array_equal(got_v, vo0), _first_diff(got_v, vo0)


def _first_diff(a: np.ndarray, b: np.ndarray) -> str:
    idx = np.flatnonzero(a != b)
    return f"{idx.size} bytes differ, first at {idx[:8].tolist()}"


def check_gather_ragged(pc, kbuf, vbuf, key_out, value_out, table: paged.RaggedTable, lens,
                        max_seq_len, *, cache_dtype, io_dtype, k_scale=None, v_scale=None,
                        entry="launch"):
    """RAGGED-table gather on the GPU and in the oracle; bit-identical outputs."""
    ko0, vo0 = np_bytes(key_out), np_bytes(value_out)
    ks, k_or = _dev_scale(k_scale, key_out.device)
    vs, v_or = _dev_scale(v_scale, key_out.device)
    st = paged.gather_kv(pc, key_out, value_out, table, lens, max_seq_len, k_scale=ks,
                         v_scale=vs, entry=entry)
    assert st == Status.OK, st
    torch.cuda.synchronize()
    oracle.gather_kv_ragged(kbuf.geometry(), vbuf.geometry(), np_bytes(kbuf.base),
                            np_bytes(vbuf.base), ko0, vo0, table.indices.cpu().numpy(),
                            table.indptr.cpu().numpy(), lens.cpu().numpy(),
                            max_seq_len=max_seq_len, heads=pc.heads, head_dim=pc.head_dim,
                            block_size=pc.block_size, num_blocks=pc.num_blocks,
                            cache_dtype=cache_dtype, io_dtype=io_dtype,
                            k_scale=k_or, v_scale=v_or)
    got_k, got_v = np_bytes(key_out), np_bytes(value_out)
    assert np.array_equal(got_k, ko0), _first_diff(got_k, ko0)
    assert np.array_equal(got_v, vo0), _first_diff(got_v, vo0)


class OffsetsPool:
    """KV_OFFSETS storage: a primary (and optional secondary) pool of
    `num_blocks` single-tensor blocks every `bytes_per_block` bytes, and K / V
    cache views over the primary pool that carry the in-block layouts."""

    def __init__(self, k_layout, v_layout, dtype, nb, bs, H, D, pack=8, pitch_pad=0,
                 secondary=True, device="cuda", gen=None):
        gen = gen or torch.Generator().manual_seed(0)
        es = TORCH_DT[dtype].itemsize
        self.bytes_per_block = bs * H * D * es + pitch_pad
        assert self.bytes_per_block % es == 0
        self.primary = random_fill(torch.empty(nb * self.bytes_per_block, dtype=torch.uint8,
                                               device=device), gen)
        self.secondary = None
        if secondary:
            self.secondary = random_fill(torch.empty_like(self.primary), gen)
        typed = self.primary.view(TORCH_DT[dtype])
        self.geoms = []
        views = []
        for layout in (k_layout, v_layout):
            shape = paged.cache_shape(layout, nb, bs, H, D, pack)
            st = list(contiguous_strides(shape))
            st[0] = self.bytes_per_block // es
            views.append(torch.as_strided(typed, shape, st))
            self.geoms.append(oracle.Geometry(layout, st,
                                              pack if layout == Layout.BLOCK_HND_PACKED else 1))
        self.pc = paged.PagedCache(views[0], views[1], Layout(k_layout), Layout(v_layout),
                                   nb, bs, H, D)

    def table(self, offsets: torch.Tensor) -> paged.OffsetsTable:
        return paged.OffsetsTable(offsets, self.primary, self.secondary, self.bytes_per_block)


def bound_offsets(offsets: np.ndarray, num_blocks: int, pool_blocks) -> np.ndarray:
    """The KV_OFFSETS table that kvx_launch_gather_kv_pools gathers like:
    an int32 KVCacheIndex entry whose index is at or past its pool's count
    (0 or >= num_blocks: num_blocks) becomes an index past every pool, which
    the gather skips as it skips indices >= num_blocks."""
    u = offsets.view(np.uint32)
    sec = (u >> 31).astype(bool)
    idx = (u & 0x7FFFFFFF).astype(np.int64)
    lim = [c if 0 < c < num_blocks else num_blocks for c in pool_blocks]
    cut = np.where(sec, idx >= lim[1], idx >= lim[0])
    return np.where(cut, np.uint32(0x7FFFFFFF), u).astype(np.uint32).view(np.int32)


def check_gather_offsets(pool: OffsetsPool, key_out, value_out, offsets, lens, max_seq_len,
                         *, cache_dtype, io_dtype, k_scale=None, v_scale=None,
                         entry="launch", pool_blocks=None):
    """KV_OFFSETS-table gather on the GPU and in the oracle; bit-identical
    outputs.  pool_blocks = (primary, secondary): the GPU takes
    kvx_launch_gather_kv_pools, the oracle the table with the entries past
    each pool's count skipped (bound_offsets)."""
    pc = pool.pc
    ko0, vo0 = np_bytes(key_out), np_bytes(value_out)
    ks, k_or = _dev_scale(k_scale, key_out.device)
    vs, v_or = _dev_scale(v_scale, key_out.device)
    st = paged.gather_kv(pc, key_out, value_out, pool.table(offsets), lens, max_seq_len,
                         k_scale=ks, v_scale=vs, entry=entry, pool_blocks=pool_blocks)
    assert st == Status.OK, st
    torch.cuda.synchronize()
    sec = None if pool.secondary is None else np_bytes(pool.secondary)
    table = offsets.cpu().numpy()
    if pool_blocks is not None:
        table = bound_offsets(table, pc.num_blocks, pool_blocks)
    oracle.gather_kv_offsets(pool.geoms[0], pool.geoms[1], np_bytes(pool.primary), sec,
                             pool.bytes_per_block, ko0, vo0, table,
                             lens.cpu().numpy(), max_blocks_per_seq=offsets.shape[3],
                             max_seq_len=max_seq_len, heads=pc.heads, head_dim=pc.head_dim,
                             block_size=pc.block_size, num_blocks=pc.num_blocks,
                             cache_dtype=cache_dtype, io_dtype=io_dtype,
                             k_scale=k_or, v_scale=v_or)
    got_k, got_v = np_bytes(key_out), np_bytes(value_out)
    assert np.array_equal(got_k, ko0), _first_diff(got_k, ko0)
    assert np.array_equal(got_v, vo0), _first_diff(got_v, vo0)
