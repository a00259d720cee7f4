"""Seeded synthetic workloads for the five benchmark configurations (c1-c5).

Each function returns a `Workload` that holds only the index metadata
(slot mapping, block table, sequence lengths) as numpy arrays plus the shapes
and dtypes; payload data is generated on the device by the caller.  All
randomness comes from numpy PCG64 with the seed recorded in the workload.

  c1  TinyLlama-1.1B prefill write + gather, f16, H=4, D=64, bs=16,
      8 seqs x 128 tokens, blocks from a seeded permutation of a 512 pool.
  c2  Llama-3-8B decode write + full-context gather, bf16, H=8, D=128,
      bs=16, 256 seqs, ctx ~ U[512, 8192], 5% of slots = -1.
  c3  Llama-3-8B chunked prefill write, bf16, 16 x 2048 tokens, K in the
      x-packed layout (x = 8), V plain NHD, random block assignment.
  c4  c2 with an FP8 E4M3 cache: 128 decode tokens quantized with per-tensor
      scales amax/448 from a seeded calibration batch, dequantizing gather.
  c5  Llama-3-70B-shaped, bs=32, 64 seqs, ctx ~ U[16384, 32768], 32 prefill
      tokens per seq written, full gather, blocks scattered over a pool of
      about 200 GB of K+V.
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np

from .abi import DType, Layout


@dataclass
class Workload:
    name: str
    seed: int
    heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    cache_dtype: DType
    io_dtype: DType
    k_layout: Layout
    v_layout: Layout
    pack: int
    # write
    slots: np.ndarray            # [T] int64 or int32
    tokens_per_seq: int | None   # prefill entry when set
    # gather
    block_table: np.ndarray      # [S, max_blocks_per_seq]
    seq_lens: np.ndarray         # [S], same dtype as block_table
    max_seq_len: int
    layers: int = 1
    notes: dict = field(default_factory=dict)

    @property
    def num_tokens(self) -> int:
        return int(self.slots.size)

    @property
    def seq_count(self) -> int:
        return int(self.block_table.shape[0])

    @property
    def max_blocks_per_seq(self) -> int:
        return int(self.block_table.shape[1])

    @property
    def row_elems(self) -> int:
        return self.heads * self.head_dim

    def gathered_tokens(self) -> int:
        n = np.minimum(self.seq_lens.astype(np.int64), self.max_seq_len)
        n = np.minimum(n, self.max_blocks_per_seq * self.block_size)
        return int(np.maximum(n, 0).sum())

    def valid_write_tokens(self) -> int:
        s = self.slots.astype(np.int64)
        ok = (s >= 0) & (s // self.block_size < self.num_blocks)
        return int(ok.sum())


def dtype_bytes(dt: DType) -> int:
    return {DType.F16: 2, DType.BF16: 2, DType.F32: 4, DType.F8_E4M3: 1,
            DType.F8_E5M2: 1}[DType(dt)]


def write_bytes(w: Workload) -> int:
    """Algorithmic bytes of one write: every valid row of K and V read from
    io and written to the cache, plus the slot array (and two f32 scales
    when quantizing)."""
    e = w.row_elems
    b = w.valid_write_tokens() * 2 * e * (dtype_bytes(w.io_dtype) + dtype_bytes(w.cache_dtype))
    b += w.num_tokens * w.slots.itemsize
    if w.cache_dtype != w.io_dtype:
        b += 8
    return int(b)


TABLE_FORMATS = ("packed", "ragged", "kv_offsets")


def _gathered_per_seq(w: Workload) -> np.ndarray:
    n = np.minimum(np.maximum(w.seq_lens.astype(np.int64), 0), w.max_seq_len)
    return np.minimum(n, w.max_blocks_per_seq * w.block_size)


def gather_bytes(w: Workload, table: str = "packed") -> int:
    """Algorithmic bytes of one gather: gathered rows of K and V read from the
    cache and written out, plus the index entries used and seq_lens.  Index
    entries per format: PACKED one per used block; RAGGED one per gathered
    token plus indptr (S + 1 entries); KV_OFFSETS two int32 (K and V) per
    used block."""
    e = w.row_elems
    n = _gathered_per_seq(w)
    blocks = (n + w.block_size - 1) // w.block_size
    b = int(n.sum()) * 2 * e * (dtype_bytes(w.cache_dtype) + dtype_bytes(w.io_dtype))
    if table == "packed":
        b += int(blocks.sum()) * w.block_table.itemsize
    elif table == "ragged":
        b += int(n.sum()) * w.block_table.itemsize + (w.seq_count + 1) * 4
    elif table == "kv_offsets":
        b += int(blocks.sum()) * 2 * 4
    else:
        raise ValueError(table)
    b += w.seq_count * w.seq_lens.itemsize
    if w.cache_dtype != w.io_dtype:
        b += 8
    return int(b)


def gathered_blocks(w: Workload) -> int:
    """Block-table entries a gather uses (logical blocks with rows)."""
    n = _gathered_per_seq(w)
    return int(((n + w.block_size - 1) // w.block_size).sum())


def ragged_table(w: Workload) -> tuple[np.ndarray, np.ndarray]:
    """The workload's block table as a RAGGED table (KVX_SPEC.md:107-114):
    one block id per gathered token, int32, and int32 indptr prefix sums."""
    n = _gathered_per_seq(w)
    parts = [w.block_table[s, np.arange(n[s]) // w.block_size] for s in range(w.seq_count)]
    indices = np.concatenate(parts).astype(np.int32) if parts else np.zeros(0, np.int32)
    indptr = np.concatenate([[0], np.cumsum(n)]).astype(np.int32)
    return indices, indptr


def kv_offsets_table(w: Workload) -> np.ndarray:
    """The workload's block table as an int32 KV_OFFSETS table
    [S, 1, 2, max_blocks_per_seq] over a pool of 2 * num_blocks blocks in
    TensorRT-LLM's pairing (K of logical block b at pool block 2b, V at
    2b + 1).  Unused entries (-1) become 0x7FFFFFFF, an index past the pool
    that the gather skips."""
    t = w.block_table.astype(np.int64)
    k = np.where(t < 0, 0x7FFFFFFF, 2 * t)
    v = np.where(t < 0, 0x7FFFFFFF, 2 * t + 1)
    return np.stack([k, v], axis=1)[:, None].astype(np.int32)


def _slots_for(positions: np.ndarray, table_row: np.ndarray, bs: int) -> np.ndarray:
    return table_row[positions // bs].astype(np.int64) * bs + positions % bs


def c1_tinyllama(seed: int = 1) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    S, L, bs, pool = 8, 128, 16, 512
    mbps = L // bs
    table = rng.permutation(pool)[: S * mbps].reshape(S, mbps).astype(np.int32)
    pos = np.arange(L)
    slots = np.concatenate([_slots_for(pos, table[s], bs) for s in range(S)])
    return Workload("c1_tinyllama_f16_prefill", seed, 4, 64, bs, pool, DType.F16,
                    DType.F16, Layout.BLOCK_NHD, Layout.BLOCK_NHD, 8,
                    slots.astype(np.int64), L, table,
                    np.full(S, L, np.int32), L, layers=22)


def _decode_tables(rng, S, lo, hi, bs, max_len, pool_blocks=None, ascending=False):
    lens = rng.integers(lo, hi, size=S, endpoint=True).astype(np.int64)
    need = (lens + bs - 1) // bs
    mbps = (max_len + bs - 1) // bs
    used = int(need.sum())
    pool = used if pool_blocks is None else int(pool_blocks)
    if pool_blocks is None:
        ids = rng.permutation(pool)
    else:
        ids = rng.choice(pool, size=used, replace=False)
    if ascending:
        ids = np.sort(ids)  # same draw, handed out in address order
    table = np.full((S, mbps), -1, np.int64)
    at = 0
    for s in range(S):
        table[s, : need[s]] = ids[at: at + need[s]]
        at += need[s]
    return lens, table, pool


def c2_llama8b_decode(seed: int = 2, batch: int = 256, order: str = "random",
                      block_size: int = 16) -> Workload:
    """c2; order "random": the sequences' blocks are a random permutation of
    the pool (the config); "ascending": the same lengths with sequence s
    taking the next blocks of the pool in address order, as a fresh
    allocator would hand them out, so that its gather reads the pool front
    to back.  block_size other than the config's 16 keeps the lengths and
    draws a pool of the larger or smaller blocks."""
    if order not in ("random", "ascending"):
        raise ValueError(order)
    if block_size <= 0 or block_size & (block_size - 1):
        raise ValueError(block_size)
    rng = np.random.Generator(np.random.PCG64(seed))
    bs, L = block_size, 8192
    lens, table, pool = _decode_tables(rng, batch, 512, 8192, bs, L,
                                       ascending=order == "ascending")
    pos = lens - 1  # the new token is the last position of each context
    slots = table[np.arange(batch), pos // bs] * bs + pos % bs
    pad = rng.choice(batch, size=int(round(0.05 * batch)), replace=False)
    slots[pad] = -1
    name = "c2_llama3_8b_decode_bf16" + ("" if order == "random" else f"_{order}")
    if bs != 16:
        name += f"_bs{bs}"
    return Workload(name, seed, 8, 128, bs, pool, DType.BF16,
                    DType.BF16, Layout.BLOCK_NHD, Layout.BLOCK_NHD, 8,
                    slots.astype(np.int64), None, table.astype(np.int32),
                    lens.astype(np.int32), L, layers=32,
                    notes={"padded_slots": int(pad.size)})


def c3_llama8b_prefill(seed: int = 3, v_layout: Layout = Layout.BLOCK_NHD, seqs: int = 16,
                       order: str = "random", shift: int = 0,
                       block_size: int = 16) -> Workload:
    """c3; `seqs` chunks of 2048 tokens over a pool of 512 blocks per
    sequence (16 and 8192 as configured).  order "random": the sequences'
    blocks are a seeded random draw from the pool; "ascending": sequence s
    takes blocks s * 128 .. s * 128 + 127 in order, as a fresh allocator
    would hand them out.  Two orders separate what random blocks change:
    "sorted" is the random draw in ascending order (random's footprint,
    ascending's order), "compact" a random permutation of ascending's
    blocks (ascending's footprint, random order).  shift > 0: every chunk
    covers positions shift .. shift + 2047 of its sequence, so it starts
    inside its first block (as a chunked prefill does after a chunk that
    ended inside a block) and takes one more block.  block_size other than
    the config's 16 keeps the pool's tokens (8192 per sequence)."""
    if block_size <= 0 or block_size & (block_size - 1) or block_size > 2048:
        raise ValueError(block_size)
    if not 0 <= shift < block_size:
        raise ValueError(shift)
    rng = np.random.Generator(np.random.PCG64(seed))
    S, chunk, bs = seqs, 2048, block_size
    pool = 8192 // bs * S
    mbps = (shift + chunk + bs - 1) // bs
    draw = rng.permutation(pool)[: S * mbps]
    if order == "random":
        ids = draw
    elif order == "ascending":
        ids = np.arange(S * mbps)
    elif order == "sorted":
        ids = np.sort(draw)
    elif order == "compact":
        ids = rng.permutation(S * mbps)
    else:
        raise ValueError(order)
    table = ids.reshape(S, mbps).astype(np.int32)
    pos = shift + np.arange(chunk)
    slots = np.concatenate([_slots_for(pos, table[s], bs) for s in range(S)])
    name = "c3_llama3_8b_prefill_packedK_bf16"
    if S != 16:
        name += f"_s{S}"
    if order != "random":
        name += f"_{order}"
    if shift:
        name += f"_shift{shift}"
    if bs != 16:
        name += f"_bs{bs}"
    return Workload(name, seed, 8, 128, bs, pool,
                    DType.BF16, DType.BF16, Layout.BLOCK_HND_PACKED, Layout(v_layout), 8,
                    slots.astype(np.int64), chunk, table,
                    np.full(S, shift + chunk, np.int32), shift + chunk)


def c4_llama8b_fp8(seed: int = 4, batch: int = 128, block_size: int = 16) -> Workload:
    w = c2_llama8b_decode(seed, batch, block_size=block_size)
    w.name = "c4_llama3_8b_decode_fp8_e4m3" + ("" if block_size == 16 else f"_bs{block_size}")
    w.cache_dtype = DType.F8_E4M3
    w.notes["calibration_seed"] = seed + 1000
    w.notes["io_sigma"] = 2.0
    return w


def c5_llama70b_long(seed: int = 5, pool_blocks: int = 1_530_000,
                     batch: int = 64) -> Workload:
    rng = np.random.Generator(np.random.PCG64(seed))
    bs, L, tps = 32, 32768, 32
    lens, table, pool = _decode_tables(rng, batch, 16384, 32768, bs, L, pool_blocks)
    slots = []
    for s in range(batch):
        pos = np.arange(lens[s] - tps, lens[s])
        slots.append(table[s, pos // bs] * bs + pos % bs)
    return Workload("c5_llama3_70b_bs32_long_bf16", seed, 8, 128, bs, pool, DType.BF16,
                    DType.BF16, Layout.BLOCK_NHD, Layout.BLOCK_NHD, 8,
                    np.concatenate(slots).astype(np.int64), tps, table.astype(np.int32),
                    lens.astype(np.int32), L)


CONFIGS = {
    "c1": c1_tinyllama,
    "c2": c2_llama8b_decode,
    "c3": c3_llama8b_prefill,
    "c4": c4_llama8b_fp8,
    "c5": c5_llama70b_long,
}
