#!/usr/bin/env python3
"""Benchmark of the KVX paged KV write + gather hot path on one MI355X.

    python bench.py [--steps K] [--warmup W]            headline + every config
    python bench.py --config cN [options]              one configuration only
    python bench.py --sweep c3 [--sweep-scales 1,2,4,8]  size sweep of c3
    python bench.py --copy-probe                       rocprofv3 calibration

Headline (benchmark configuration c2): Llama-3-8B-shaped decode, bf16, 32 layers,
8 KV heads x 128, block_size 16, batch 256, contexts U[512, 8192], 5% of
slots -1.  One step = for each of the 32 layers (each with its own ~4.6 GB
paged K+V pool): the decode write of 256 new tokens, then the gather of
every sequence's full context into contiguous [256, 8192, 8, 128] K and V
buffers (shared across layers, as an attention workspace would be).  All
inputs are resident in HBM before timing; every launch goes through the C
ABI (kvx_launch_write_kv* / kvx_launch_gather_kv*) on one HIP stream.

value = algorithmic bytes of the whole step / step time (GB/s, 1e9), where
algorithmic bytes are the bytes a perfect implementation must move: every
valid K/V row read once and written once, plus the index arrays used
(kvx_amd.workloads.write_bytes / gather_bytes).

roofline: the dominant kernel (the gather): its algorithmic bytes per
launch / its mean launch duration, measured with HIP events recorded on the
launch stream after every launch inside the timed region (a launch runs from
the event before it to its own).  `traffic` is
the HBM bytes per launch of the committed rocprofv3 counter summary
(profiles/traffic_<kind>_<workload>.json), used only when that summary was
taken of the same algorithmic bytes and of the kernel sources now in the
tree (sha256 of kvx_amd/csrc's kernel files); otherwise null.

configs: the other benchmark configurations, each timed the same way in the
same run (c1 TinyLlama, c3 chunked prefill write, c4 FP8 E4M3 decode with a
dequantizing gather, c5 Llama-3-70B bs32 on a ~200 GB pool), each with its
kernels' mean / median, GB/s, fraction of peak and its own CPU baseline.

stream_ceiling: plain streaming copy / read / write / widen kernels
(libkvx_amd_probe.so, several launch shapes, the fastest reported) over the
same byte count as the dominant kernel, on buffers beyond the 256 MB
Infinity Cache: the best the box sustains with no index work (widen: the
FP8 dequantizing gather's 8-byte loads and 16-byte stores).  Over each
config's own pools and block table, with no slot, table, layout or
conversion work: c3's block_scatter / block_gather (the write's bytes
copied into, and out of, its randomly drawn blocks), and for the PACKED
gathers of NHD caches block_gather (c1, c2, c5: the blocks the gather
reads, in table order, copied to contiguous rows) or block_widen (c4: the
same with 8-byte reads stored as 16-byte chunks).

cpu_baseline: the CPU oracle's OpenMP fast path (row memcpy; table-driven
casts for FP8) timed on this host's cores, threads pinned, over a bounded
sample of the same workload.

write_graph: the headline's 32 decode writes captured in one HIP graph and
replayed with every cache level flushed before each replay (a 1 GiB read),
so the device time per write is an HBM figure without per-call launch cost.
"""
from __future__ import annotations

import os

# Pin the CPU baseline's OpenMP threads (one per core, in order) unless the
# caller chose otherwise; libgomp reads these when it initialises.
os.environ.setdefault("OMP_PROC_BIND", "close")
os.environ.setdefault("OMP_PLACES", "cores")

import argparse  # noqa: E402
import ctypes as C  # noqa: E402
import hashlib  # noqa: E402
import json  # noqa: E402
import statistics  # noqa: E402
import sys  # noqa: E402
import time  # noqa: E402
from pathlib import Path  # noqa: E402

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = ("achieved HBM GB/s (% of peak) and tokens/s for KV write+gather, "
          "1 MI355X")
PEAK_HBM_GBS = 8000.0
# Timed launches of the dominant kernel per sub-configuration, at least.
MIN_LAUNCHES = {"c1": 64, "c3": 64, "c4": 64, "c5": 20}
CPU_SAMPLE_SEQS = {"c1": 8, "c2": 64, "c3": 16, "c4": 32, "c5": 8}


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default=None, choices=["c1", "c2", "c3", "c4", "c5"],
                   help="run one configuration as the headline, without the others "
                        "(default: c2 as the headline, then c1, c3, c4, c5)")
    p.add_argument("--table", default="packed", choices=["packed", "ragged", "kv_offsets"],
                   help="block-table format of the gather (c1, c2, c4, c5); kv_offsets "
                        "puts K and V blocks in one TensorRT-LLM-style pool")
    p.add_argument("--write-entry", default="launch", choices=["launch", "torch_op"],
                   help="issue the writes through kvx_launch_write_kv* (ctypes) or the "
                        "PyTorch-ROCm op _C_cache_ops.reshape_and_cache_flash_kvx "
                        "(c1, c2, c4, c5: NHD caches)")
    p.add_argument("--layout", default=None, choices=["nhd", "hnd", "packed", "vllm"],
                   help="c2 / c3 / c5: cache layout of K and V (default NHD; c3: K "
                        "HND_PACKED x = 8, V NHD).  packed: "
                        "HND_PACKED x = 8; vllm: K HND_PACKED x = 8 and V "
                        "KVX_LAYOUT_BLOCK_CUSTOM [num_blocks, H, D, block_size], vLLM's "
                        "paged-attention pair (PACKED / RAGGED tables only)")
    p.add_argument("--heads", type=int, default=None,
                   help="c2 - c5: KV heads per GPU (one tensor-parallel rank's shard is "
                        "8 / TP; 6 or 12 are other models' counts); the block table, "
                        "lengths and slots are unchanged")
    p.add_argument("--head-dim", type=int, default=None,
                   help="c2 - c5: elements per head (a multiple of 8, e.g. 96 or 80); "
                        "heads x head_dim may not exceed the config's 8 x 128")
    p.add_argument("--fp8", default="e4m3", choices=["e4m3", "e5m2"],
                   help="c4: FP8 format of the cache")
    p.add_argument("--scales", default="tensor",
                   choices=["tensor", "head", "block", "block_head"],
                   help="c4: FP8 scale granularity (per tensor, per KV head, per physical "
                        "block, per block and head)")
    p.add_argument("--layers", type=int, default=None,
                   help="override the layer count of c1/c2/c4")
    p.add_argument("--c3-order", default="random",
                   choices=["random", "ascending", "sorted", "compact"],
                   help="c3: block assignment: a random draw from the pool (the config), "
                        "ascending as a fresh allocator hands blocks out, the random draw "
                        "sorted (random's footprint in ascending order), or ascending's "
                        "blocks permuted (ascending's footprint in random order)")
    p.add_argument("--c2-order", default="random", choices=["random", "ascending"],
                   help="c2: block assignment: a random permutation of the pool (the "
                        "config), or ascending as a fresh allocator hands blocks out (the "
                        "gather then reads the pool front to back)")
    p.add_argument("--block-size", type=int, default=None,
                   help="c2 / c3 / c4: tokens per block (a power of two; the configs' is 16), "
                        "same lengths (c2, c4) or chunks and pool tokens (c3), the pool drawn in "
                        "blocks of this size")
    p.add_argument("--c3-shift", type=int, default=0,
                   help="c3: every chunk starts this many tokens (0-15) into its first "
                        "block, as a chunked prefill continuing a chunk that ended inside "
                        "a block")
    p.add_argument("--c3-seqs", type=int, default=16,
                   help="c3: 2048-token chunks per write (pool 512 blocks per chunk)")
    p.add_argument("--sweep", default=None, choices=["c3"],
                   help="time c3's write, the PACKED gather of the same table and a plain "
                        "copy of the same bytes at several sizes; fit time = intercept + "
                        "bytes / slope")
    p.add_argument("--sweep-scales", default="1,2,4,8",
                   help="--sweep: multiples of c3's 16 sequences")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=5.0,
                   help="CPU baseline sampling budget per configuration")
    p.add_argument("--profile-only", action="store_true",
                   help="time only the KV kernels (no CPU baseline, stream ceiling or "
                        "graph): the command profiler runs use")
    p.add_argument("--detail", default=None, metavar="PATH",
                   help="also write the full record (every stream shape, every config's "
                        "full kernel, ceiling and CPU-baseline figures) to PATH as JSON; the "
                        "line on stdout stays compact")
    p.add_argument("--copy-probe", action="store_true",
                   help="only run three plain 1 GiB device copies: the known-size "
                        "kernel that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return p.parse_args()


def copy_probe() -> None:
    import torch

    a = torch.ones(1024**3 // 4, dtype=torch.float32, device="cuda")
    b = torch.empty_like(a)
    torch.cuda.synchronize()
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print("copy probe: 3 x 1 GiB device copies", flush=True)


# ---------------------------------------------------------------------------
# Device setup per configuration.

class Launch:
    """One prepared C-ABI call: descriptors are built once, outside timing."""

    def __init__(self, kind, fn, args, nbytes, tokens):
        self.kind, self.fn, self.args = kind, fn, args
        self.nbytes, self.tokens = nbytes, tokens

    def __call__(self, stream_handle):
        st = self.fn(*self.args, stream_handle)
        if st != 0:
            raise RuntimeError(f"{self.kind} launch returned status {st}")


class Built:
    """A configuration on the device: the workload, the per-step launch
    lists (rotated by step index), the config record and every buffer."""

    def __init__(self, w, steps, cfg, keep, extra=None):
        self.w, self.steps, self.cfg, self.keep = w, steps, cfg, keep
        self.extra = extra or {}


def reshape_rows(w, name, heads=None, head_dim=None, room=1.0):
    """--heads / --head-dim: give c2's, c3's, c4's or c5's rows another head count or head size
    (the block table, lengths and slots stay).  The row may outgrow the config's by at
    most `room` (the caller's factor of memory to spare, e.g. fewer layers), so the pools
    fit wherever the config does."""
    if heads is None and head_dim is None:
        return
    h = w.heads if heads is None else heads
    d = w.head_dim if head_dim is None else head_dim
    if name not in ("c2", "c3", "c4", "c5"):
        raise SystemExit("--heads / --head-dim apply to c2, c3, c4 and c5")
    if h <= 0 or d <= 0 or d % 8 != 0 or h * d > w.heads * w.head_dim * room:
        raise SystemExit("--heads and --head-dim: positive, head_dim a multiple of 8, "
                         f"heads x head_dim at most {room:g} x {w.heads} x {w.head_dim} "
                         "(c2 / c4: fewer --layers leave room for larger rows)")
    if heads is not None:
        w.name = f"{w.name}_h{h}"
    if head_dim is not None:
        w.name = f"{w.name}_d{d}"
    w.heads, w.head_dim = h, d


def gather_granules(w, pools, outs, dev):
    """The granule probe's inputs for a PACKED gather of contiguous NHD
    blocks: every buffer set is one layer's (K pool, V pool) with the shared
    (K, V) outputs, and the map lists, sequence by sequence, the blocks that
    hold its first min(seq_len, max_seq_len) rows; "gather" (copy) or
    "widen" (FP8 cache, 16-bit outputs).  None when a listed id is outside
    the pool or the outputs are too short."""
    import numpy as np
    import torch

    bs = w.block_size
    n = np.minimum(np.maximum(w.seq_lens.astype(np.int64), 0), w.max_seq_len)
    ids = np.concatenate([w.block_table[s, :(int(n[s]) + bs - 1) // bs]
                          for s in range(w.seq_count)]).astype(np.int64)
    if ids.size == 0 or ids.min() < 0 or ids.max() >= w.num_blocks:
        return None
    widen = w.cache_dtype != w.io_dtype
    kc = pools[0][0]
    gb = kc.stride(0) * kc.element_size()
    ko = outs[0]
    if ids.size * gb * (2 if widen else 1) > ko.numel() * ko.element_size():
        return None
    blk = torch.tensor(ids, dtype=torch.int64, device=dev)
    sets = [(k, v, outs[0].view(-1), outs[1].view(-1)) for k, v in pools]
    return sets, blk, ("widen",) if widen else ("gather",)


def build_config(name: str, dev, layers_override=None, table_fmt="packed",
                 write_entry="launch", fp8="e4m3", scales="tensor", layout=None,
                 heads=None, c3_seqs=16, c3_order="random", c3_gathers=False,
                 c2_order="random", c3_shift=0, head_dim=None, block_size=None) -> Built:
    import numpy as np
    import torch

    from kvx_amd import abi, paged, workloads as W
    from kvx_amd.abi import DType, Layout

    lib = abi.load()
    tdt = {DType.BF16: torch.bfloat16, DType.F16: torch.float16,
           DType.F8_E4M3: torch.float8_e4m3fn, DType.F8_E5M2: torch.float8_e5m2}
    if name == "c3":
        w = W.c3_llama8b_prefill(seqs=c3_seqs, order=c3_order, shift=c3_shift,
                                 block_size=block_size or 16)
    elif name == "c2":
        w = W.c2_llama8b_decode(order=c2_order, block_size=block_size or 16)
    elif name == "c4":
        w = W.c4_llama8b_fp8(block_size=block_size or 16)
    else:
        w = W.CONFIGS[name]()
    keep = []  # keeps every buffer and descriptor alive
    if (fp8 != "e4m3" or scales != "tensor") and name != "c4":
        raise SystemExit("--fp8 / --scales apply to c4")
    if scales != "tensor" and write_entry == "torch_op":
        raise SystemExit("the torch op takes per-tensor scales")
    if fp8 == "e5m2":
        w.cache_dtype = DType.F8_E5M2
        w.name = w.name.replace("fp8_e4m3", "fp8_e5m2")
    if scales != "tensor":
        w.name = f"{w.name}_scale_{scales}"
    # larger rows fit when fewer layers (c2 / c4) or c3's single write leave room
    room = 1.0
    if name in ("c2", "c4") and layers_override:
        room = max(1.0, w.layers / layers_override)
    elif name == "c3":
        room = 4.0
    reshape_rows(w, name, heads, head_dim, room)
    if block_size is not None and name not in ("c2", "c3", "c4"):
        raise SystemExit("--block-size applies to c2, c3 and c4")
    if layout is not None:
        if name not in ("c2", "c3", "c5"):
            raise SystemExit("--layout applies to c2, c3 and c5")
        if write_entry == "torch_op":
            raise SystemExit("--layout combines with the launch entry")
        if table_fmt == "kv_offsets" and layout == "vllm":
            raise SystemExit("KV_OFFSETS pools hold K and V blocks of one layout")
        lay = {"nhd": (Layout.BLOCK_NHD, Layout.BLOCK_NHD),
               "hnd": (Layout.BLOCK_HND, Layout.BLOCK_HND),
               "packed": (Layout.BLOCK_HND_PACKED, Layout.BLOCK_HND_PACKED),
               "vllm": (Layout.BLOCK_HND_PACKED, Layout.BLOCK_CUSTOM)}[layout]
        w.k_layout, w.v_layout = lay
        w.name = f"{w.name}_{layout}"

    if table_fmt != "packed" and name == "c3":
        raise SystemExit("c3 has no gather: --table applies to c1, c2, c4, c5")
    if write_entry == "torch_op" and name == "c3":
        raise SystemExit("the torch op writes vLLM's NHD caches; c3's K is x-packed")
    op = None
    if write_entry == "torch_op":
        from kvx_amd import torch_ops

        torch_ops.load()
        op = torch.ops._C_cache_ops.reshape_and_cache_flash_kvx

    def fill(t):
        if t.dtype in (torch.float8_e4m3fn, torch.float8_e5m2):
            t.view(torch.uint8).random_(0, 256)
        else:
            t.normal_()

    def cache_for(wl):
        """(cache the write uses, cache the gather uses)"""
        if table_fmt == "kv_offsets":
            pool, pc = paged.alloc_block_pool(wl.num_blocks, wl.block_size, wl.heads,
                                              wl.head_dim, tdt[wl.cache_dtype], dev,
                                              wl.k_layout, wl.pack)
            fill(pool.key_cache)
            return pc, pool
        if wl.v_layout == Layout.BLOCK_CUSTOM:  # --layout vllm
            kc = torch.empty(paged.cache_shape(wl.k_layout, wl.num_blocks, wl.block_size,
                                               wl.heads, wl.head_dim, wl.pack),
                             dtype=tdt[wl.cache_dtype], device=dev)
            vstore = torch.empty((wl.num_blocks, wl.heads, wl.head_dim, wl.block_size),
                                 dtype=tdt[wl.cache_dtype], device=dev)
            pc = paged.PagedCache(kc, paged.custom_view(vstore, "bhdo"), wl.k_layout,
                                  wl.v_layout, wl.num_blocks, wl.block_size, wl.heads,
                                  wl.head_dim)
        else:
            pc = paged.alloc_cache(wl.num_blocks, wl.block_size, wl.heads, wl.head_dim,
                                   tdt[wl.cache_dtype], dev, wl.k_layout, wl.v_layout,
                                   wl.pack)
        for t in (pc.key_cache, pc.value_cache):
            fill(t)
        return pc, pc

    def rows(wl, sigma=1.0):
        x = torch.empty((wl.num_tokens, wl.heads, wl.head_dim), dtype=tdt[wl.io_dtype],
                        device=dev)
        return x.normal_(0.0, sigma)

    slots = torch.tensor(w.slots, device=dev)
    lens = torch.tensor(w.seq_lens, device=dev)
    offsets = None
    if table_fmt == "ragged":
        indices, indptr = W.ragged_table(w)
        table = paged.RaggedTable(torch.tensor(indices, device=dev),
                                  torch.tensor(indptr, device=dev))
        keep += [table.indices, table.indptr]
    elif table_fmt == "kv_offsets":
        offsets = torch.tensor(W.kv_offsets_table(w), device=dev)
        table = None  # one OffsetsTable per pool, built in gather_launch
        keep.append(offsets)
    else:
        table = torch.tensor(w.block_table, device=dev)
        keep.append(table)
    keep += [slots, lens]
    wbytes, gbytes = W.write_bytes(w), W.gather_bytes(w, table_fmt)
    if scales != "tensor":
        # scale reads replace the two per-tensor f32 values already counted
        per_blk = {"head": 0, "block": 1, "block_head": w.heads}[scales]
        per_tensor = w.heads if scales == "head" else 0
        wbytes += 8 * (per_tensor + per_blk * w.valid_write_tokens()) - 8
        gbytes += 8 * (per_tensor + per_blk * int(W.gathered_blocks(w))) - 8
    wtok, gtok = w.valid_write_tokens(), w.gathered_tokens()
    steps = []  # list of per-step launch lists (rotated by step index)

    def write_launch(pc, key, val, ks=None, vs=None):
        if op is not None:
            # the op writes on torch's current stream (the bench stream)
            one = torch.ones(1, dtype=torch.float32, device=dev)
            kvd = ("fp8_e5m2" if fp8 == "e5m2" else "fp8") if ks is not None else "auto"
            args = (key, val, pc.key_cache, pc.value_cache, slots, kvd,
                    one if ks is None else ks, one if vs is None else vs)
            keep.extend([pc, key, val, one])

            def call(_stream):
                op(*args)
                return 0

            return Launch("write", call, (), wbytes, wtok)
        cd = pc.desc()
        wd = paged.build_write(pc, key, val, slots, ks, vs)
        keep.extend([pc, key, val, cd, wd])
        if w.tokens_per_seq:
            return Launch("write", lib.kvx_launch_write_kv_prefill,
                          (C.byref(cd), C.byref(wd), w.tokens_per_seq), wbytes, wtok)
        return Launch("write", lib.kvx_launch_write_kv, (C.byref(cd), C.byref(wd)),
                      wbytes, wtok)

    def gather_launch(pc, ko, vo, ks=None, vs=None):
        tb = paged.pool_table(pc, offsets) if table_fmt == "kv_offsets" else table
        cd = paged.gather_cache_desc(pc, tb)
        gd = paged.build_gather(ko, vo, tb, lens, w.max_seq_len)
        keep.extend([cd, gd, tb])
        if ks is not None:
            ksd, vsd = paged.scale_desc_of(ks), paged.scale_desc_of(vs)
            keep.extend([ksd, vsd])
            return Launch("gather", lib.kvx_launch_gather_kv_dequant,
                          (C.byref(cd), C.byref(gd), C.byref(ksd), C.byref(vsd)),
                          gbytes, gtok)
        return Launch("gather", lib.kvx_launch_gather_kv, (C.byref(cd), C.byref(gd)),
                      gbytes, gtok)

    extra = {}
    if name in ("c1", "c2", "c4"):
        layers = layers_override or w.layers
        out_dt = tdt[w.io_dtype]
        ko = torch.empty((w.seq_count, w.max_seq_len, w.heads, w.head_dim), dtype=out_dt,
                         device=dev)
        vo = torch.empty_like(ko)
        keep += [ko, vo]
        ks = vs = None
        if name == "c4":
            g = torch.Generator(device=dev).manual_seed(w.notes["calibration_seed"])
            cal_k = torch.randn((w.num_tokens, w.heads, w.head_dim), generator=g,
                                device=dev) * 2.0
            cal_v = torch.randn((w.num_tokens, w.heads, w.head_dim), generator=g,
                                device=dev) * 2.0
            top = 57344.0 if fp8 == "e5m2" else 448.0
            ks = (cal_k.abs().max() / top).reshape(1).float()
            vs = (cal_v.abs().max() / top).reshape(1).float()
            extra["scales"] = (float(ks.item()), float(vs.item()))
            if scales != "tensor":
                # per-head amax / top, and (block kinds) a seeded per-block factor
                gs = torch.Generator(device=dev).manual_seed(w.notes["calibration_seed"] + 1)
                hk = cal_k.abs().amax(dim=(0, 2)) / top
                hv = cal_v.abs().amax(dim=(0, 2)) / top
                nb = w.num_blocks * (2 if table_fmt == "kv_offsets" else 1)
                fk = torch.rand((nb, 1), generator=gs, device=dev) + 0.5
                fv = torch.rand((nb, 1), generator=gs, device=dev) + 0.5
                vals = {"head": (hk, hv),
                        "block": ((fk * ks).reshape(nb), (fv * vs).reshape(nb)),
                        "block_head": (fk * hk, fv * hv)}[scales]
                gran = {"head": abi.ScaleGranularity.PER_HEAD,
                        "block": abi.ScaleGranularity.PER_BLOCK,
                        "block_head": abi.ScaleGranularity.PER_BLOCK_HEAD}[scales]
                ks = paged.Scales(vals[0].float().contiguous(), gran)
                vs = paged.Scales(vals[1].float().contiguous(), gran)
            keep += [ks, vs]
        step = []
        pools = []
        for _ in range(layers):
            pc, gc = cache_for(w)
            sigma = w.notes.get("io_sigma", 1.0)
            step.append(write_launch(pc, rows(w, sigma), rows(w, sigma), ks, vs))
            step.append(gather_launch(gc, ko, vo, ks, vs))
            pools.append((gc.key_cache, gc.value_cache))
        steps.append(step)
        if (table_fmt == "packed" and w.cache_dtype == w.io_dtype
                and w.k_layout == w.v_layout == Layout.BLOCK_NHD):
            # the gather's valid rows are a plain copy's worth of each pool
            n = np.minimum(np.maximum(w.seq_lens.astype(np.int64), 0), w.max_seq_len)
            extra["pool_copy"] = (pools, (ko, vo), int(n.sum()) * w.heads * w.head_dim
                                  * W.dtype_bytes(w.cache_dtype))
        if table_fmt == "packed" and w.k_layout == w.v_layout == Layout.BLOCK_NHD:
            gran = gather_granules(w, pools[:4], (ko, vo), dev)
            if gran is not None:
                keep.append(gran[1])
                extra["granules"] = gran
        cfg = {"layers": layers}
    elif name == "c3":
        # four rotating buffer sets (> the 256 MB Infinity Cache)
        gathers = []
        sets = []
        for _ in range(4):
            pc, _ = cache_for(w)
            key, val = rows(w), rows(w)
            steps.append([write_launch(pc, key, val)])
            sets.append((pc.key_cache, pc.value_cache, key, val))
            if c3_gathers:
                # the PACKED gather of the same table back into this set's
                # io buffers, [S, 2048, H, D]: it returns the rows just written
                shape = (w.seq_count, w.max_seq_len, w.heads, w.head_dim)
                gathers.append(gather_launch(pc, key.view(shape), val.view(shape)))
        extra["gathers"] = gathers
        # the granule probe's block map: group g of bs tokens fills block
        # slots[g * bs] / bs (chunks that start on a block boundary)
        bs = w.block_size
        grp = w.slots.reshape(-1, bs) if w.num_tokens % bs == 0 else None
        if (grp is not None and c3_shift == 0 and (grp >= 0).all()
                and (grp == grp[:, :1] + np.arange(bs)).all() and (grp[:, 0] % bs == 0).all()):
            blk = torch.tensor(grp[:, 0] // bs, dtype=torch.int64, device=dev)
            keep.append(blk)
            extra["granules"] = (sets, blk, ("scatter", "gather"))
        cfg = {"buffer_sets": 4, "block_order": c3_order}
    else:  # c5
        pc, gc = cache_for(w)
        ko = torch.empty((w.seq_count, w.max_seq_len, w.heads, w.head_dim),
                         dtype=torch.bfloat16, device=dev)
        vo = torch.empty_like(ko)
        keep += [ko, vo]
        steps.append([write_launch(pc, rows(w), rows(w)), gather_launch(gc, ko, vo)])
        cfg = {"layers": 1, "pool_bytes": 2 * pc.key_cache.numel() * pc.key_cache.element_size()}
        if table_fmt == "packed" and w.k_layout == w.v_layout == Layout.BLOCK_NHD:
            n = np.minimum(np.maximum(w.seq_lens.astype(np.int64), 0), w.max_seq_len)
            extra["pool_copy"] = ([(gc.key_cache, gc.value_cache)], (ko, vo),
                                  int(n.sum()) * w.heads * w.head_dim * 2)
            gran = gather_granules(w, [(gc.key_cache, gc.value_cache)], (ko, vo), dev)
            if gran is not None:
                keep.append(gran[1])
                extra["granules"] = gran
    torch.cuda.synchronize()
    if table_fmt != "packed":
        w.name = f"{w.name}_{table_fmt}"
    if name == "c4":
        cfg.update({"fp8": fp8, "scales": scales})
    cfg.update({"workload": w.name, "table": table_fmt, "write_entry": write_entry,
                "seed": w.seed, "heads": w.heads,
                "head_dim": w.head_dim, "block_size": w.block_size,
                "num_tokens": w.num_tokens, "seq_count": w.seq_count,
                "max_seq_len": w.max_seq_len, "pool_blocks": w.num_blocks,
                "cache_dtype": w.cache_dtype.name, "io_dtype": w.io_dtype.name,
                "k_layout": w.k_layout.name, "v_layout": w.v_layout.name})
    return Built(w, steps, cfg, keep, extra)


# ---------------------------------------------------------------------------
# Timing.

def time_launches(steps, K, W, stream):
    """W untimed warmup steps, then K steps with one HIP event after every
    launch: a launch's time runs from the event before it (the previous
    launch's, or the region's start) to its own, so it includes the gap
    after the previous kernel.  One event per launch instead of a pair
    around each: every event record on the stream costs the timed region
    time of its own (c2, same process: 49.58 ms per step with a pair around
    every launch, 49.25 with a pair around each gather only, 49.05 with
    none).  Returns (total ms, [(ms, launch)], wall seconds)."""
    import torch

    sh = stream.cuda_stream
    for i in range(W):
        for launch in steps[i % len(steps)]:
            launch(sh)
    torch.cuda.synchronize()
    per_step = [steps[i % len(steps)] for i in range(K)]
    evs = [torch.cuda.Event(enable_timing=True) for _ in range(sum(len(s) for s in per_step))]
    t_start = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    k = 0
    order = []
    for s in per_step:
        for launch in s:
            launch(sh)
            evs[k].record(stream)
            order.append(launch)
            k += 1
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    timed, prev = [], t_start
    for e, l in zip(evs, order):
        timed.append((prev.elapsed_time(e), l))
        prev = e
    return t_start.elapsed_time(evs[-1]), timed, wall


def summarize(ms_total, timed, K):
    """Whole-step and per-kernel figures of one timed region."""
    ms_per_step = ms_total / K
    by_kind = {}
    for ms, launch in timed:
        by_kind.setdefault(launch.kind, []).append((ms, launch))
    step_bytes = sum(l.nbytes for _, l in timed) / K
    step_tokens = {}
    for _, l in timed:
        step_tokens[l.kind] = step_tokens.get(l.kind, 0) + l.tokens / K
    value = step_bytes / (ms_per_step / 1e3) / 1e9
    kernels = {}
    for kind, lst in by_kind.items():
        ms = [x for x, _ in lst]
        mean_ms = statistics.fmean(ms)
        med_ms = statistics.median(ms)
        nbytes = lst[0][1].nbytes
        gbps = nbytes / (mean_ms / 1e3) / 1e9
        per_step = max(1, len(ms) // K)  # launches of this kind per step: c1/c2/c4 layers
        kernels[kind] = {
            "launches": len(ms), "mean_ms": round(mean_ms, 5),
            "median_ms": round(med_ms, 5),
            "by_position_ms": [round(statistics.fmean(ms[j::per_step]), 5)
                               for j in range(per_step)],
            "bytes_per_launch": nbytes,
            "GBps": round(gbps, 1),
            "GBps_median": round(nbytes / (med_ms / 1e3) / 1e9, 1),
            "frac": round(gbps / PEAK_HBM_GBS, 4),
            "tokens_per_s": round(lst[0][1].tokens / (mean_ms / 1e3), 1),
        }
    dom = max(kernels, key=lambda k_: kernels[k_]["mean_ms"] * kernels[k_]["launches"])
    return {"ms_per_step": round(ms_per_step, 4), "value": round(value, 1),
            "pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
            "tokens_per_s": {k_: round(v / (ms_per_step / 1e3), 1)
                             for k_, v in step_tokens.items()},
            "kernels": kernels, "dominant": dom}


# ---------------------------------------------------------------------------
# Streaming ceilings (libkvx_amd_probe.so).

class Probe:
    """Plain copy / read / write kernels over byte counts beyond the
    Infinity Cache: the best stream of this box, beside the KV kernels."""

    OPS = ("copy", "read", "write", "widen")

    def __init__(self):
        from kvx_amd import build as kbuild

        if not kbuild.PROBE_LIB.exists():
            raise RuntimeError(f"{kbuild.PROBE_LIB} is not built (python -m kvx_amd.build)")
        L = C.CDLL(str(kbuild.PROBE_LIB))
        vp, i64, i = C.c_void_p, C.c_int64, C.c_int
        L.kvx_probe_copy.argtypes = [vp, vp, i64, i, vp]
        L.kvx_probe_read.argtypes = [vp, i64, vp, i, vp]
        L.kvx_probe_write.argtypes = [vp, i64, C.c_uint32, i, vp]
        L.kvx_probe_widen.argtypes = [vp, vp, i64, i, vp]
        L.kvx_probe_shape.argtypes = [i, C.POINTER(i), C.POINTER(i)]
        L.kvx_probe_granules.argtypes = [vp, vp, i64, vp, i, i, i, vp]
        L.kvx_probe_granules_widen.argtypes = [vp, vp, i64, vp, i, i, vp]
        self.L = L
        self.shapes = []
        for k in range(L.kvx_probe_shapes()):
            t, u = C.c_int(), C.c_int()
            L.kvx_probe_shape(k, C.byref(t), C.byref(u))
            self.shapes.append((t.value, u.value))

    def ceiling(self, nbytes, stream, reps=4, rotate_bytes=1 << 30):
        """Per op: {bytes moved per launch, GB/s of the fastest shape, that
        shape (threads, chunks per lane), mean us}.  Copy moves 2 * nbytes
        (read + write); read and write move nbytes; widen reads w = 2/3 of
        nbytes (rounded to 16 bytes) as 8-byte chunks and writes each as a
        16-byte chunk, moving 3 * w (about 2 * nbytes, the copy's bytes) in
        the FP8 dequantizing gather's 1:2 mix.  Launches rotate over buffer pairs
        covering at least `rotate_bytes` per side, so that each one's data
        has left L2 and the Infinity Cache before it is reused; every pair
        runs at least `reps` times per (op, shape)."""
        import torch

        nbytes = max(16, nbytes // 16 * 16)
        wbytes = max(16, 2 * nbytes // 3 // 16 * 16)  # widen's read bytes
        pairs = max(1, min(1024, -(-rotate_bytes // nbytes)))
        cycles = max(1, -(-reps // pairs))
        src_all = torch.empty(pairs * nbytes, dtype=torch.uint8, device="cuda").fill_(3)
        dst_all = torch.empty(2 * pairs * nbytes, dtype=torch.uint8, device="cuda")
        bufs = [(dst_all[2 * i * nbytes:2 * (i + 1) * nbytes],
                 src_all[i * nbytes:(i + 1) * nbytes]) for i in range(pairs)]
        sink = torch.zeros(1024, dtype=torch.uint8, device="cuda")
        sh = stream.cuda_stream
        out = {}
        for op in self.OPS:
            best = None
            every = {}  # "threads x chunks per lane" -> GB/s
            for k, shape in enumerate(self.shapes):
                def one(d, s):
                    if op == "copy":
                        return self.L.kvx_probe_copy(d.data_ptr(), s.data_ptr(), nbytes, k, sh)
                    if op == "read":
                        return self.L.kvx_probe_read(s.data_ptr(), nbytes, sink.data_ptr(), k,
                                                     sh)
                    if op == "widen":
                        return self.L.kvx_probe_widen(d.data_ptr(), s.data_ptr(), wbytes, k, sh)
                    return self.L.kvx_probe_write(d.data_ptr(), nbytes, 7, k, sh)

                for d, s in bufs:
                    if one(d, s) != 0:
                        raise RuntimeError(f"probe {op} shape {shape} failed")
                evs = []
                for _ in range(cycles):
                    for d, s in bufs:
                        e0 = torch.cuda.Event(enable_timing=True)
                        e1 = torch.cuda.Event(enable_timing=True)
                        e0.record(stream)
                        one(d, s)
                        e1.record(stream)
                        evs.append((e0, e1))
                torch.cuda.synchronize()
                ms = statistics.fmean(a.elapsed_time(b) for a, b in evs)
                moved = 3 * wbytes if op == "widen" else {"copy": 2}.get(op, 1) * nbytes
                gbps = moved / (ms / 1e3) / 1e9
                every[f"{shape[0]}x{shape[1]}"] = round(gbps, 1)
                if best is None or gbps > best["GBps"]:
                    best = {"bytes_per_launch": moved, "GBps": round(gbps, 1),
                            "frac": round(gbps / PEAK_HBM_GBS, 4),
                            "shape": list(shape), "mean_us": round(ms * 1e3, 2)}
            best["GBps_by_shape"] = every
            out[op] = best
        out["buffers"] = pairs
        out["footprint_bytes"] = 2 * pairs * nbytes
        del bufs, sink, src_all, dst_all
        torch.cuda.empty_cache()
        return out

    def granules(self, sets, blk, mode, stream, reps=6):
        """The data movement of a paged write ("scatter"), gather ("gather")
        or FP8 -> 16-bit dequantizing gather ("widen": 8-byte reads, each
        stored as one 16-byte chunk) over a config's own block table and
        pools, with no slot, table, layout or conversion work: for every
        buffer set (K pool, V pool, K rows, V rows), one launch moves the K
        rows into (or out of) the pool blocks that `blk` names and one the V
        rows; HIP events time the pair.  Granule = one cache block, whose
        bytes the pool's block stride gives.  Fastest shape: {bytes per
        pair, GB/s, frac, shape, mean us, by shape}."""
        import torch

        kc = sets[0][0]
        gb = kc.stride(0) * kc.element_size()
        if gb & (gb - 1) or gb < 16:
            raise ValueError("granule (block bytes) must be a power of two >= 16")
        glog = gb.bit_length() - 1
        nbytes = blk.numel() * gb  # pool bytes per tensor
        rows_bytes = 2 * nbytes if mode == "widen" else nbytes
        for kp, vp_, kr, vr in sets:
            if min(kr.numel() * kr.element_size(), vr.numel() * vr.element_size()) < rows_bytes:
                raise ValueError("rows shorter than the mapped blocks")
            if int(blk.max()) >= kp.shape[0] or int(blk.max()) >= vp_.shape[0]:
                raise ValueError("block map past a pool")
        sh = stream.cuda_stream
        best, every = None, {}
        for k, shape in enumerate(self.shapes):
            def one(st):
                for pool, rows_ in ((st[0], st[2]), (st[1], st[3])):
                    if mode == "widen":
                        rc = self.L.kvx_probe_granules_widen(rows_.data_ptr(), pool.data_ptr(),
                                                             nbytes, blk.data_ptr(), glog, k, sh)
                    else:
                        rc = self.L.kvx_probe_granules(pool.data_ptr(), rows_.data_ptr(), nbytes,
                                                       blk.data_ptr(), glog,
                                                       int(mode == "scatter"), k, sh)
                    if rc:
                        raise RuntimeError(f"granule probe {mode} shape {shape} failed")
            for st in sets:
                one(st)
            evs = []
            for _ in range(reps):
                for st in sets:
                    e0 = torch.cuda.Event(enable_timing=True)
                    e1 = torch.cuda.Event(enable_timing=True)
                    e0.record(stream)
                    one(st)
                    e1.record(stream)
                    evs.append((e0, e1))
            torch.cuda.synchronize()
            ms = statistics.fmean(a.elapsed_time(b) for a, b in evs)
            moved = 2 * (nbytes + rows_bytes)  # K and V: pool side + rows side
            gbps = moved / (ms / 1e3) / 1e9
            every[f"{shape[0]}x{shape[1]}"] = round(gbps, 1)
            if best is None or gbps > best["GBps"]:
                best = {"bytes_per_launch": moved, "GBps": round(gbps, 1),
                        "frac": round(gbps / PEAK_HBM_GBS, 4), "shape": list(shape),
                        "mean_us": round(ms * 1e3, 2)}
        best["GBps_by_shape"] = every
        return best

    def pool_copy(self, pools, outs, nbytes, shape, stream, reps=3):
        """A plain copy of each layer's own K and V pools (their first
        `nbytes` each) into the gather's output buffers, with the copy
        shape `shape`: the same bytes through the same physical memory as
        that layer's gather, front to back.  {bytes per layer, mean / median
        us over layers, GB/s, frac, us per layer}."""
        import torch

        k = self.shapes.index(tuple(shape))
        ko, vo = outs
        sh = stream.cuda_stream
        for kc, vc in pools:
            if min(kc.numel() * kc.element_size(), vc.numel() * vc.element_size(),
                   ko.numel() * ko.element_size()) < nbytes:
                raise ValueError("pool copy larger than a pool or the output")
        per_layer = [[] for _ in pools]
        for r in range(reps + 1):
            evs = []
            for kc, vc in pools:
                e0 = torch.cuda.Event(enable_timing=True)
                e1 = torch.cuda.Event(enable_timing=True)
                e0.record(stream)
                for src, dst in ((kc, ko), (vc, vo)):
                    if self.L.kvx_probe_copy(dst.data_ptr(), src.data_ptr(), nbytes, k, sh):
                        raise RuntimeError("pool copy failed")
                e1.record(stream)
                evs.append((e0, e1))
            torch.cuda.synchronize()
            if r:  # the first pass warms up
                for j, (e0, e1) in enumerate(evs):
                    per_layer[j].append(e0.elapsed_time(e1) * 1e3)
        us = [statistics.median(x) for x in per_layer]
        mean_us = statistics.fmean(us)
        gbps = 4 * nbytes / (mean_us / 1e6) / 1e9
        return {"bytes_per_launch": 4 * nbytes, "mean_us": round(mean_us, 2),
                "median_us": round(statistics.median(us), 2), "GBps": round(gbps, 1),
                "frac": round(gbps / PEAK_HBM_GBS, 4), "shape": list(shape),
                "by_layer_us": [round(x, 1) for x in us]}


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's fast path on a bounded sample.

def cpu_model() -> str:
    info = {}
    try:
        for line in open("/proc/cpuinfo"):
            if ":" in line:
                k, v = (x.strip() for x in line.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    name = info.get("model name", "unknown")
    extra = [f"family {info.get('cpu family', '?')} model {info.get('model', '?')} "
             f"stepping {info.get('stepping', '?')}"]
    if "hypervisor" in info.get("flags", "").split():
        extra.append("virtual machine")
    return f"{name} ({', '.join(extra)})"


def cpu_baseline(w, seconds: float, sample_seqs: int, gather: bool = True,
                 scales=(0.01, 0.01), table_fmt="packed"):
    """The oracle's fast write (+ gather) over the first `sample_seqs`
    sequences of `w` on a compacted pool (the blocks they use, renumbered),
    timed for about `seconds`; GB/s of the same algorithmic bytes as the GPU
    figures.  FP8 caches use the quantizing / dequantizing fast paths with
    per-tensor scales."""
    import numpy as np

    import oracle
    from kvx_amd import workloads as W
    from kvx_amd.abi import DType, Layout, contiguous_strides
    from kvx_amd.paged import cache_shape

    if Layout.BLOCK_CUSTOM in (w.k_layout, w.v_layout):
        return None  # the sample below builds the canonical layouts only
    n_s = min(w.seq_count, sample_seqs)
    table = w.block_table[:n_s].astype(np.int64)
    ok = (table >= 0) & (table < w.num_blocks)
    used = np.unique(table[ok])
    remap = np.full(int(w.num_blocks), -1, np.int64)
    remap[used] = np.arange(used.size)
    sub_table = np.where(ok, remap[np.where(ok, table, 0)], -1)
    slots = w.slots.astype(np.int64)
    bs = w.block_size
    blk = np.where(slots >= 0, slots // bs, -1)
    keep_tok = (blk >= 0) & np.isin(blk, used)
    sub_slots = np.where(keep_tok, remap[np.maximum(blk, 0)] * bs + slots % bs, -1)
    sub_slots = sub_slots[keep_tok | (slots < 0)]
    sub = W.Workload(w.name + "_cpu_sample", w.seed, w.heads, w.head_dim, bs, int(used.size),
                     w.cache_dtype, w.io_dtype, w.k_layout, w.v_layout, w.pack,
                     sub_slots, w.tokens_per_seq, sub_table.astype(w.block_table.dtype),
                     w.seq_lens[:n_s].copy(), w.max_seq_len)
    cs, is_ = W.dtype_bytes(w.cache_dtype), W.dtype_bytes(w.io_dtype)
    fp8 = w.cache_dtype in (DType.F8_E4M3, DType.F8_E5M2)
    if not fp8 and cs != is_:
        return None
    rng = np.random.default_rng(0)
    E = w.heads * w.head_dim
    blk_elems = bs * E
    kc = rng.integers(0, 255, size=used.size * blk_elems * cs, dtype=np.uint8)
    vc = rng.integers(0, 255, size=used.size * blk_elems * cs, dtype=np.uint8)
    if fp8:
        # N(0, 1) rows in the io dtype (the quantizing write reads numbers)
        def normal_rows():
            x = rng.standard_normal(sub_slots.size * E).astype(np.float32)
            if w.io_dtype == DType.BF16:
                x = (x.view(np.uint32) >> 16).astype(np.uint16)
            elif w.io_dtype == DType.F16:
                x = x.astype(np.float16)
            return x.view(np.uint8)

        key, val = normal_rows(), normal_rows()
    else:
        key = rng.integers(0, 255, size=sub_slots.size * E * is_, dtype=np.uint8)
        val = rng.integers(0, 255, size=sub_slots.size * E * is_, dtype=np.uint8)
    ko = np.zeros(n_s * w.max_seq_len * E * is_ if gather else 0, np.uint8)
    vo = np.zeros_like(ko)

    def geom(layout):
        st = contiguous_strides(cache_shape(layout, used.size, bs, w.heads, w.head_dim,
                                            w.pack))
        return oracle.Geometry(layout, st, w.pack if layout == Layout.BLOCK_HND_PACKED else 1)

    gk, gv = geom(w.k_layout), geom(w.v_layout)
    lens = sub.seq_lens
    tbl = sub.block_table
    common = dict(heads=w.heads, head_dim=w.head_dim, block_size=bs,
                  num_blocks=int(used.size))
    gcommon = dict(common, seq_count=n_s, max_blocks_per_seq=w.max_blocks_per_seq,
                   max_seq_len=w.max_seq_len)

    def once():
        t0 = time.perf_counter()
        if fp8:
            th = oracle.write_kv_quant_fast(gk, gv, key, val, kc, vc, sub_slots,
                                            io_dtype=w.io_dtype, cache_dtype=w.cache_dtype,
                                            k_scale=scales[0], v_scale=scales[1], **common)
            if gather:
                oracle.gather_kv_dequant_fast(gk, gv, kc, vc, ko, vo, tbl, lens,
                                              cache_dtype=w.cache_dtype, io_dtype=w.io_dtype,
                                              k_scale=scales[0], v_scale=scales[1], **gcommon)
        else:
            th = oracle.write_kv_fast(gk, gv, key, val, kc, vc, sub_slots, elem_size=cs,
                                      **common)
            if gather:
                oracle.gather_kv_fast(gk, gv, kc, vc, ko, vo, tbl, lens, elem_size=cs,
                                      **gcommon)
        return time.perf_counter() - t0, th

    once()  # touch every page first
    times, start = [], time.perf_counter()
    threads = 1
    while len(times) < 3 or time.perf_counter() - start < seconds:
        dt, threads = once()
        times.append(dt)
        if len(times) >= 200:
            break
    med = statistics.median(times)
    nbytes = W.write_bytes(sub) + (W.gather_bytes(sub) if gather else 0)
    tokens = sub.valid_write_tokens() + (sub.gathered_tokens() if gather else 0)
    prev = oracle.set_threads(1)
    try:
        one = statistics.median(once()[0] for _ in range(3))
    finally:
        oracle.set_threads(prev)
    what = "write+gather" if gather else "write"
    cast = "; FP8 casts by table lookup" if fp8 else ""
    sample = (f"{w.name} one layer: {'all' if n_s == w.seq_count else f'first {n_s} of'} "
              f"{w.seq_count} sequences (write {sub.valid_write_tokens()} tokens"
              + (f", gather {sub.gathered_tokens()} tokens" if gather else "")
              + f") on a compacted pool of {used.size} blocks; oracle row-memcpy {what}"
              f"{cast}, OpenMP; median of {len(times)} runs")
    if table_fmt != "packed":
        sample += ("; the oracle's fast path reads the PACKED form of this workload's table "
                   "(same rows and bytes)")
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": int(threads),
            "single_thread": {"value": round(nbytes / one / 1e9, 3), "unit": "GB/s",
                              "cores": 1, "seconds_per_run": round(one, 4)},
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "binding": {k: os.environ.get(k) for k in ("OMP_PROC_BIND", "OMP_PLACES")},
            "kind": "port", "sample": sample,
            "tokens_per_s": round(tokens / med, 1),
            "seconds_per_run": round(med, 4)}


# ---------------------------------------------------------------------------
# Extras of the headline.

def write_graph(steps, stream, flush_bytes: int = 1 << 30, reps: int = 10):
    """The workload's cache writes replayed from one HIP graph: every write
    launch of the steps, captured once on the bench stream, so the per-call
    host cost of the launch path is paid at capture only (as under vLLM's
    graph-mode decode).  Before each replay a read of `flush_bytes` (outside
    the timed events) evicts the inputs and the cache rows from L2 and the
    Infinity Cache, so the time per write is that of HBM-resident data."""
    import torch

    writes = [l for s in steps for l in s if l.kind == "write"]
    if not writes:
        return None
    probe = Probe()
    flush = torch.empty(flush_bytes, dtype=torch.uint8, device="cuda").fill_(1)
    sink = torch.zeros(1024, dtype=torch.uint8, device="cuda")
    sh = stream.cuda_stream
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for l in writes:
            l(sh)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    evs = []
    for _ in range(reps):
        if probe.L.kvx_probe_read(flush.data_ptr(), flush_bytes, sink.data_ptr(), 2, sh) != 0:
            raise RuntimeError("flush read failed")
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        g.replay()
        e1.record(stream)
        evs.append((e0, e1))
    torch.cuda.synchronize()
    ms = statistics.fmean(a.elapsed_time(b) for a, b in evs) / len(writes)
    del g, flush, sink
    torch.cuda.empty_cache()
    return {"launches_per_graph": len(writes), "replays": reps,
            "caches": f"flushed before each replay ({flush_bytes >> 20} MiB read)",
            "us_per_write": round(ms * 1e3, 3),
            "GBps": round(writes[0].nbytes / (ms / 1e3) / 1e9, 1)}


def kernel_sources_digest() -> str:
    """sha256 over the kernel sources (the device code and the launch
    planning): a counter summary taken of other sources is stale."""
    from kvx_amd import build as kbuild

    h = hashlib.sha256()
    for name in sorted(["kernels.h", "fp_convert.h", "kvx_internal.h"] +
                       [s for s in kbuild.SOURCES if s.endswith(".hip")]):
        h.update(name.encode())
        h.update((kbuild.CSRC / name).read_bytes())
    return h.hexdigest()


def load_traffic(kind: str, workload: str, algo_bytes: int, root: Path = REPO):
    """HBM bytes per launch from the committed rocprofv3 counter summary of
    this kernel kind and workload (root/profiles), with its file name, or
    (None, reason) when there is none or it was taken of other bytes or
    other kernel sources."""
    rel = f"profiles/traffic_{kind}_{workload}.json"
    p = root / rel
    if not p.exists():
        return None, f"{rel}: none"
    try:
        d = json.loads(p.read_text())
    except (OSError, ValueError):
        return None, f"{rel}: unreadable"
    if d.get("algorithmic_bytes") != algo_bytes:
        return None, f"{rel}: taken of {d.get('algorithmic_bytes')} algorithmic bytes"
    if d.get("kernel_sources_sha256") != kernel_sources_digest():
        return None, f"{rel}: taken of other kernel sources"
    return d.get("bytes_per_launch"), rel


def roofline_of(summary, workload):
    k = summary["kernels"][summary["dominant"]]
    traffic, src = load_traffic(summary["dominant"], workload, k["bytes_per_launch"])
    return {"bound": "hbm", "achieved": k["GBps"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
            "frac": k["frac"], "traffic": traffic, "traffic_source": src,
            "kernel": summary["dominant"],
            "algorithmic_bytes_per_launch": k["bytes_per_launch"],
            "frac_median": round(k["GBps_median"] / PEAK_HBM_GBS, 4)}


def stream_ceilings(b, nbytes, stream):
    """The probe's ceilings for `nbytes` per side, plus (NHD copy gathers)
    the copy of the built config's own pools; holds no reference to the
    pools past its return, so that the caller's `del` frees them."""
    probe = Probe()
    ceiling = probe.ceiling(nbytes, stream)
    if "pool_copy" in b.extra:
        pools, outs, n = b.extra["pool_copy"]
        ceiling["pool_copy"] = probe.pool_copy(pools, outs, n, ceiling["copy"]["shape"],
                                               stream)
    if "granules" in b.extra:
        sets, blk, modes = b.extra["granules"]
        for mode in modes:
            ceiling[f"block_{mode}"] = probe.granules(sets, blk, mode, stream)
    return ceiling


def run_config(name, dev, stream, K, W, args, cpu: bool, **kw):
    """Build, time and summarise one configuration, then free it."""
    import torch

    b = build_config(name, dev, **kw)
    ms_total, timed, wall = time_launches(b.steps, K, W, stream)
    res = summarize(ms_total, timed, K)
    res["roofline"] = roofline_of(res, b.w.name)
    res["config"] = b.cfg
    res["steps"], res["warmup"] = K, W
    res["dtype"] = {"F8_E4M3": "fp8_e4m3", "F8_E5M2": "fp8_e5m2"}.get(
        b.w.cache_dtype.name, b.w.io_dtype.name.lower())
    res["wall_s_timed"] = round(wall, 3)
    extras = {}
    if not args.profile_only:
        dom = res["kernels"][res["dominant"]]
        extras["stream_ceiling"] = stream_ceilings(b, dom["bytes_per_launch"] // 2, stream)
    w, steps = b.w, b.steps
    scales = b.extra.get("scales", (0.01, 0.01))
    del b
    torch.cuda.empty_cache()
    if cpu:
        res["cpu_baseline"] = cpu_baseline(w, args.cpu_seconds, CPU_SAMPLE_SEQS[name],
                                           gather=name != "c3", scales=scales,
                                           table_fmt=kw.get("table_fmt", "packed"))
    res.update(extras)
    return res


def sweep_c3(args, dev, stream):
    """c3's write, the PACKED gather of the same table, and a plain copy of
    the same bytes, at several multiples of c3's size; least-squares fit of
    mean time = intercept + bytes / slope for each."""
    import numpy as np
    import torch

    probe = Probe()
    rows = []
    for n in (int(x) for x in args.sweep_scales.split(",")):
        b = build_config("c3", dev, c3_seqs=16 * n, c3_order=args.c3_order, c3_gathers=True)
        reps = max(8, 64 // n)
        _, tw, _ = time_launches(b.steps, 4 * reps, 4, stream)
        gsteps = [[g] for g in b.extra["gathers"]]
        _, tg, _ = time_launches(gsteps, 4 * reps, 4, stream)
        wbytes, gbytes = b.steps[0][0].nbytes, gsteps[0][0].nbytes
        del b, gsteps
        torch.cuda.empty_cache()
        cp = probe.ceiling(wbytes // 2, stream, reps=max(2, reps // 2))
        wms = [x for x, _ in tw]
        gms = [x for x, _ in tg]
        rows.append({"scale": n, "tokens": 32768 * n,
                     "write": {"bytes": wbytes, "mean_us": round(statistics.fmean(wms) * 1e3, 2),
                               "median_us": round(statistics.median(wms) * 1e3, 2)},
                     "gather": {"bytes": gbytes,
                                "mean_us": round(statistics.fmean(gms) * 1e3, 2),
                                "median_us": round(statistics.median(gms) * 1e3, 2)},
                     "copy": {"bytes": cp["copy"]["bytes_per_launch"],
                              "mean_us": cp["copy"]["mean_us"], "shape": cp["copy"]["shape"]}})
        print(json.dumps(rows[-1]), flush=True)
    fits = {}
    for kind in ("write", "gather", "copy"):
        x = np.array([r[kind]["bytes"] for r in rows], float)
        y = np.array([r[kind]["mean_us"] for r in rows], float)
        if len(rows) >= 2:
            slope_us_per_byte, icpt = np.polyfit(x, y, 1)
            fits[kind] = {"slope_GBps": round(1e-3 / slope_us_per_byte, 1),
                          "slope_frac": round(1e-3 / slope_us_per_byte / PEAK_HBM_GBS, 4),
                          "intercept_us": round(float(icpt), 2)}
    print(json.dumps({"sweep": "c3", "block_order": args.c3_order, "rows": rows,
                      "fit": fits}), flush=True)


# The stdout line stays short: the full figures go to --detail.

def compact_kernel(k):
    return {x: k[x] for x in ("launches", "mean_ms", "median_ms", "bytes_per_launch", "GBps",
                              "frac", "tokens_per_s")}


def compact_ceiling(c):
    if c is None:
        return None
    out = {op: {"GBps": c[op]["GBps"], "frac": c[op]["frac"], "shape": c[op]["shape"]}
           for op in Probe.OPS}
    if "pool_copy" in c:
        pc = c["pool_copy"]
        out["pool_copy"] = {"GBps": pc["GBps"], "frac": pc["frac"], "shape": pc["shape"],
                            "layer_us": [min(pc["by_layer_us"]), max(pc["by_layer_us"])]}
    for op in ("block_scatter", "block_gather", "block_widen"):
        if op in c:
            out[op] = {"GBps": c[op]["GBps"], "frac": c[op]["frac"], "shape": c[op]["shape"]}
    return out


def compact_cpu(c):
    if c is None:
        return None
    return {"value": c["value"], "unit": c["unit"], "cores": c["cores"],
            "single_thread": c["single_thread"]["value"], "kind": c["kind"],
            "cpu_model": c["cpu_model"], "sample": c["sample"]}


def compact_config(r):
    rf = r["roofline"]
    out = {"workload": r["config"]["workload"], "value": r["value"],
           "ms_per_step": r["ms_per_step"],
           "kernels": {k: {x: v[x] for x in ("mean_ms", "median_ms", "GBps", "frac")}
                       for k, v in r["kernels"].items()},
           "roofline": {x: rf[x] for x in ("kernel", "frac", "frac_median", "traffic")}}
    if r.get("stream_ceiling"):
        out["ceiling_frac"] = {op: r["stream_ceiling"][op]["frac"]
                               for op in ("copy", "widen", "pool_copy", "block_scatter",
                                          "block_gather", "block_widen")
                               if op in r["stream_ceiling"]}
    c = r.get("cpu_baseline")
    if c:
        out["cpu_baseline"] = {"value": c["value"], "cores": c["cores"],
                               "single_thread": c["single_thread"]["value"], "kind": c["kind"]}
    return out


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(the paged write/gather shards by KV head or by sequence with no "
              "exchange).  Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)

    if args.copy_probe:
        copy_probe()
        return

    import torch

    dev = torch.device("cuda:0")
    stream = torch.cuda.Stream(device=dev)
    torch.cuda.set_stream(stream)  # launches that use torch's current stream

    if args.sweep:
        sweep_c3(args, dev, stream)
        return

    head = args.config or "c2"
    kw = dict(layers_override=args.layers, table_fmt=args.table,
              write_entry=args.write_entry, fp8=args.fp8, scales=args.scales,
              layout=args.layout, heads=args.heads, c3_seqs=args.c3_seqs,
              c3_order=args.c3_order, c2_order=args.c2_order, c3_shift=args.c3_shift,
              head_dim=args.head_dim, block_size=args.block_size)
    K, W = args.steps, args.warmup
    cpu = not args.no_cpu_baseline and not args.profile_only

    b = build_config(head, dev, **kw)
    ms_total, timed, wall = time_launches(b.steps, K, W, stream)
    res = summarize(ms_total, timed, K)
    roofline = roofline_of(res, b.w.name)
    ceiling = graph = None
    if not args.profile_only:
        dom = res["kernels"][res["dominant"]]
        ceiling = stream_ceilings(b, dom["bytes_per_launch"] // 2, stream)
        graph = write_graph(b.steps, stream)
    w, cfg = b.w, b.cfg
    scales = b.extra.get("scales", (0.01, 0.01))
    del b
    torch.cuda.empty_cache()

    configs = {}
    if args.config is None:
        for name in ("c1", "c3", "c4", "c5"):
            ks = max(K, -(-MIN_LAUNCHES[name] // {"c1": 22, "c4": 32}.get(name, 1)))
            configs[name] = run_config(name, dev, stream, ks, W, args, cpu)
            print(f"config {name}: " + ", ".join(
                f"{k} {v['mean_ms'] * 1e3:.1f} us ({v['frac']:.3f})"
                for k, v in configs[name]["kernels"].items()), file=sys.stderr, flush=True)

    cpu_res = None
    if cpu:
        cpu_res = cpu_baseline(w, args.cpu_seconds, CPU_SAMPLE_SEQS[head],
                               gather=head != "c3", scales=scales, table_fmt=args.table)

    detail = {"kernels": res["kernels"], "roofline": roofline, "stream_ceiling": ceiling,
              "write_graph": graph, "cpu_baseline": cpu_res, "configs": configs}
    if args.detail:
        Path(args.detail).write_text(json.dumps(detail) + "\n")
    out = {
        "metric": METRIC, "value": res["value"], "unit": "GB/s", "n_gpus": 1,
        "steps": K, "warmup": W, "ms_per_step": res["ms_per_step"],
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"F8_E4M3": "fp8_e4m3", "F8_E5M2": "fp8_e5m2"}.get(
            w.cache_dtype.name, w.io_dtype.name.lower()),
        "data": "synthetic",
        "config": cfg,
        "pct_of_peak": res["pct_of_peak"],
        "tokens_per_s": res["tokens_per_s"],
        "kernels": {k: compact_kernel(v) for k, v in res["kernels"].items()},
        "roofline": roofline,
        "stream_ceiling": compact_ceiling(ceiling),
        "write_graph": graph,
        "cpu_baseline": compact_cpu(cpu_res),
        "configs": {name: compact_config(r) for name, r in configs.items()},
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
