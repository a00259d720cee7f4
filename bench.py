#!/usr/bin/env python3
"""Benchmark of the KVX paged KV write + gather hot path on one MI355X.

    python bench.py [--steps K] [--warmup W] [--config c2] [--no-cpu-baseline]

Default workload: Llama-3-8B-shaped decode, bf16, 32
layers, 8 KV heads x 128, block_size 16, batch 256, contexts U[512, 8192],
5% of slots -1.  One step = for each of the 32 layers (each with its own
~4.6 GB paged K+V pool): the decode write of 256 new tokens, then the gather
of every sequence's full context into contiguous [256, 8192, 8, 128] K and V
buffers (shared across layers, as an attention workspace would be).  All
inputs are resident in HBM before timing; every launch goes through the
C ABI (kvx_launch_write_kv / kvx_launch_gather_kv) on one HIP stream.

value = algorithmic bytes of the whole step / step time (GB/s, 1e9), where
algorithmic bytes are the bytes a perfect implementation must move: every
valid K/V row read once and written once, plus the index arrays used
(kvx_amd.workloads.write_bytes / gather_bytes).

The roofline entry is for the dominant kernel (the gather): its algorithmic
bytes per launch / its mean launch duration, the duration measured with HIP
events recorded on the launch stream around every gather launch inside the
timed region.  `traffic` is read from the committed rocprofv3 counter
summary (profiles/) when present.

cpu_baseline: the CPU oracle's row-memcpy write + gather (oracle/, OpenMP)
timed on this host's cores over a bounded sample of the same workload.

Outside the timed region: copy_reference (torch's device copy of 1 GiB on
the same stream) and write_graph (the workload's writes captured in one HIP
graph and replayed: device time per write without per-call launch cost).
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import statistics
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO))

METRIC = ("achieved HBM GB/s (% of peak) and tokens/s for KV write+gather, "
          "1 MI355X")
PEAK_HBM_GBS = 8000.0


def parse_args():
    p = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=10)
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--config", default="c2", choices=["c1", "c2", "c3", "c4", "c5"])
    p.add_argument("--table", default="packed", choices=["packed", "ragged", "kv_offsets"],
                   help="block-table format of the gather (c1, c2, c4, c5); kv_offsets "
                        "puts K and V blocks in one TensorRT-LLM-style pool")
    p.add_argument("--write-entry", default="launch", choices=["launch", "torch_op"],
                   help="issue the writes through kvx_launch_write_kv* (ctypes) or the "
                        "PyTorch-ROCm op _C_cache_ops.reshape_and_cache_flash_kvx "
                        "(c1, c2, c4, c5: NHD caches)")
    p.add_argument("--layout", default=None, choices=["nhd", "hnd", "packed", "vllm"],
                   help="c2 / c5: cache layout of K and V (default NHD).  packed: "
                        "HND_PACKED x = 8; vllm: K HND_PACKED x = 8 and V "
                        "KVX_LAYOUT_BLOCK_CUSTOM [num_blocks, H, D, block_size], vLLM's "
                        "paged-attention pair (PACKED / RAGGED tables only)")
    p.add_argument("--heads", type=int, default=None,
                   help="c2 / c5: KV heads per GPU (one tensor-parallel rank's shard: "
                        "8 / TP); the block table, lengths and slots are unchanged")
    p.add_argument("--fp8", default="e4m3", choices=["e4m3", "e5m2"],
                   help="c4: FP8 format of the cache")
    p.add_argument("--scales", default="tensor",
                   choices=["tensor", "head", "block", "block_head"],
                   help="c4: FP8 scale granularity (per tensor, per KV head, per physical "
                        "block, per block and head)")
    p.add_argument("--layers", type=int, default=None,
                   help="override the layer count of c1/c2/c4")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-seconds", type=float, default=10.0,
                   help="CPU baseline sampling budget")
    p.add_argument("--profile-only", action="store_true",
                   help="skip the CPU baseline (profiler runs)")
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


def build_config(name: str, layers_override, dev, table_fmt="packed", write_entry="launch",
                 fp8="e4m3", scales="tensor", layout=None, heads=None):
    import torch

    from kvx_amd import abi, paged, workloads as W
    from kvx_amd.abi import DType, Layout

    lib = abi.load()
    tdt = {DType.BF16: torch.bfloat16, DType.F16: torch.float16,
           DType.F8_E4M3: torch.float8_e4m3fn, DType.F8_E5M2: torch.float8_e5m2}
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
    if heads is not None:
        if name not in ("c2", "c5") or heads <= 0 or w.heads % heads != 0:
            raise SystemExit("--heads applies to c2 and c5 and must divide 8")
        w.heads = heads
        w.name = f"{w.name}_h{heads}"
    if layout is not None:
        if name not in ("c2", "c5"):
            raise SystemExit("--layout applies to c2 and c5")
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
        for _ in range(layers):
            pc, gc = cache_for(w)
            sigma = w.notes.get("io_sigma", 1.0)
            step.append(write_launch(pc, rows(w, sigma), rows(w, sigma), ks, vs))
            step.append(gather_launch(gc, ko, vo, ks, vs))
        steps.append(step)
        cfg = {"layers": layers}
    elif name == "c3":
        # four rotating buffer sets (> the 256 MB Infinity Cache)
        for _ in range(4):
            pc, _ = cache_for(w)
            steps.append([write_launch(pc, rows(w), rows(w))])
        cfg = {"buffer_sets": 4}
    else:  # c5
        pc, gc = cache_for(w)
        ko = torch.empty((w.seq_count, w.max_seq_len, w.heads, w.head_dim),
                         dtype=torch.bfloat16, device=dev)
        vo = torch.empty_like(ko)
        keep += [ko, vo]
        steps.append([write_launch(pc, rows(w), rows(w)), gather_launch(gc, ko, vo)])
        cfg = {"layers": 1}
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
    return w, steps, cfg, keep


# ---------------------------------------------------------------------------
# CPU baseline: the oracle's fast path on a bounded sample.

def cpu_baseline(w, seconds: float):
    import numpy as np

    import oracle
    from kvx_amd import workloads as W
    from kvx_amd.abi import Layout

    n_s = min(w.seq_count, 64)
    table = w.block_table[:n_s].astype(np.int64)
    used = np.unique(table[table >= 0])
    remap = np.full(int(w.num_blocks), -1, np.int64)
    remap[used] = np.arange(used.size)
    sub_table = np.where(table >= 0, remap[np.maximum(table, 0)], -1)
    slots = w.slots.astype(np.int64)
    bs = w.block_size
    # tokens whose slot lands in a sampled sequence's blocks
    blk = np.where(slots >= 0, slots // bs, -1)
    keep_tok = (blk >= 0) & np.isin(blk, used)
    sub_slots = np.where(keep_tok, remap[np.maximum(blk, 0)] * bs + slots % bs, -1)
    sub_slots = sub_slots[keep_tok | (slots < 0)]
    sub = W.Workload(w.name + "_cpu_sample", w.seed, w.heads, w.head_dim, bs, int(used.size),
                     w.cache_dtype, w.io_dtype, w.k_layout, w.v_layout, w.pack,
                     sub_slots, w.tokens_per_seq, sub_table.astype(w.block_table.dtype),
                     w.seq_lens[:n_s].copy(), w.max_seq_len)
    es = W.dtype_bytes(w.cache_dtype)
    if W.dtype_bytes(w.io_dtype) != es:
        return None  # the CPU fast path is a byte copy; no dequant baseline
    if Layout.BLOCK_CUSTOM in (w.k_layout, w.v_layout):
        return None  # the sample below builds canonical layouts only
    rng = np.random.default_rng(0)
    E = w.heads * w.head_dim
    blk_elems = bs * E
    kc = rng.integers(0, 255, size=used.size * blk_elems * es, dtype=np.uint8)
    vc = rng.integers(0, 255, size=used.size * blk_elems * es, dtype=np.uint8)
    key = rng.integers(0, 255, size=sub_slots.size * E * es, dtype=np.uint8)
    val = rng.integers(0, 255, size=sub_slots.size * E * es, dtype=np.uint8)
    ko = np.zeros(n_s * w.max_seq_len * E * es, np.uint8)
    vo = np.zeros_like(ko)
    from kvx_amd.paged import cache_shape
    from kvx_amd.abi import contiguous_strides

    def geom(layout):
        st = contiguous_strides(cache_shape(layout, used.size, bs, w.heads, w.head_dim,
                                            w.pack))
        return oracle.Geometry(layout, st, w.pack if layout == Layout.BLOCK_HND_PACKED else 1)

    gk, gv = geom(w.k_layout), geom(w.v_layout)
    lens = sub.seq_lens
    tbl = sub.block_table

    def once():
        t0 = time.perf_counter()
        th = oracle.write_kv_fast(gk, gv, key, val, kc, vc, sub_slots, heads=w.heads,
                                  head_dim=w.head_dim, block_size=bs,
                                  num_blocks=int(used.size), elem_size=es)
        oracle.gather_kv_fast(gk, gv, kc, vc, ko, vo, tbl, lens, seq_count=n_s,
                              max_blocks_per_seq=w.max_blocks_per_seq,
                              max_seq_len=w.max_seq_len, heads=w.heads,
                              head_dim=w.head_dim, block_size=bs,
                              num_blocks=int(used.size), elem_size=es)
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
    nbytes = W.write_bytes(sub) + W.gather_bytes(sub)
    # the same sample on one thread, three runs
    prev = oracle.set_threads(1)
    try:
        one = statistics.median(once()[0] for _ in range(3))
    finally:
        oracle.set_threads(prev)
    return {"value": round(nbytes / med / 1e9, 3), "unit": "GB/s", "cores": int(threads),
            "single_thread": {"value": round(nbytes / one / 1e9, 3), "unit": "GB/s",
                              "cores": 1, "seconds_per_run": round(one, 4)},
            "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "kind": "port",
            "sample": (f"{w.name} one layer: first {n_s} of {w.seq_count} sequences "
                       f"(gather {sub.gathered_tokens()} tokens, write "
                       f"{sub.valid_write_tokens()} tokens) on a compacted pool of "
                       f"{used.size} blocks; oracle row-memcpy write+gather, OpenMP; "
                       f"median of {len(times)} runs"),
            "tokens_per_s": round((sub.gathered_tokens() + sub.valid_write_tokens()) / med, 1),
            "seconds_per_run": round(med, 4)}


def cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def copy_reference(stream, nbytes: int = 1 << 30, reps: int = 5):
    """torch's device-to-device copy_ of `nbytes` on `stream` (read plus
    write bytes per second): a plain copy beside the roofline, for the same
    box and run."""
    import torch

    a = torch.empty(nbytes // 4, dtype=torch.int32, device="cuda").fill_(7)
    b = torch.empty_like(a)
    with torch.cuda.stream(stream):
        for _ in range(2):
            b.copy_(a)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(reps)]
        for e0, e1 in ev:
            e0.record(stream)
            b.copy_(a)
            e1.record(stream)
    torch.cuda.synchronize()
    ms = statistics.fmean(e0.elapsed_time(e1) for e0, e1 in ev)
    del a, b
    torch.cuda.empty_cache()
    return {"kernel": "torch copy_ device to device", "bytes_per_copy": 2 * nbytes,
            "GBps": round(2 * nbytes / (ms / 1e3) / 1e9, 1), "reps": reps}


def write_graph(steps, stream, reps: int = 10, min_launches: int = 32):
    """The workload's cache writes replayed from a HIP graph: every write
    launch of every step, repeated to at least `min_launches` launches, is
    captured once on the bench stream, so the per-call host cost of the
    launch path (descriptor checks, planning, the launch itself) is paid at
    capture only, as under vLLM's graph-mode decode.  `reps` replays are
    queued back to back between two events, so the device never waits for
    the host; reports the mean device time per write."""
    import torch

    writes = [l for s in steps for l in s if l.kind == "write"]
    if not writes:
        return None
    rounds = -(-min_launches // len(writes))
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=stream):
        for _ in range(rounds):
            for l in writes:
                l(stream.cuda_stream)
    for _ in range(2):
        g.replay()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(reps):
        g.replay()
    e1.record(stream)
    torch.cuda.synchronize()
    n = reps * rounds * len(writes)
    ms = e0.elapsed_time(e1) / n
    del g
    return {"launches_per_graph": rounds * len(writes), "replays": reps,
            "us_per_write": round(ms * 1e3, 3),
            "GBps": round(writes[0].nbytes / (ms / 1e3) / 1e9, 1)}


def load_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 counter summary."""
    p = REPO / "profiles" / f"traffic_{kernel}_{workload}.json"
    if not p.exists():
        return None
    try:
        return json.loads(p.read_text()).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


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
    w, steps, cfg, keep = build_config(args.config, args.layers, dev, args.table,
                                       args.write_entry, args.fp8, args.scales, args.layout,
                                       args.heads)
    stream = torch.cuda.Stream(device=dev)
    sh = stream.cuda_stream
    torch.cuda.set_stream(stream)  # launches that use torch's current stream

    for i in range(args.warmup):
        for launch in steps[i % len(steps)]:
            launch(sh)
    torch.cuda.synchronize()

    K = args.steps
    per_step = [steps[i % len(steps)] for i in range(K)]
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
           for _ in range(sum(len(s) for s in per_step))]
    t_start = torch.cuda.Event(enable_timing=True)
    t_end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    t_start.record(stream)
    k = 0
    kinds = []
    for s in per_step:
        for launch in s:
            e0, e1 = evs[k]
            e0.record(stream)
            launch(sh)
            e1.record(stream)
            kinds.append(launch)
            k += 1
    t_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    ms_total = t_start.elapsed_time(t_end)
    ms_per_step = ms_total / K

    by_kind = {}
    for (e0, e1), launch in zip(evs, kinds):
        by_kind.setdefault(launch.kind, []).append((e0.elapsed_time(e1), launch))
    step_bytes = sum(l.nbytes for s in per_step for l in s) / K
    step_tokens = {}
    for s in per_step:
        for l in s:
            step_tokens[l.kind] = step_tokens.get(l.kind, 0) + l.tokens / K
    value = step_bytes / (ms_per_step / 1e3) / 1e9

    kernels = {}
    for kind, lst in by_kind.items():
        ms = [x for x, _ in lst]
        mean_ms = statistics.fmean(ms)
        nbytes = lst[0][1].nbytes
        kernels[kind] = {
            "launches": len(ms), "mean_ms": round(mean_ms, 5),
            "median_ms": round(statistics.median(ms), 5),
            "bytes_per_launch": nbytes,
            "GBps": round(nbytes / (mean_ms / 1e3) / 1e9, 1),
            "tokens_per_s": round(lst[0][1].tokens / (mean_ms / 1e3), 1),
        }
    dom = max(kernels, key=lambda k_: kernels[k_]["mean_ms"] * kernels[k_]["launches"])
    achieved = kernels[dom]["GBps"]
    roofline = {"bound": "hbm", "achieved": achieved, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(achieved / PEAK_HBM_GBS, 4),
                "traffic": load_traffic(dom, w.name), "kernel": dom,
                "algorithmic_bytes_per_launch": kernels[dom]["bytes_per_launch"]}

    copy_ref = None if args.profile_only else copy_reference(stream)
    graph = None if args.profile_only else write_graph(steps, stream)
    cpu = None
    if not args.no_cpu_baseline and not args.profile_only:
        cpu = cpu_baseline(w, args.cpu_seconds)
        if cpu is not None and args.table != "packed":
            cpu["sample"] += ("; the oracle's fast path reads the PACKED form of this "
                              "workload's table (same rows and bytes)")

    out = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": K, "warmup": args.warmup, "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": {"F8_E4M3": "fp8_e4m3", "F8_E5M2": "fp8_e5m2"}.get(
            w.cache_dtype.name, w.io_dtype.name.lower()),
        "data": "synthetic",
        "config": cfg,
        "pct_of_peak": round(100.0 * value / PEAK_HBM_GBS, 2),
        "tokens_per_s": {k_: round(v / (ms_per_step / 1e3), 1)
                         for k_, v in step_tokens.items()},
        "kernels": kernels,
        "roofline": roofline,
        "copy_reference": copy_ref,
        "write_graph": graph,
        "cpu_baseline": cpu,
        "wall_s_timed": round(wall, 3),
    }
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
