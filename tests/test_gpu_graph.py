"""The write and gather entry points captured in a HIP graph and replayed.

vLLM-ROCm captures its decode step, cache writes included, in HIP graphs
and replays it with new contents in the same buffers.  The launch path
therefore has to be capturable: it launches kernels on the caller's stream
and nothing else (no allocation, no host synchronisation, no memset), and
every value that changes between steps (slots, block ids, sequence
lengths, RAGGED offsets, FP8 scales) is read by the kernels from device
memory, not folded into the launch on the host.

Each test captures once, then replays several times.  Before each replay
new inputs are copied into the captured buffers by ordinary eager work;
after it, the caches and outputs are compared byte for byte with the CPU
oracle, which replays the same sequence of writes and gathers on host
copies of every buffer.
"""
import numpy as np
import pytest
import torch

import oracle
from kvx_amd import abi, paged, torch_ops
from kvx_amd.abi import DType, Layout, ScaleGranularity, Status

from gpu_helpers import CacheBuf, CustomBuf, np_bytes, random_fill

pytestmark = pytest.mark.gpu
DEV = "cuda"
REPLAYS = 4


@pytest.fixture(autouse=True, scope="module")
def _load():
    # load the libraries (and register their kernels) before any capture
    abi.load()
    torch_ops.load()


def host(t):
    return np_bytes(t)


def assert_same(got, want, what):
    idx = np.flatnonzero(got != want)
    assert idx.size == 0, f"{what}: {idx.size} bytes differ, first at {idx[:6].tolist()}"


def make_buffers(kind, dtype, nb, bs, H, D, gen):
    """(PagedCache, K buffer, V buffer) for a layout pair: "nhd", or "vllm"
    (K x-packed x = 8, V CUSTOM [num_blocks, H, D, block_size])."""
    if kind == "nhd":
        k = CacheBuf(Layout.BLOCK_NHD, dtype, nb, bs, H, D, 8, DEV, gen)
        v = CacheBuf(Layout.BLOCK_NHD, dtype, nb, bs, H, D, 8, DEV, gen)
        vl = Layout.BLOCK_NHD
    else:
        k = CacheBuf(Layout.BLOCK_HND_PACKED, dtype, nb, bs, H, D, 8, DEV, gen)
        v = CustomBuf(dtype, nb, bs, H, D, "bhdo", gen=gen)
        vl = Layout.BLOCK_CUSTOM
    pc = paged.PagedCache(k.view, v.view, k.layout, vl, nb, bs, H, D)
    return pc, k, v


def decode_inputs(rng, S, L, nb, bs, mbps):
    """Per-replay decode inputs: sequence lengths in [0, L] (some zero or
    past the table), a block table with -1 and out-of-range ids, and one
    new token per sequence at position len - 1 (slot -1 for empty ones)."""
    lens = rng.integers(0, L + 1, size=S).astype(np.int32)
    lens[0] = L
    lens[1] = 0
    table = rng.permutation(nb)[: S * mbps].reshape(S, mbps).astype(np.int32)
    table[rng.random(table.shape) < 0.1] = -1
    table[2, 0] = nb + 3  # out of range: skipped by write and gather
    slots = np.full(S, -1, dtype=np.int64)
    for s in range(S):
        if lens[s] > 0:
            b = table[s, (lens[s] - 1) // bs]
            if b >= 0:
                slots[s] = int(b) * bs + (lens[s] - 1) % bs
    return lens, table, slots


def ragged_of(table, lens, bs, total):
    """RAGGED indices / indptr for the same mapping as a PACKED table
    (token t of sequence s in block table[s, t // bs]), padded to `total`
    indices so the captured buffer keeps its size."""
    idx, ptr = [], [0]
    for s in range(table.shape[0]):
        n = int(lens[s])
        idx.extend(int(table[s, t // bs]) for t in range(n))
        ptr.append(len(idx))
    out = np.full(total, -1, dtype=np.int32)
    out[: len(idx)] = idx
    return out, np.asarray(ptr, dtype=np.int32)


@pytest.mark.parametrize("kind", ["nhd", "vllm"])
@pytest.mark.parametrize("fmt", ["packed", "ragged"])
def test_decode_step_graph_replays(kind, fmt):
    """A decode step (write one token per sequence, then gather every
    sequence) captured once and replayed with new tokens, slots, lengths
    and tables."""
    gen = torch.Generator().manual_seed(7)
    rng = np.random.default_rng(11 + 2 * ["nhd", "vllm"].index(kind) + (fmt == "ragged"))
    nb, bs, H, D, S, L = 96, 16, 2, 64, 6, 80
    mbps = (L + bs - 1) // bs
    dt = DType.BF16
    pc, kb, vb = make_buffers(kind, dt, nb, bs, H, D, gen)
    key = random_fill(torch.empty((S, H, D), dtype=torch.bfloat16, device=DEV), gen)
    value = random_fill(torch.empty_like(key), gen)
    slots = torch.full((S,), -1, dtype=torch.int64, device=DEV)
    lens = torch.zeros(S, dtype=torch.int32, device=DEV)
    table = torch.full((S, mbps), -1, dtype=torch.int32, device=DEV)
    indices = torch.full((S * L,), -1, dtype=torch.int32, device=DEV)
    indptr = torch.zeros(S + 1, dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    tb = table if fmt == "packed" else paged.RaggedTable(indices, indptr)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert paged.write_kv(pc, key, value, slots) == Status.OK
        assert paged.gather_kv(pc, ko, vo, tb, lens, L) == Status.OK
    torch.cuda.synchronize()
    # capture records the launches without running them
    hk, hv, hko, hvo = host(kb.base), host(vb.base), host(ko), host(vo)
    gk, gv = kb.geometry(), vb.geometry()

    for rep in range(REPLAYS):
        ln, tab, sl = decode_inputs(rng, S, L, nb, bs, mbps)
        k_new = rng.integers(0, 1 << 16, size=(S, H, D), dtype=np.uint16)
        v_new = rng.integers(0, 1 << 16, size=(S, H, D), dtype=np.uint16)
        key.view(torch.int16).copy_(torch.from_numpy(k_new.view(np.int16)))
        value.view(torch.int16).copy_(torch.from_numpy(v_new.view(np.int16)))
        slots.copy_(torch.from_numpy(sl))
        lens.copy_(torch.from_numpy(ln))
        table.copy_(torch.from_numpy(tab))
        ind, ptr = ragged_of(tab, ln, bs, S * L)
        indices.copy_(torch.from_numpy(ind))
        indptr.copy_(torch.from_numpy(ptr))
        g.replay()
        torch.cuda.synchronize()

        oracle.write_kv(gk, gv, k_new, v_new, hk, hv, sl, heads=H, head_dim=D, block_size=bs,
                        num_blocks=nb, io_dtype=dt, cache_dtype=dt)
        if fmt == "packed":
            oracle.gather_kv(gk, gv, hk, hv, hko, hvo, tab, ln, seq_count=S,
                             max_blocks_per_seq=mbps, max_seq_len=L, heads=H, head_dim=D,
                             block_size=bs, num_blocks=nb, cache_dtype=dt, io_dtype=dt)
        else:
            oracle.gather_kv_ragged(gk, gv, hk, hv, hko, hvo, ind, ptr, ln, max_seq_len=L,
                                    heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                                    cache_dtype=dt, io_dtype=dt)
        assert_same(host(kb.base), hk, f"replay {rep} key cache")
        assert_same(host(vb.base), hv, f"replay {rep} value cache")
        assert_same(host(ko), hko, f"replay {rep} key out")
        assert_same(host(vo), hvo, f"replay {rep} value out")


@pytest.mark.parametrize("gran", [ScaleGranularity.PER_TENSOR, ScaleGranularity.PER_HEAD])
def test_fp8_write_and_dequant_gather_graph_replays(gran):
    """Quantizing write and dequantizing gather of an FP8 E4M3 cache in one
    graph; the scale values change between replays, so they must be read
    on the device at run time."""
    gen = torch.Generator().manual_seed(3)
    rng = np.random.default_rng(5 + int(gran))
    nb, bs, H, D, S, L = 64, 16, 4, 64, 5, 64
    mbps = L // bs
    pc, kb, vb = make_buffers("nhd", DType.F8_E4M3, nb, bs, H, D, gen)
    key = torch.empty((S, H, D), dtype=torch.bfloat16, device=DEV)
    value = torch.empty_like(key)
    slots = torch.full((S,), -1, dtype=torch.int64, device=DEV)
    lens = torch.zeros(S, dtype=torch.int32, device=DEV)
    table = torch.full((S, mbps), -1, dtype=torch.int32, device=DEV)
    ko = random_fill(torch.empty((S, L, H, D), dtype=torch.bfloat16, device=DEV), gen)
    vo = random_fill(torch.empty_like(ko), gen)
    n = 1 if gran == ScaleGranularity.PER_TENSOR else H
    ksv = torch.ones(n, dtype=torch.float32, device=DEV)
    vsv = torch.ones(n, dtype=torch.float32, device=DEV)
    ks, vs = paged.Scales(ksv, gran), paged.Scales(vsv, gran)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert paged.write_kv(pc, key, value, slots, k_scale=ks, v_scale=vs) == Status.OK
        assert paged.gather_kv(pc, ko, vo, table, lens, L, k_scale=ks, v_scale=vs) == Status.OK
    torch.cuda.synchronize()
    hk, hv, hko, hvo = host(kb.base), host(vb.base), host(ko), host(vo)
    gk, gv = kb.geometry(), vb.geometry()

    for rep in range(REPLAYS):
        ln, tab, sl = decode_inputs(rng, S, L, nb, bs, mbps)
        kx = (rng.standard_normal((S, H, D)) * 3).astype(np.float32)
        vx = (rng.standard_normal((S, H, D)) * 3).astype(np.float32)
        key.copy_(torch.from_numpy(kx).to(torch.bfloat16))
        value.copy_(torch.from_numpy(vx).to(torch.bfloat16))
        k_sc = rng.uniform(0.005, 0.05, size=n).astype(np.float32)
        v_sc = rng.uniform(0.005, 0.05, size=n).astype(np.float32)
        ksv.copy_(torch.from_numpy(k_sc))
        vsv.copy_(torch.from_numpy(v_sc))
        slots.copy_(torch.from_numpy(sl))
        lens.copy_(torch.from_numpy(ln))
        table.copy_(torch.from_numpy(tab))
        g.replay()
        torch.cuda.synchronize()

        if gran == ScaleGranularity.PER_TENSOR:
            ok, ov = float(k_sc[0]), float(v_sc[0])
        else:
            ok, ov = oracle.Scale.per_head(k_sc), oracle.Scale.per_head(v_sc)
        oracle.write_kv(gk, gv, host(key), host(value), hk, hv, sl, heads=H, head_dim=D,
                        block_size=bs, num_blocks=nb, io_dtype=DType.BF16,
                        cache_dtype=DType.F8_E4M3, k_scale=ok, v_scale=ov)
        oracle.gather_kv(gk, gv, hk, hv, hko, hvo, tab, ln, seq_count=S, max_blocks_per_seq=mbps,
                         max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                         cache_dtype=DType.F8_E4M3, io_dtype=DType.BF16, k_scale=ok,
                         v_scale=ov)
        assert_same(host(kb.base), hk, f"replay {rep} key cache")
        assert_same(host(vb.base), hv, f"replay {rep} value cache")
        assert_same(host(ko), hko, f"replay {rep} key out")
        assert_same(host(vo), hvo, f"replay {rep} value out")


def test_prefill_tile_write_graph_replays():
    """The tiled prefill write (K x-packed, V NHD, whole-block chunks)
    captured once.  Later replays spoil some groups (-1 slots, swapped
    offsets, a chunk shifted inside its block), which the kernels route to
    the per-token and two-run paths on the device: the captured launch is
    the same for every slot pattern."""
    gen = torch.Generator().manual_seed(9)
    rng = np.random.default_rng(21)
    nb, bs, H, D = 64, 16, 8, 128
    S, tps = 4, 32
    T = S * tps
    k = CacheBuf(Layout.BLOCK_HND_PACKED, DType.BF16, nb, bs, H, D, 8, DEV, gen)
    v = CacheBuf(Layout.BLOCK_NHD, DType.BF16, nb, bs, H, D, 8, DEV, gen)
    pc = paged.PagedCache(k.view, v.view, k.layout, v.layout, nb, bs, H, D)
    key = torch.empty((T, H, D), dtype=torch.bfloat16, device=DEV)
    value = torch.empty_like(key)
    slots = torch.full((T,), -1, dtype=torch.int64, device=DEV)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        assert paged.write_kv(pc, key, value, slots, tokens_per_seq=tps) == Status.OK
    torch.cuda.synchronize()
    hk, hv = host(k.base), host(v.base)

    for rep in range(REPLAYS):
        blocks = rng.permutation(nb)[: S * tps // bs]
        sl = np.concatenate([b * bs + np.arange(bs) for b in blocks]).astype(np.int64)
        if rep >= 1:
            sl[3] = -1                                   # group 0: an invalid slot
            sl[bs + 4], sl[bs + 5] = sl[bs + 5], sl[bs + 4]  # group 1: swapped offsets
        if rep >= 2:
            # group 2: starts at offset 5 of its block and runs into the next one
            b0, b1 = blocks[2], blocks[3]
            sl[2 * bs: 3 * bs] = np.concatenate([b0 * bs + np.arange(5, bs),
                                                 b1 * bs + np.arange(0, 5)])
            sl[3 * bs: 4 * bs] = -1
        kx = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
        vx = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
        key.view(torch.int16).copy_(torch.from_numpy(kx.view(np.int16)))
        value.view(torch.int16).copy_(torch.from_numpy(vx.view(np.int16)))
        slots.copy_(torch.from_numpy(sl))
        g.replay()
        torch.cuda.synchronize()
        oracle.write_kv(k.geometry(), v.geometry(), kx, vx, hk, hv, sl, heads=H, head_dim=D,
                        block_size=bs, num_blocks=nb, io_dtype=DType.BF16,
                        cache_dtype=DType.BF16)
        assert_same(host(k.base), hk, f"replay {rep} key cache")
        assert_same(host(v.base), hv, f"replay {rep} value cache")


def test_torch_op_graph_replays():
    """torch.ops._C_cache_ops.reshape_and_cache_flash_kvx captured in a
    torch CUDA graph, as vLLM's cudagraph mode captures reshape_and_cache_flash,
    replayed with new rows and slots into vLLM's HND cache view."""
    op = torch.ops._C_cache_ops.reshape_and_cache_flash_kvx
    gen = torch.Generator().manual_seed(4)
    rng = np.random.default_rng(8)
    nb, bs, H, D, T = 32, 16, 4, 64, 24
    kc = torch.empty((nb, H, bs, D), dtype=torch.float16, device=DEV).permute(0, 2, 1, 3)
    vc = torch.empty((nb, H, bs, D), dtype=torch.float16, device=DEV).permute(0, 2, 1, 3)
    for c in (kc, vc):
        random_fill(c.permute(0, 2, 1, 3), gen)
    key = torch.empty((T, H, D), dtype=torch.float16, device=DEV)
    value = torch.empty_like(key)
    slots = torch.full((T,), -1, dtype=torch.int64, device=DEV)
    one = torch.ones(1, dtype=torch.float32, device=DEV)
    torch.cuda.synchronize()

    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        op(key, value, kc, vc, slots, "auto", one, one)
    torch.cuda.synchronize()
    storage = [c.permute(0, 2, 1, 3) for c in (kc, vc)]  # the contiguous [nb, H, bs, D]
    want = [host(s) for s in storage]
    geo = oracle.Geometry(Layout.BLOCK_NHD, kc.stride(), 1)

    for rep in range(REPLAYS):
        sl = rng.permutation(nb * bs)[:T].astype(np.int64)
        sl[rng.random(T) < 0.2] = -1
        kx = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
        vx = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
        key.view(torch.int16).copy_(torch.from_numpy(kx.view(np.int16)))
        value.view(torch.int16).copy_(torch.from_numpy(vx.view(np.int16)))
        slots.copy_(torch.from_numpy(sl))
        g.replay()
        torch.cuda.synchronize()
        oracle.write_kv(geo, geo, kx, vx, want[0], want[1], sl, heads=H, head_dim=D,
                        block_size=bs, num_blocks=nb, io_dtype=DType.F16,
                        cache_dtype=DType.F16)
        assert_same(host(storage[0]), want[0], f"replay {rep} key cache")
        assert_same(host(storage[1]), want[1], f"replay {rep} value cache")
