"""bench.py's bookkeeping, on the CPU: the provenance rule of
roofline.traffic, the CPU model string, and the streaming-probe library's
launch shapes (no kernel is launched)."""
import json
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO))

import bench  # noqa: E402


def _profile(tmp_path, **fields):
    (tmp_path / "profiles").mkdir(exist_ok=True)
    d = {"bytes_per_launch": 1000, "algorithmic_bytes": 990,
         "kernel_sources_sha256": bench.kernel_sources_digest()}
    d.update(fields)
    (tmp_path / "profiles" / "traffic_gather_wl.json").write_text(json.dumps(d))


def test_traffic_used_only_for_same_bytes_and_sources(tmp_path):
    assert bench.load_traffic("gather", "wl", 990, tmp_path)[0] is None  # no summary
    _profile(tmp_path)
    val, src = bench.load_traffic("gather", "wl", 990, tmp_path)
    assert val == 1000 and src == "profiles/traffic_gather_wl.json"
    val, why = bench.load_traffic("gather", "wl", 991, tmp_path)
    assert val is None and "990" in why
    _profile(tmp_path, kernel_sources_sha256="0" * 64)
    val, why = bench.load_traffic("gather", "wl", 990, tmp_path)
    assert val is None and "other kernel sources" in why


def test_kernel_sources_digest_covers_every_kernel_unit():
    from kvx_amd import build as kbuild

    units = [s for s in kbuild.SOURCES if s.endswith(".hip")]
    assert "dispatch.hip" in units and any(u.startswith("kernels_") for u in units)
    d = bench.kernel_sources_digest()
    assert len(d) == 64 and d == bench.kernel_sources_digest()


def test_committed_traffic_summaries_name_their_workload():
    for p in (REPO / "profiles").glob("traffic_*.json"):
        d = json.loads(p.read_text())
        assert p.name == f"traffic_{d['kind']}_{d['workload']}.json"
        # A prefill chunk that starts inside a block reads up to one block of
        # rows a second time per tile (the block-owning write's speculative
        # loads); every other summary is within 5% of the algorithmic bytes.
        top = 1.3 if "_shift" in d["workload"] else 1.05
        assert 0.99 < d["bytes_per_launch"] / d["algorithmic_bytes"] < top


def test_cpu_model_string():
    m = bench.cpu_model()
    assert m == "unknown" or "family" in m


def test_probe_shapes():
    from kvx_amd import build as kbuild

    if not kbuild.PROBE_LIB.exists():
        pytest.skip("libkvx_amd_probe.so is not built")
    shapes = bench.Probe().shapes
    assert (64, 1) in shapes and (256, 1) in shapes
    assert all(t in (64, 128, 256, 512, 1024) and u in (1, 2, 4) for t, u in shapes)


def test_compact_line_keeps_ceiling_and_pool_copy():
    op = {"GBps": 6600.0, "frac": 0.825, "shape": [64, 1], "mean_us": 1.0,
          "GBps_by_shape": {"64x1": 6600.0}, "bytes_per_launch": 32}
    full = {k: dict(op) for k in bench.Probe.OPS}
    full["buffers"], full["footprint_bytes"] = 4, 128
    full["pool_copy"] = {"GBps": 6700.0, "frac": 0.8375, "shape": [64, 1],
                         "by_layer_us": [1401.0, 1369.0, 1380.5], "mean_us": 1383.5}
    c = bench.compact_ceiling(full)
    assert set(c) == set(bench.Probe.OPS) | {"pool_copy"}
    assert c["pool_copy"]["layer_us"] == [1369.0, 1401.0]
    assert "GBps_by_shape" not in c["copy"] and "by_layer_us" not in c["pool_copy"]
    del full["pool_copy"]
    assert set(bench.compact_ceiling(full)) == set(bench.Probe.OPS)
    assert bench.compact_ceiling(None) is None


def test_reshape_rows():
    from kvx_amd import workloads as W

    w = W.CONFIGS["c5"]()
    name = w.name
    bench.reshape_rows(w, "c5")
    assert (w.heads, w.head_dim, w.name) == (8, 128, name)
    bench.reshape_rows(w, "c5", heads=6)
    assert (w.heads, w.head_dim, w.name) == (6, 128, name + "_h6")
    w = W.CONFIGS["c5"]()
    bench.reshape_rows(w, "c5", heads=12, head_dim=64)
    assert (w.heads, w.head_dim, w.name) == (12, 64, name + "_h12_d64")
    w = W.c3_llama8b_prefill()
    bench.reshape_rows(w, "c3", heads=6)
    assert (w.heads, w.head_dim) == (6, 128)
    w = W.c2_llama8b_decode()
    bench.reshape_rows(w, "c2", 8, 256, room=2.0)
    assert (w.heads, w.head_dim) == (8, 256)
    with pytest.raises(SystemExit):
        bench.reshape_rows(W.c2_llama8b_decode(), "c2", 8, 256)
    for name_, h, d in [("c1", 4, None), ("c5", 12, 128), ("c5", None, 84), ("c5", 0, None)]:
        with pytest.raises(SystemExit):
            bench.reshape_rows(W.CONFIGS["c5"](), name_, h, d)


def test_c2_block_size_keeps_lengths():
    from kvx_amd import workloads as W

    a, b = W.c2_llama8b_decode(), W.c2_llama8b_decode(block_size=128)
    assert (a.seq_lens == b.seq_lens).all() and b.name == a.name + "_bs128"
    assert b.num_blocks == int(((b.seq_lens.astype("int64") + 127) // 128).sum())
    assert sorted(b.block_table[b.block_table >= 0].tolist()) == list(range(b.num_blocks))
    with pytest.raises(ValueError):
        W.c2_llama8b_decode(block_size=48)


def test_c3_block_size_keeps_chunks():
    from kvx_amd import workloads as W

    a, b = W.c3_llama8b_prefill(), W.c3_llama8b_prefill(block_size=128)
    assert (a.name, a.num_blocks, a.block_table.shape) == (
        "c3_llama3_8b_prefill_packedK_bf16", 8192, (16, 128))
    assert b.name == a.name + "_bs128" and b.num_blocks == 1024 and b.block_table.shape == (16, 16)
    assert W.write_bytes(a) == W.write_bytes(b)
    assert len(set(b.slots.tolist())) == b.slots.size and (b.slots // 128 < 1024).all()
    with pytest.raises(ValueError):
        W.c3_llama8b_prefill(block_size=24)


@pytest.mark.gpu
def test_probe_kernels_move_the_right_bytes():
    """Every launch shape of the streaming probes: copy reproduces its
    source, write fills its range with the value, widen stores each 8-byte
    source chunk twice in one 16-byte chunk, read leaves its sink untouched
    (the sink word is written only for a sentinel the data never produce);
    bytes past each range stay as they were."""
    import torch

    from kvx_amd import build as kbuild

    if not kbuild.PROBE_LIB.exists():
        pytest.skip("libkvx_amd_probe.so is not built")
    p = bench.Probe()
    n = 3 * 4096 + 48  # not a multiple of any workgroup's chunks
    g = torch.Generator().manual_seed(5)
    src = torch.randint(0, 256, (n,), dtype=torch.uint8, generator=g).cuda()
    sh = torch.cuda.current_stream().cuda_stream
    for k, shape in enumerate(p.shapes):
        dst = torch.full((2 * n + 64,), 0xAB, dtype=torch.uint8, device="cuda")
        assert p.L.kvx_probe_copy(dst.data_ptr(), src.data_ptr(), n, k, sh) == 0
        torch.cuda.synchronize()
        assert torch.equal(dst[:n], src), shape
        assert bool((dst[n:] == 0xAB).all()), shape

        dst.fill_(0xAB)
        assert p.L.kvx_probe_widen(dst.data_ptr(), src.data_ptr(), n, k, sh) == 0
        torch.cuda.synchronize()
        pairs = src.view(-1, 8)
        assert torch.equal(dst[:2 * n].view(-1, 16), torch.cat([pairs, pairs], dim=1)), shape
        assert bool((dst[2 * n:] == 0xAB).all()), shape

        dst.fill_(0xAB)
        assert p.L.kvx_probe_write(dst.data_ptr(), n, 0x01020304, k, sh) == 0
        torch.cuda.synchronize()
        want = torch.tensor([4, 3, 2, 1], dtype=torch.uint8, device="cuda").repeat(n // 4)
        assert torch.equal(dst[:n], want) and bool((dst[n:] == 0xAB).all()), shape

        sink = torch.full((1024,), 0x5A, dtype=torch.uint8, device="cuda")
        assert p.L.kvx_probe_read(src.data_ptr(), n, sink.data_ptr(), k, sh) == 0
        torch.cuda.synchronize()
        assert bool((sink == 0x5A).all()), shape
    # sizes that are not a multiple of 16 bytes are refused
    assert p.L.kvx_probe_widen(dst.data_ptr(), src.data_ptr(), 24, 0, sh) == 1


@pytest.mark.gpu
def test_granule_probe_moves_the_mapped_blocks():
    """kvx_probe_granules in every shape: scatter puts granule g of the
    contiguous rows into pool granule map[g] and leaves the other pool
    granules as they were; gather brings them back; sizes that are not a
    whole number of granules are refused."""
    import torch

    from kvx_amd import build as kbuild

    if not kbuild.PROBE_LIB.exists():
        pytest.skip("libkvx_amd_probe.so is not built")
    p = bench.Probe()
    glog, ng, npool = 10, 24, 64  # 1 KiB granules, 24 of a 64-granule pool
    gb = 1 << glog
    g = torch.Generator().manual_seed(9)
    blk = torch.randperm(npool, generator=g)[:ng].to(torch.int64)
    rows = torch.randint(0, 256, (ng * gb,), dtype=torch.uint8, generator=g)
    sh = torch.cuda.current_stream().cuda_stream
    for k, shape in enumerate(p.shapes):
        pool = torch.full((npool * gb,), 0xCD, dtype=torch.uint8, device="cuda")
        lin, m = rows.cuda(), blk.cuda()
        assert p.L.kvx_probe_granules(pool.data_ptr(), lin.data_ptr(), ng * gb, m.data_ptr(),
                                      glog, 1, k, sh) == 0
        torch.cuda.synchronize()
        want = torch.full((npool, gb), 0xCD, dtype=torch.uint8)
        want[blk] = rows.view(ng, gb)
        assert torch.equal(pool.cpu().view(npool, gb), want), shape
        back = torch.zeros_like(lin)
        assert p.L.kvx_probe_granules(pool.data_ptr(), back.data_ptr(), ng * gb, m.data_ptr(),
                                      glog, 0, k, sh) == 0
        torch.cuda.synchronize()
        assert torch.equal(back.cpu(), rows), shape
    assert p.L.kvx_probe_granules(pool.data_ptr(), lin.data_ptr(), gb + 16, m.data_ptr(), glog,
                                  1, 0, sh) == 1


@pytest.mark.gpu
def test_granule_widen_probe_reads_the_mapped_blocks():
    """kvx_probe_granules_widen in every shape: 8-byte chunk i of the mapped
    pool granules is 16-byte chunk i of the output, stored twice over; bytes
    past the output's end stay as they were."""
    import torch

    from kvx_amd import build as kbuild

    if not kbuild.PROBE_LIB.exists():
        pytest.skip("libkvx_amd_probe.so is not built")
    p = bench.Probe()
    glog, ng, npool = 9, 20, 48  # 512-byte granules, 20 of a 48-granule pool
    gb = 1 << glog
    g = torch.Generator().manual_seed(11)
    blk = torch.randperm(npool, generator=g)[:ng].to(torch.int64)
    pool_h = torch.randint(0, 256, (npool * gb,), dtype=torch.uint8, generator=g)
    read = pool_h.view(npool, gb)[blk].reshape(-1, 8)
    want = torch.cat([read, read], dim=1).reshape(-1)
    pool, m = pool_h.cuda(), blk.cuda()
    sh = torch.cuda.current_stream().cuda_stream
    for k, shape in enumerate(p.shapes):
        out = torch.full((2 * ng * gb + 64,), 0xEE, dtype=torch.uint8, device="cuda")
        assert p.L.kvx_probe_granules_widen(out.data_ptr(), pool.data_ptr(), ng * gb, m.data_ptr(),
                                            glog, k, sh) == 0
        torch.cuda.synchronize()
        assert torch.equal(out[:2 * ng * gb].cpu(), want), shape
        assert bool((out[2 * ng * gb:] == 0xEE).all()), shape
    assert p.L.kvx_probe_granules_widen(out.data_ptr(), pool.data_ptr(), gb + 8, m.data_ptr(),
                                        glog, 0, sh) == 1
