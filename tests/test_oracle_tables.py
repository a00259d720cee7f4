"""Pins of the oracle's RAGGED and KV_OFFSETS gathers — CPU only.

The two table formats (KVX_SPEC.md:107-122) have no executable counterpart in
the reference (kvx_paged_kv.cu:549-550 returns UNSUPPORTED for them), so the
oracle restatement is pinned by:
  - numpy brute force over shaped per-block views (no stride arithmetic
    shared with the oracle), with -1 / out-of-range ids, short indptr
    ranges, S32/S64 index, indptr and length dtypes, every layout and mixed
    K / V layouts;
  - reduction to the PACKED gather (itself pinned against the reference's
    kernel test and numpy in test_oracle.py): a RAGGED list that expands a
    packed table token by token, and a KV_OFFSETS table whose K and V
    columns both equal the packed table over a pool that is the cache
    tensor, give the packed result bit for bit;
  - the dequantizing variants equal the copy variants followed by the pinned
    scalar dequantize.
"""
import numpy as np
import pytest

import oracle
from kvx_amd.abi import DType, Layout, contiguous_strides
from kvx_amd.paged import cache_shape

from test_oracle import NP_DT, _view_tokens

LAYOUTS = [Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED]


def _geom(layout, shape, pack):
    return oracle.Geometry(layout, contiguous_strides(shape),
                           pack if layout == Layout.BLOCK_HND_PACKED else 1)


def _rand_bytes(rng, n):
    return rng.integers(0, 255, size=n, dtype=np.uint8)


def _case(rng, seed):
    dt = [DType.F32, DType.F16, DType.BF16, DType.F8_E4M3][seed % 4]
    H, D = int(rng.choice([1, 2, 3])), int(rng.choice([4, 8, 16]))
    pack = int(rng.choice([d for d in (1, 2, 4, 8) if D % d == 0]))
    bs, nb = int(rng.choice([1, 2, 4, 8])), int(rng.integers(2, 9))
    kl, vl = rng.choice(LAYOUTS), rng.choice(LAYOUTS)
    return dt, NP_DT[dt], H, D, pack, bs, nb, kl, vl


@pytest.mark.parametrize("seed", range(16))
def test_ragged_vs_numpy(seed):
    rng = np.random.default_rng(100 + seed)
    dt, npdt, H, D, pack, bs, nb, kl, vl = _case(rng, seed)
    es = np.dtype(npdt).itemsize
    kshape = cache_shape(kl, nb, bs, H, D, pack)
    vshape = cache_shape(vl, nb, bs, H, D, pack)
    kc = _rand_bytes(rng, int(np.prod(kshape)) * es).view(npdt)
    vc = _rand_bytes(rng, int(np.prod(vshape)) * es).view(npdt)
    gk, gv = _geom(kl, kshape, pack), _geom(vl, vshape, pack)

    S, L = int(rng.integers(1, 5)), int(rng.integers(1, 3 * bs + 3))
    counts = rng.integers(0, L + 3, size=S)
    idt = [np.int32, np.int64][seed % 2]
    pdt = [np.int32, np.int64][(seed // 2) % 2]
    ldt = [np.int32, np.int64][(seed // 4) % 2]
    indptr = np.concatenate([[0], np.cumsum(counts)]).astype(pdt)
    indices = rng.integers(-1, nb + 2, size=int(indptr[-1])).astype(idt)
    lens = rng.integers(-1, L + 3, size=S).astype(ldt)
    fill = _rand_bytes(rng, S * L * H * D * es)
    ko, vo = fill.copy().view(npdt), fill[::-1].copy().view(npdt)
    want_k = ko.copy().reshape(S, L, H, D)
    want_v = vo.copy().reshape(S, L, H, D)
    ktok = _view_tokens(kc.reshape(kshape), kl, H, D, pack)
    vtok = _view_tokens(vc.reshape(vshape), vl, H, D, pack)
    for s in range(S):
        for i in range(int(indptr[s]), int(indptr[s + 1])):
            t = i - int(indptr[s])
            if t >= L or t >= lens[s]:
                continue
            bid = int(indices[i])
            if 0 <= bid < nb:
                want_k[s, t] = ktok[bid, t % bs].reshape(H, D)
                want_v[s, t] = vtok[bid, t % bs].reshape(H, D)
    oracle.gather_kv_ragged(gk, gv, kc, vc, ko, vo, indices, indptr, lens, max_seq_len=L,
                            heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                            cache_dtype=dt, io_dtype=dt)
    assert np.array_equal(ko.view(np.uint8), want_k.reshape(-1).view(np.uint8))
    assert np.array_equal(vo.view(np.uint8), want_v.reshape(-1).view(np.uint8))


def _pool_blocks(pool: np.ndarray, bpb: int, layout, npdt, bs, H, D, pack):
    """[nblocks, bs, H, D(/x, x)] token views of single-tensor blocks placed
    every `bpb` bytes in a byte pool."""
    shape = cache_shape(layout, 1, bs, H, D, pack)[1:]
    nbytes = int(np.prod(shape)) * np.dtype(npdt).itemsize
    out = []
    for b in range(pool.size // bpb):
        blk = pool[b * bpb: b * bpb + nbytes].view(npdt).reshape(shape)
        out.append(_view_tokens(blk[None], layout, H, D, pack)[0])
    return out


@pytest.mark.parametrize("seed", range(16))
def test_kv_offsets_vs_numpy(seed):
    rng = np.random.default_rng(200 + seed)
    dt, npdt, H, D, pack, bs, nb, kl, vl = _case(rng, seed)
    es = np.dtype(npdt).itemsize
    block_bytes = bs * H * D * es
    bpb = block_bytes + int(rng.choice([0, es, 64]))          # padded pitch allowed
    pools = [_rand_bytes(rng, nb * bpb), _rand_bytes(rng, nb * bpb)]
    with_secondary = seed % 3 != 0
    kblk = [_pool_blocks(p, bpb, kl, npdt, bs, H, D, pack) for p in pools]
    vblk = [_pool_blocks(p, bpb, vl, npdt, bs, H, D, pack) for p in pools]
    gk = _geom(kl, cache_shape(kl, nb, bs, H, D, pack), pack)
    gv = _geom(vl, cache_shape(vl, nb, bs, H, D, pack), pack)

    S, L = int(rng.integers(1, 5)), int(rng.integers(1, 3 * bs + 3))
    mbps = int(rng.integers(1, (L + bs - 1) // bs + 2))
    raw = rng.integers(0, nb + 2, size=(S, 1, 2, mbps)).astype(np.uint32)
    raw |= (rng.random(raw.shape) < 0.4).astype(np.uint32) << 31    # secondary flag
    table = raw.view(np.int32)
    ldt = [np.int32, np.int64][seed % 2]
    lens = rng.integers(-1, L + 3, size=S).astype(ldt)
    fill = _rand_bytes(rng, S * L * H * D * es)
    ko, vo = fill.copy().view(npdt), fill[::-1].copy().view(npdt)
    want = [ko.copy().reshape(S, L, H, D), vo.copy().reshape(S, L, H, D)]
    blocks = [kblk, vblk]
    for s in range(S):
        for t in range(min(L, max(int(lens[s]), 0))):
            if t // bs >= mbps:
                continue
            for kv in range(2):
                r = int(raw[s, 0, kv, t // bs])
                pool, idx = r >> 31, r & 0x7FFFFFFF
                if idx >= nb or (pool == 1 and not with_secondary):
                    continue
                want[kv][s, t] = blocks[kv][pool][idx][t % bs].reshape(H, D)
    oracle.gather_kv_offsets(gk, gv, pools[0], pools[1] if with_secondary else None, bpb,
                             ko, vo, table, lens, max_blocks_per_seq=mbps, max_seq_len=L,
                             heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                             cache_dtype=dt, io_dtype=dt)
    assert np.array_equal(ko.view(np.uint8), want[0].reshape(-1).view(np.uint8))
    assert np.array_equal(vo.view(np.uint8), want[1].reshape(-1).view(np.uint8))


@pytest.mark.parametrize("layout", LAYOUTS)
def test_tables_reduce_to_packed(layout):
    rng = np.random.default_rng(7)
    H, D, pack, bs, nb = 2, 16, 8, 4, 6
    S, L, mbps = 3, 11, 3
    shape = cache_shape(layout, nb, bs, H, D, pack)
    kc = rng.standard_normal(int(np.prod(shape))).astype(np.float32)
    vc = rng.standard_normal(kc.size).astype(np.float32)
    g = _geom(layout, shape, pack)
    table = rng.integers(-1, nb + 1, size=(S, mbps)).astype(np.int32)
    lens = np.array([11, 5, 0], np.int32)
    kw = dict(max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
              cache_dtype=DType.F32, io_dtype=DType.F32)

    def outs():
        return np.full(S * L * H * D, 9.0, np.float32), np.full(S * L * H * D, -9.0, np.float32)

    pk, pv = outs()
    oracle.gather_kv(g, g, kc, vc, pk, pv, table, lens, seq_count=S, max_blocks_per_seq=mbps,
                     **kw)
    # RAGGED: one index per token, indptr over each sequence's padded length
    indices = np.concatenate([[table[s, t // bs] for t in range(mbps * bs)] for s in range(S)])
    indptr = np.arange(S + 1, dtype=np.int64) * mbps * bs
    rk, rv = outs()
    oracle.gather_kv_ragged(g, g, kc, vc, rk, rv, indices.astype(np.int32), indptr, lens, **kw)
    assert np.array_equal(rk, pk) and np.array_equal(rv, pv)
    # KV_OFFSETS: K / V columns equal the packed table (negatives become
    # out-of-range primary indices), pools are the cache tensors
    off = np.where(table < 0, 0x7FFFFFFF, table).astype(np.int32)
    kt = np.stack([off, off], axis=1)[:, None]                      # [S, 1, 2, M]
    bpb = int(np.prod(shape[1:])) * 4
    ok, ov = outs()
    oracle.gather_kv_offsets(g, g, kc.view(np.uint8), None, bpb, ok, np.empty_like(ov), kt,
                             lens, max_blocks_per_seq=mbps, **kw)
    oracle.gather_kv_offsets(g, g, vc.view(np.uint8), None, bpb, np.empty_like(ok), ov, kt,
                             lens, max_blocks_per_seq=mbps, **kw)
    assert np.array_equal(ok, pk) and np.array_equal(ov, pv)


def test_table_dequant_is_copy_then_dequant():
    rng = np.random.default_rng(11)
    H, D, bs, nb, S, L = 2, 8, 4, 5, 2, 9
    shape = cache_shape(Layout.BLOCK_HND, nb, bs, H, D)
    kc = _rand_bytes(rng, int(np.prod(shape)))
    vc = _rand_bytes(rng, kc.size)
    g = _geom(Layout.BLOCK_HND, shape, 1)
    lens = np.array([9, 6], np.int32)
    indptr = np.array([0, 9, 15], np.int32)
    indices = rng.integers(0, nb, size=15).astype(np.int32)
    table = rng.integers(0, nb, size=(S, 1, 2, 3)).astype(np.int32)
    bpb = bs * H * D
    ks, vs = 0.37, 2.5
    for io in (DType.F32, DType.F16, DType.BF16):
        npio = np.uint32 if io == DType.F32 else np.uint16
        n = S * L * H * D
        for fmt in ("ragged", "offsets"):
            bk, bv = np.zeros(n, np.uint8), np.zeros(n, np.uint8)
            dk, dv = np.zeros(n, npio), np.zeros(n, npio)
            common = dict(max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb)
            for o_k, o_v, cdt, idt, sc in ((bk, bv, DType.F8_E4M3, DType.F8_E4M3, (1.0, 1.0)),
                                           (dk, dv, DType.F8_E4M3, io, (ks, vs))):
                if fmt == "ragged":
                    oracle.gather_kv_ragged(g, g, kc, vc, o_k, o_v, indices, indptr, lens,
                                            cache_dtype=cdt, io_dtype=idt, k_scale=sc[0],
                                            v_scale=sc[1], **common)
                else:
                    oracle.gather_kv_offsets(g, g, kc, vc, bpb, o_k, o_v, table, lens,
                                             max_blocks_per_seq=3, cache_dtype=cdt,
                                             io_dtype=idt, k_scale=sc[0], v_scale=sc[1],
                                             **common)
            # every written row is dequant(copied byte); unwritten rows stay 0
            written = np.zeros((S, L), bool)
            written[0, :9] = written[1, :6] = True
            mask = np.repeat(written.reshape(-1), H * D)
            assert np.array_equal(dk[mask], oracle.dequantize_e4m3(bk[mask], ks, io))
            assert np.array_equal(dv[mask], oracle.dequantize_e4m3(bv[mask], vs, io))
            assert not dk[~mask].any() and not dv[~mask].any()


def test_workload_tables_match_packed():
    """kvx_amd.workloads' RAGGED and KV_OFFSETS forms of c1's table gather
    the same rows as the PACKED table (the bench's --table variants)."""
    from kvx_amd import workloads as W

    w = W.c1_tinyllama()
    H, D, bs, nb, L = w.heads, w.head_dim, w.block_size, w.num_blocks, w.max_seq_len
    S = w.seq_count
    rng = np.random.default_rng(1)
    shape = cache_shape(Layout.BLOCK_NHD, nb, bs, H, D)
    kc = _rand_bytes(rng, int(np.prod(shape)) * 2).view(np.uint16)   # f16 bits
    vc = _rand_bytes(rng, kc.nbytes).view(np.uint16)
    g = _geom(Layout.BLOCK_NHD, shape, 1)
    kw = dict(max_seq_len=L, heads=H, head_dim=D, block_size=bs, cache_dtype=DType.F16,
              io_dtype=DType.F16)
    pk, pv = np.zeros(S * L * H * D, np.uint16), np.zeros(S * L * H * D, np.uint16)
    oracle.gather_kv(g, g, kc, vc, pk, pv, w.block_table, w.seq_lens, seq_count=S,
                     max_blocks_per_seq=w.max_blocks_per_seq, num_blocks=nb, **kw)
    indices, indptr = W.ragged_table(w)
    rk, rv = np.zeros_like(pk), np.zeros_like(pv)
    oracle.gather_kv_ragged(g, g, kc, vc, rk, rv, indices, indptr, w.seq_lens, num_blocks=nb,
                            **kw)
    assert np.array_equal(rk, pk) and np.array_equal(rv, pv)
    # one pool holding K of block b at 2b and V at 2b + 1
    pool = np.empty((2 * nb,) + shape[1:], np.uint16)
    pool[0::2], pool[1::2] = kc.reshape(shape), vc.reshape(shape)
    ok, ov = np.zeros_like(pk), np.zeros_like(pv)
    oracle.gather_kv_offsets(g, g, pool.view(np.uint8).reshape(-1), None,
                             int(np.prod(shape[1:])) * 2, ok, ov, W.kv_offsets_table(w),
                             w.seq_lens, max_blocks_per_seq=w.max_blocks_per_seq,
                             num_blocks=2 * nb, **kw)
    assert np.array_equal(ok, pk) and np.array_equal(ov, pv)
    assert W.gather_bytes(w, "ragged") - W.gather_bytes(w) == \
        (indices.size - w.block_table.size) * 4 + (S + 1) * 4


def test_bound_offsets_marks_entries_past_their_pool():
    """The KV_OFFSETS table the pool-bounded gather is checked against:
    entries at or past their pool's count become an index past every pool;
    a count of 0, or one above num_blocks, means num_blocks."""
    from gpu_helpers import bound_offsets

    S = np.uint32(1 << 31)
    X = np.uint32(0x7FFFFFFF)
    raw = np.array([[3, 7 | S, 9, 2 | S], [X, 12, 4 | S, 5 | S]], dtype=np.uint32)
    got = bound_offsets(raw.view(np.int32), 10, (0, 5)).view(np.uint32)
    want = np.array([[3, X, 9, 2 | S], [X, X, 4 | S, X]], dtype=np.uint32)
    assert np.array_equal(got, want)
    got = bound_offsets(raw.view(np.int32), 10, (4, 50)).view(np.uint32)
    want = np.array([[3, 7 | S, X, 2 | S], [X, X, 4 | S, 5 | S]], dtype=np.uint32)
    assert np.array_equal(got, want)
    # no narrowing leaves the table as it is
    assert np.array_equal(bound_offsets(raw.view(np.int32), 13, (0, 0)).view(np.uint32), raw)
