"""Pins of the oracle's KVX_LAYOUT_BLOCK_CUSTOM addressing — CPU only.

A CUSTOM cache tensor is the logical axes (block, offset, head, dim), or
(block, offset, head, dim / x, x), placed in memory in any order by its
strides (KVX_SPEC.md:57, :77).  The oracle's write and gather over such
tensors are checked against numpy advanced indexing through np.transpose
views of the storage, which shares no stride arithmetic with the oracle,
for orders with the block axis outermost or not, dims split or not, padded
last axes, -1 / out-of-range slots and block ids; and by reduction: the
CUSTOM orders that spell NHD, HND and HND_PACKED give the bytes of those
layouts' own (separately pinned) paths.
"""
import numpy as np
import pytest

import oracle
from kvx_amd.abi import DType, Layout

from test_oracle import geom

ORDERS = [("bohd", None), ("bhod", None), ("bhdo", None), ("obhd", None), ("hbod", None),
          ("bdho", None), ("dohb", None), ("bhpox", 4), ("bhopx", 2), ("xpbho", 4),
          ("bohpx", 8)]


def custom_storage(order, x, nb, bs, H, D, rng, pad=0):
    """(storage, logical numpy view, oracle geometry) of a uint16 tensor."""
    sizes = {"b": nb, "o": bs, "h": H}
    if x is None:
        sizes["d"] = D
        logical = "bohd"
    else:
        sizes["p"], sizes["x"] = D // x, x
        logical = "bohpx"
    shape = [sizes[a] for a in order]
    shape[-1] += pad
    base = rng.integers(0, 1 << 16, size=shape, dtype=np.uint16)
    view = base[..., : sizes[order[-1]]].transpose([order.index(a) for a in logical])
    g = oracle.Geometry.custom([s // base.itemsize for s in view.strides], D, x)
    return base, view, g


def element_view(view, x):
    """[b, o, h, d] indexing of a logical view (splits d for x-split views)."""
    if x is None:
        return view
    X = view.shape[4]
    d = np.arange(view.shape[3] * X)  # d = p * x + i
    return view[:, :, :, d // X, d % X]


@pytest.mark.parametrize("korder,kx", ORDERS)
def test_custom_write_and_gather_vs_numpy(korder, kx):
    rng = np.random.default_rng(ORDERS.index((korder, kx)) + 900)
    nb, bs, H, D = 5, 4, 3, 8
    vorder, vx = ORDERS[(ORDERS.index((korder, kx)) + 3) % len(ORDERS)]
    kbase, _, gk = custom_storage(korder, kx, nb, bs, H, D, rng, pad=1)
    vbase, _, gv = custom_storage(vorder, vx, nb, bs, H, D, rng)
    T = 14
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    slots[rng.random(T) < 0.2] = -1
    slots[3] = nb * bs + 1  # block past the end
    key = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)

    want_k, want_v = kbase.copy(), vbase.copy()
    ek = want_k[..., : kbase.shape[-1] - 1].transpose(    # K's last axis is padded by 1
        [korder.index(a) for a in ("bohpx" if kx else "bohd")])
    ev = want_v.transpose([vorder.index(a) for a in ("bohpx" if vx else "bohd")])
    for t, slot in enumerate(slots.tolist()):
        b, o = divmod(slot, bs)
        if slot < 0 or b >= nb:
            continue
        for h in range(H):
            for d in range(D):
                ik = (b, o, h, d) if kx is None else (b, o, h, d // kx, d % kx)
                iv = (b, o, h, d) if vx is None else (b, o, h, d // vx, d % vx)
                ek[ik] = key[t, h, d]
                ev[iv] = val[t, h, d]
    kc, vc = kbase.reshape(-1).copy(), vbase.reshape(-1).copy()
    oracle.write_kv(gk, gv, key, val, kc, vc, slots, heads=H, head_dim=D, block_size=bs,
                    num_blocks=nb, io_dtype=DType.BF16, cache_dtype=DType.BF16)
    assert np.array_equal(kc, want_k.reshape(-1))
    assert np.array_equal(vc, want_v.reshape(-1))

    # gather from the written caches, through the numpy views
    kcache = kc.reshape(kbase.shape)
    vcache = vc.reshape(vbase.shape)
    kv = element_view(kcache[..., : kbase.shape[-1] - 1].transpose(
        [korder.index(a) for a in ("bohpx" if kx else "bohd")]), kx)
    vv = element_view(vcache.transpose([vorder.index(a) for a in ("bohpx" if vx else "bohd")]),
                      vx)
    S, L, mbps = 3, 10, 4
    table = rng.integers(-1, nb + 1, size=(S, mbps)).astype(np.int32)
    lens = np.array([10, 7, 13], np.int32)
    ko = rng.integers(0, 1 << 16, size=(S, L, H, D), dtype=np.uint16)
    vo = rng.integers(0, 1 << 16, size=(S, L, H, D), dtype=np.uint16)
    want_ko, want_vo = ko.copy(), vo.copy()
    for s in range(S):
        for t in range(min(int(lens[s]), L)):
            b = int(table[s, t // bs])
            if b < 0 or b >= nb:
                continue
            want_ko[s, t] = kv[b, t % bs]
            want_vo[s, t] = vv[b, t % bs]
    oracle.gather_kv(gk, gv, kc, vc, ko, vo, table, lens, seq_count=S, max_blocks_per_seq=mbps,
                     max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                     cache_dtype=DType.BF16, io_dtype=DType.BF16)
    assert np.array_equal(ko, want_ko) and np.array_equal(vo, want_vo)


@pytest.mark.parametrize("order,x,layout", [("bohd", None, Layout.BLOCK_NHD),
                                            ("bhod", None, Layout.BLOCK_HND),
                                            ("bhpox", 4, Layout.BLOCK_HND_PACKED)])
def test_custom_orders_reduce_to_named_layouts(order, x, layout):
    rng = np.random.default_rng(950)
    nb, bs, H, D = 6, 4, 2, 16
    _, _, gc = custom_storage(order, x, nb, bs, H, D, rng)
    gn = geom(layout, nb, bs, H, D, pack=x or 8)
    T = 20
    slots = rng.permutation(nb * bs)[:T].astype(np.int32)
    slots[::5] = -1
    key = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
    val = rng.integers(0, 1 << 16, size=(T, H, D), dtype=np.uint16)
    init = rng.integers(0, 1 << 16, size=nb * bs * H * D, dtype=np.uint16)
    out = []
    for g in (gc, gn):
        kc, vc = init.copy(), init[::-1].copy()
        oracle.write_kv(g, g, key, val, kc, vc, slots, heads=H, head_dim=D, block_size=bs,
                        num_blocks=nb, io_dtype=DType.F16, cache_dtype=DType.F16)
        out.append((kc, vc))
    assert np.array_equal(out[0][0], out[1][0]) and np.array_equal(out[0][1], out[1][1])
    for g in (gc, gn):
        assert all(oracle.cache_offset(g, b, o, h, d) == oracle.cache_offset(gn, b, o, h, d)
                   for b in (0, 5) for o in range(bs) for h in range(H) for d in (0, 3, 15))
