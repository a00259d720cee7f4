"""Pins of the oracle's FP8 paths beyond per-tensor E4M3 — CPU only.

E5M2 casts are pinned in test_oracle.py (torch golden fixtures, special
values, the kernels' own cast source).  Here the element placement and the
scale indexing of the quantizing write and the dequantizing gathers are
pinned against numpy on shaped views: every written byte must equal the
pinned scalar cast (oracle.quantize_fp8 / dequantize_fp8) of its source
element with the scale of its (physical block, head), for per-tensor,
per-head, per-block and per-block-head scales with non-contiguous scale
strides, both FP8 formats, every io dtype and mixed K / V layouts.
"""
import numpy as np
import pytest

import oracle
from kvx_amd.abi import DType, Layout, contiguous_strides
from kvx_amd.paged import cache_shape

from test_oracle import _view_tokens

LAYOUTS = [Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED]
IO_NP = {DType.F32: np.uint32, DType.F16: np.uint16, DType.BF16: np.uint16}


def _geom(layout, shape, pack):
    return oracle.Geometry(layout, contiguous_strides(shape),
                           pack if layout == Layout.BLOCK_HND_PACKED else 1)


def _scales(kind, rng, nb, H):
    """(oracle.Scale, function (b, h) -> float) with padded strides."""
    if kind == "tensor":
        v = float(rng.uniform(0.01, 2.0))
        return v, lambda b, h: v
    if kind == "head":
        buf = rng.uniform(0.01, 2.0, size=3 * H).astype(np.float32)   # stride 3
        return oracle.Scale(buf, 0, 3), lambda b, h: buf[3 * h]
    if kind == "block":
        buf = rng.uniform(0.01, 2.0, size=2 * nb).astype(np.float32)  # stride 2
        return oracle.Scale(buf, 2, 0), lambda b, h: buf[2 * b]
    # block-head stored head-major: element (b, h) at h * nb + b
    buf = rng.uniform(0.01, 2.0, size=nb * H).astype(np.float32)
    return oracle.Scale(buf, 1, nb), lambda b, h: buf[h * nb + b]


def _np_float_bits(x: np.ndarray, io) -> np.ndarray:
    if io == DType.F32:
        return x.astype(np.float32).view(np.uint32)
    if io == DType.F16:
        return x.astype(np.float16).view(np.uint16)
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)   # bf16, RNE
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


@pytest.mark.parametrize("kind", ["tensor", "head", "block", "block_head"])
@pytest.mark.parametrize("fp8", [oracle.E4M3, oracle.E5M2])
@pytest.mark.parametrize("io", [DType.BF16, DType.F16, DType.F32])
def test_scaled_write_and_gather_vs_numpy(kind, fp8, io):
    rng = np.random.default_rng(
        ["tensor", "head", "block", "block_head"].index(kind) * 100 + fp8 * 10 + int(io))
    H, D, bs, nb, pack = 3, 8, 4, 5, 4
    kl, vl = LAYOUTS[int(io) % 3], LAYOUTS[(int(io) + fp8) % 3]
    kshape = cache_shape(kl, nb, bs, H, D, pack)
    vshape = cache_shape(vl, nb, bs, H, D, pack)
    gk, gv = _geom(kl, kshape, pack), _geom(vl, vshape, pack)
    T = 12
    slots = rng.permutation(nb * bs)[:T].astype(np.int64)
    slots[rng.random(T) < 0.2] = -1
    key = _np_float_bits(rng.standard_normal((T, H, D)) * 40, io)
    val = _np_float_bits(rng.standard_normal((T, H, D)) * 3, io)
    ks_o, ks_f = _scales(kind, rng, nb, H)
    vs_o, vs_f = _scales(kind, rng, nb, H)
    kc = rng.integers(0, 255, size=int(np.prod(kshape)), dtype=np.uint8)
    vc = rng.integers(0, 255, size=int(np.prod(vshape)), dtype=np.uint8)
    want_k, want_v = kc.copy(), vc.copy()
    wk = _view_tokens(want_k.reshape(kshape), kl, H, D, pack)
    wv = _view_tokens(want_v.reshape(vshape), vl, H, D, pack)
    for t, slot in enumerate(slots.tolist()):
        if slot < 0:
            continue
        b, o = divmod(slot, bs)
        for h in range(H):
            qk = oracle.quantize_fp8(key[t, h], io, ks_f(b, h), fp8)
            qv = oracle.quantize_fp8(val[t, h], io, vs_f(b, h), fp8)
            wk[b, o, h] = qk.reshape(wk[b, o, h].shape)
            wv[b, o, h] = qv.reshape(wv[b, o, h].shape)
    oracle.write_kv(gk, gv, key, val, kc, vc, slots, heads=H, head_dim=D, block_size=bs,
                    num_blocks=nb, io_dtype=io, cache_dtype=fp8, k_scale=ks_o, v_scale=vs_o)
    assert np.array_equal(kc, want_k) and np.array_equal(vc, want_v)

    # dequantizing gather (PACKED and RAGGED) of random cache bytes
    S, L, mbps = 2, 9, 3
    table = rng.integers(-1, nb, size=(S, mbps)).astype(np.int32)
    lens = np.array([9, 6], np.int32)
    kt = _view_tokens(kc.reshape(kshape), kl, H, D, pack)
    vt = _view_tokens(vc.reshape(vshape), vl, H, D, pack)
    npio = IO_NP[io]
    fill = rng.integers(0, 255, size=S * L * H * D * np.dtype(npio).itemsize, dtype=np.uint8)
    ko, vo = fill.copy().view(npio), fill[::-1].copy().view(npio)
    want_ko = ko.copy().reshape(S, L, H, D)
    want_vo = vo.copy().reshape(S, L, H, D)
    for s in range(S):
        for t in range(lens[s]):
            b = int(table[s, t // bs])
            if b < 0:
                continue
            for h in range(H):
                want_ko[s, t, h] = oracle.dequantize_fp8(kt[b, t % bs, h].reshape(-1),
                                                         ks_f(b, h), io, fp8)
                want_vo[s, t, h] = oracle.dequantize_fp8(vt[b, t % bs, h].reshape(-1),
                                                         vs_f(b, h), io, fp8)
    ko2, vo2 = ko.copy(), vo.copy()
    oracle.gather_kv(gk, gv, kc, vc, ko, vo, table, lens, seq_count=S, max_blocks_per_seq=mbps,
                     max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                     cache_dtype=fp8, io_dtype=io, k_scale=ks_o, v_scale=vs_o)
    assert np.array_equal(ko, want_ko.reshape(-1)) and np.array_equal(vo, want_vo.reshape(-1))
    indices = np.concatenate([[table[s, t // bs] for t in range(L)] for s in range(S)])
    indptr = np.array([0, L, 2 * L], np.int32)
    oracle.gather_kv_ragged(gk, gv, kc, vc, ko2, vo2, indices.astype(np.int32), indptr, lens,
                            max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                            cache_dtype=fp8, io_dtype=io, k_scale=ks_o, v_scale=vs_o)
    assert np.array_equal(ko2, ko) and np.array_equal(vo2, vo)
