"""Pins of the CPU oracle (oracle/kvx_oracle.c) — CPU only.

The oracle is the checker for every GPU parity test, so it is itself checked
against things it does not share code with:
  - the closed-form cases of the reference's own kernel test
    (tests/kvx_kernel_test.cu:160-786), with the expected offsets computed by
    that test's host loops, made bit-exact;
  - numpy advanced indexing on shaped arrays (a textbook scatter/gather that
    uses the layouts' shapes, not the oracle's stride arithmetic) on random
    small cases with -1 slots, out-of-range blocks, S32/S64 indices, every
    layout, mixed K/V layouts and padded (non-canonical) strides;
  - write -> gather round trips and untouched-region invariants;
  - torch's float8_e4m3fn / bfloat16 / float16 casts (tests/golden fixtures)
    and numpy's float16 cast for the FP8 path;
  - the kernels' own cast source (kvx_amd/csrc/fp_convert.h) compiled for the
    host, across every rounding boundary (tests/fp_convert_check.cpp).
"""
import subprocess
from pathlib import Path

import numpy as np
import pytest

import oracle
from kvx_amd.abi import DType, Layout
from kvx_amd.paged import cache_shape
from kvx_amd.abi import contiguous_strides

from conftest import REPO

GOLDEN = REPO / "tests" / "golden" / "fp8_e4m3_golden.npz"
GOLDEN_E5M2 = REPO / "tests" / "golden" / "fp8_e5m2_golden.npz"
NP_DT = {DType.F32: np.float32, DType.F16: np.float16, DType.BF16: np.uint16,
         DType.F8_E4M3: np.uint8, DType.F8_E5M2: np.uint8}


def geom(layout, nb, bs, H, D, pack=8, shape_strides=None):
    shape = cache_shape(layout, nb, bs, H, D, pack)
    st = contiguous_strides(shape) if shape_strides is None else shape_strides
    return oracle.Geometry(layout, st, pack if layout == Layout.BLOCK_HND_PACKED else 1)


def bf16_bits(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bits (RNE) without the oracle, for building inputs."""
    u = x.astype(np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def encode(vals: np.ndarray, dt) -> np.ndarray:
    if dt == DType.F32:
        return vals.astype(np.float32)
    if dt == DType.F16:
        return vals.astype(np.float16)
    return bf16_bits(vals)


# ---------------------------------------------------------------------------
# Reference kernel-test cases, bit-exact.

def _ref_write_case(dt, H, D, tps, layout):
    """tests/kvx_kernel_test.cu:160-309 (NHD) / :311-454 (HND)."""
    S, L, bs = 2, 4, 4
    mbps = (L + bs - 1) // bs
    nb = S * mbps
    T = S * tps
    n = T * H * D
    i = np.arange(n, dtype=np.float32)
    key = encode(np.float32(0.1) + np.float32(0.01) * i, dt)
    val = encode(np.float32(0.1) + np.float32(0.01) * i + np.float32(0.5), dt)
    slots = np.full(T, -1, np.int64)
    for s in range(S):
        for t in range(tps):
            p = L - tps + t
            slots[s * tps + t] = (s * mbps + p // bs) * bs + p % bs
    g = geom(layout, nb, bs, H, D)
    kc = np.zeros(nb * bs * H * D, key.dtype)
    vc = np.zeros_like(kc)
    oracle.write_kv(g, g, key, val, kc, vc, slots, heads=H, head_dim=D, block_size=bs,
                    num_blocks=nb, io_dtype=dt, cache_dtype=dt)
    for t in range(T):
        b, o = divmod(int(slots[t]), bs)
        for h in range(H):
            for d in range(D):
                idx = (t * H + h) * D + d
                if layout == Layout.BLOCK_NHD:   # kvx_kernel_test.cu:274-277
                    off = ((b * bs + o) * H + h) * D + d
                else:                            # HND host loop, :417-446
                    off = ((b * H + h) * bs + o) * D + d
                assert kc[off] == key[idx] and vc[off] == val[idx]


@pytest.mark.parametrize("dt", [DType.F32, DType.F16, DType.BF16])
def test_reference_write_cases(dt):
    for H, D, tps in [(2, 4, 1), (1, 7, 1), (2, 4, 2)]:          # :459-461
        _ref_write_case(dt, H, D, tps, Layout.BLOCK_NHD)
    for H, D, tps in [(2, 4, 1), (1, 7, 2)]:                     # :463-464
        _ref_write_case(dt, H, D, tps, Layout.BLOCK_HND)


@pytest.mark.parametrize("dt", [DType.F32, DType.F16, DType.BF16])
def test_reference_gather_case(dt):
    """tests/kvx_kernel_test.cu:629-786"""
    S, L, bs, H, D = 2, 4, 4, 2, 4
    mbps = 1
    nb = S * mbps
    n = nb * bs * H * D
    i = np.arange(n, dtype=np.float32)
    kc = encode(np.float32(0.05) + np.float32(0.01) * i, dt)
    vc = encode(np.float32(0.05) + np.float32(0.01) * i + np.float32(0.5), dt)
    table = np.arange(S * mbps, dtype=np.int32).reshape(S, mbps)
    lens = np.full(S, L, np.int32)
    ko = np.zeros(S * L * H * D, kc.dtype)
    vo = np.zeros_like(ko)
    g = geom(Layout.BLOCK_NHD, nb, bs, H, D)
    oracle.gather_kv(g, g, kc, vc, ko, vo, table, lens, seq_count=S, max_blocks_per_seq=mbps,
                     max_seq_len=L, heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                     cache_dtype=dt, io_dtype=dt)
    for s in range(S):
        for t in range(L):
            bid = table[s, t // bs]
            for h in range(H):
                for d in range(D):
                    out = ((s * L + t) * H + h) * D + d
                    src = ((bid * bs + t % bs) * H + h) * D + d
                    assert ko[out] == kc[src] and vo[out] == vc[src]


# ---------------------------------------------------------------------------
# Brute force against numpy advanced indexing.

def _view_tokens(cache: np.ndarray, layout, H, D, pack):
    """A [nb, bs, H, D] view of a shaped cache array ([nb, bs, H, D/x, x]
    for the packed layout)."""
    if layout == Layout.BLOCK_NHD:
        return cache
    if layout == Layout.BLOCK_HND:
        return cache.transpose(0, 2, 1, 3)
    # [nb, H, D/x, bs, x] -> [nb, bs, H, D/x, x]
    return cache.transpose(0, 3, 1, 2, 4)


def _np_write(kview, key, slots, bs, nb, H, D, packed):
    for t, slot in enumerate(slots.tolist()):
        if slot < 0 or slot // bs >= nb:
            continue
        b, o = divmod(slot, bs)
        row = key[t].reshape(H, D)
        if packed:
            kview[b, o] = row.reshape(H, D // kview.shape[-1], kview.shape[-1])
        else:
            kview[b, o] = row


def _padded(shape, dtype, rng, pad_axis):
    """A C-order buffer holding `shape` with extra padding along pad_axis;
    returns (base buffer, shaped strided view, element strides)."""
    big = list(shape)
    big[pad_axis] += 3
    base = rng.integers(0, 255, size=int(np.prod(big)) * np.dtype(dtype).itemsize,
                        dtype=np.uint8).view(dtype)
    view = base.reshape(big)[tuple(slice(0, n) for n in shape)]
    st = tuple(s // np.dtype(dtype).itemsize for s in view.strides)
    return base, view, st


@pytest.mark.parametrize("seed", range(24))
def test_write_gather_vs_numpy_indexing(seed):
    rng = np.random.default_rng(seed)
    layouts = [Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED]
    kl, vl = rng.choice(layouts), rng.choice(layouts)
    dt = [DType.F32, DType.F16, DType.BF16, DType.F8_E4M3][seed % 4]
    npdt = NP_DT[dt]
    H, D = int(rng.choice([1, 2, 3])), int(rng.choice([4, 8, 16]))
    pack = int(rng.choice([d for d in (1, 2, 4, 8) if D % d == 0]))
    bs, nb = int(rng.choice([1, 3, 4, 8])), int(rng.integers(2, 9))
    T = int(rng.integers(1, 20))
    slot_dt = np.int64 if seed % 2 else np.int32
    total_slots = nb * bs
    slots = rng.permutation(total_slots + bs * 2)[:T].astype(slot_dt)  # some OOB blocks
    T = slots.size
    slots[rng.random(T) < 0.2] = -1
    key = rng.integers(0, 255, size=T * H * D * np.dtype(npdt).itemsize,
                       dtype=np.uint8).view(npdt)
    val = rng.integers(0, 255, size=key.nbytes, dtype=np.uint8).view(npdt)

    kshape = cache_shape(kl, nb, bs, H, D, pack)
    vshape = cache_shape(vl, nb, bs, H, D, pack)
    kbase, kview, kst = _padded(kshape, npdt, rng, int(rng.integers(0, len(kshape))))
    vbase, vview, vst = _padded(vshape, npdt, rng, int(rng.integers(0, len(vshape))))
    gk = oracle.Geometry(kl, kst, pack if kl == Layout.BLOCK_HND_PACKED else 1)
    gv = oracle.Geometry(vl, vst, pack if vl == Layout.BLOCK_HND_PACKED else 1)

    want_k, want_v = kbase.copy(), vbase.copy()
    # numpy: index the strided views of the expected buffers
    wkv = np.lib.stride_tricks.as_strided(want_k, kview.shape, kview.strides)
    wvv = np.lib.stride_tricks.as_strided(want_v, vview.shape, vview.strides)
    _np_write(_view_tokens(wkv, kl, H, D, pack), key.reshape(T, H * D), slots, bs, nb, H, D,
              kl == Layout.BLOCK_HND_PACKED)
    _np_write(_view_tokens(wvv, vl, H, D, pack), val.reshape(T, H * D), slots, bs, nb, H, D,
              vl == Layout.BLOCK_HND_PACKED)

    oracle.write_kv(gk, gv, key, val, kbase, vbase, slots, heads=H, head_dim=D,
                    block_size=bs, num_blocks=nb, io_dtype=dt, cache_dtype=dt)
    assert np.array_equal(kbase.view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(vbase.view(np.uint8), want_v.view(np.uint8))

    # gather from the same cache, random table with -1 and out-of-range ids
    S, L = int(rng.integers(1, 5)), int(rng.integers(1, 3 * bs + 2))
    mbps = int(rng.integers(1, (L + bs - 1) // bs + 2))
    idt = np.int64 if seed % 3 == 0 else np.int32
    table = rng.integers(-1, nb + 2, size=(S, mbps)).astype(idt)
    lens = rng.integers(-1, L + 3, size=S).astype(idt)
    fill = rng.integers(0, 255, size=S * L * H * D * np.dtype(npdt).itemsize, dtype=np.uint8)
    ko, vo = fill.copy().view(npdt), fill[::-1].copy().view(npdt)
    want_ko, want_vo = ko.copy().reshape(S, L, H, D), vo.copy().reshape(S, L, H, D)
    ktok = _view_tokens(kview, kl, H, D, pack)
    vtok = _view_tokens(vview, vl, H, D, pack)
    for s in range(S):
        for t in range(L):
            if t >= lens[s] or t // bs >= mbps:
                continue
            bid = int(table[s, t // bs])
            if bid < 0 or bid >= nb:
                continue
            want_ko[s, t] = ktok[bid, t % bs].reshape(H, D)
            want_vo[s, t] = vtok[bid, t % bs].reshape(H, D)
    oracle.gather_kv(gk, gv, kbase, vbase, ko, vo, table, lens, seq_count=S,
                     max_blocks_per_seq=mbps, max_seq_len=L, heads=H, head_dim=D,
                     block_size=bs, num_blocks=nb, cache_dtype=dt, io_dtype=dt)
    assert np.array_equal(ko.view(np.uint8), want_ko.reshape(-1).view(np.uint8))
    assert np.array_equal(vo.view(np.uint8), want_vo.reshape(-1).view(np.uint8))

    # the fast CPU-baseline variants agree with the element-wise oracle
    if all(st[-1] == 1 for st in (kst, vst)):
        kb2, vb2 = kbase.copy(), vbase.copy()
        oracle.write_kv_fast(gk, gv, key, val, kb2, vb2, slots, heads=H, head_dim=D,
                             block_size=bs, num_blocks=nb, elem_size=np.dtype(npdt).itemsize)
        assert np.array_equal(kb2.view(np.uint8), kbase.view(np.uint8))
        ko2, vo2 = fill.copy().view(npdt), fill[::-1].copy().view(npdt)
        oracle.gather_kv_fast(gk, gv, kbase, vbase, ko2, vo2, table, lens, seq_count=S,
                              max_blocks_per_seq=mbps, max_seq_len=L, heads=H, head_dim=D,
                              block_size=bs, num_blocks=nb,
                              elem_size=np.dtype(npdt).itemsize)
        assert np.array_equal(ko2.view(np.uint8), ko.view(np.uint8))
        assert np.array_equal(vo2.view(np.uint8), vo.view(np.uint8))


def test_roundtrip_c1_shapes():
    """Write 8 x 128 TinyLlama-shaped tokens, gather them back: identity, and
    every cache block outside the table untouched."""
    from kvx_amd.workloads import c1_tinyllama

    w = c1_tinyllama()
    rng = np.random.default_rng(7)
    H, D, bs, nb = w.heads, w.head_dim, w.block_size, w.num_blocks
    key = rng.standard_normal(w.num_tokens * H * D).astype(np.float16)
    val = rng.standard_normal(w.num_tokens * H * D).astype(np.float16)
    g = geom(Layout.BLOCK_NHD, nb, bs, H, D)
    kc = np.full(nb * bs * H * D, np.float16(-7.0))
    vc = kc.copy()
    oracle.write_kv(g, g, key, val, kc, vc, w.slots, heads=H, head_dim=D, block_size=bs,
                    num_blocks=nb, io_dtype=DType.F16, cache_dtype=DType.F16)
    used = np.zeros(nb, bool)
    used[w.block_table.reshape(-1)] = True
    assert np.all(kc.reshape(nb, -1)[~used] == np.float16(-7.0))
    ko = np.zeros(w.seq_count * w.max_seq_len * H * D, np.float16)
    vo = ko.copy()
    oracle.gather_kv(g, g, kc, vc, ko, vo, w.block_table, w.seq_lens, seq_count=w.seq_count,
                     max_blocks_per_seq=w.max_blocks_per_seq, max_seq_len=w.max_seq_len,
                     heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                     cache_dtype=DType.F16, io_dtype=DType.F16)
    assert np.array_equal(ko.view(np.uint16), key.view(np.uint16))
    assert np.array_equal(vo.view(np.uint16), val.view(np.uint16))


def test_cache_offset_closed_forms():
    """kvx_paged_kv.cu:54-75 on canonical strides equals the row-major index
    of the layout's shape."""
    nb, bs, H, D, x = 3, 4, 2, 16, 8
    for layout in (Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED):
        g = geom(layout, nb, bs, H, D, x)
        shape = cache_shape(layout, nb, bs, H, D, x)
        for b, o, h, d in [(0, 0, 0, 0), (2, 3, 1, 15), (1, 2, 0, 9), (2, 0, 1, 7)]:
            idx = {Layout.BLOCK_NHD: (b, o, h, d), Layout.BLOCK_HND: (b, h, o, d),
                   Layout.BLOCK_HND_PACKED: (b, h, d // x, o, d % x)}[layout]
            assert oracle.cache_offset(g, b, o, h, d) == np.ravel_multi_index(idx, shape)


# ---------------------------------------------------------------------------
# FP8 and the other casts.

@pytest.fixture(scope="module")
def golden():
    return np.load(GOLDEN, allow_pickle=False)


def test_quantize_matches_torch_golden(golden):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for i, s in enumerate(golden["scales"]):
        got = oracle.quantize_e4m3(bits, DType.BF16, float(s))
        assert np.array_equal(got, golden["quant_from_bf16"][i]), float(s)


def test_dequantize_matches_torch_golden(golden):
    codes = np.arange(256, dtype=np.uint8)
    for i, s in enumerate(golden["scales"]):
        for dt, key in [(DType.BF16, "dequant_bf16"), (DType.F16, "dequant_f16"),
                        (DType.F32, "dequant_f32")]:
            got = oracle.dequantize_e4m3(codes, float(s), dt)
            assert np.array_equal(got, golden[key][i]), (float(s), key)


def test_e4m3_special_values():
    L = oracle.lib()
    assert L.oracle_f32_to_e4m3(448.0) == 0x7E
    assert L.oracle_f32_to_e4m3(-1e30) == 0xFE
    assert L.oracle_f32_to_e4m3(float("inf")) == 0x7E
    assert L.oracle_f32_to_e4m3(float("nan")) == 0x7F
    assert L.oracle_f32_to_e4m3(2.0 ** -9) == 0x01       # smallest subnormal
    assert L.oracle_f32_to_e4m3(2.0 ** -10) == 0x00      # tie -> even (0)
    assert L.oracle_f32_to_e4m3(3 * 2.0 ** -10) == 0x02  # tie -> even (2)
    assert L.oracle_f32_to_e4m3(-0.0) == 0x80
    assert L.oracle_f32_to_e4m3(1.0) == 0x38
    assert L.oracle_f32_to_e4m3(1.0625) == 0x38          # tie -> even mantissa
    assert L.oracle_f32_to_e4m3(1.1875) == 0x3A          # tie -> even mantissa
    assert L.oracle_e4m3_to_f32(0x7E) == 448.0
    assert L.oracle_e4m3_to_f32(0x08) == 2.0 ** -6
    assert np.isnan(L.oracle_e4m3_to_f32(0xFF))


@pytest.fixture(scope="module")
def golden_e5m2():
    return np.load(GOLDEN_E5M2, allow_pickle=False)


def test_e5m2_quantize_matches_torch_golden(golden_e5m2):
    bits = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    for i, s in enumerate(golden_e5m2["scales"]):
        for dt, key in [(DType.BF16, "quant_from_bf16"), (DType.F16, "quant_from_f16")]:
            got = oracle.quantize_fp8(bits, dt, float(s), oracle.E5M2)
            assert np.array_equal(got, golden_e5m2[key][i]), (float(s), key)


def test_e5m2_dequantize_matches_torch_golden(golden_e5m2):
    codes = np.arange(256, dtype=np.uint8)
    for i, s in enumerate(golden_e5m2["scales"]):
        for dt, key in [(DType.BF16, "dequant_bf16"), (DType.F16, "dequant_f16"),
                        (DType.F32, "dequant_f32")]:
            got = oracle.dequantize_fp8(codes, float(s), dt, oracle.E5M2)
            assert np.array_equal(got, golden_e5m2[key][i]), (float(s), key)


def test_e5m2_special_values():
    L = oracle.lib()
    assert L.oracle_f32_to_e5m2(57344.0) == 0x7B
    assert L.oracle_f32_to_e5m2(61440.0) == 0x7B         # would round to inf: saturates
    assert L.oracle_f32_to_e5m2(float("-inf")) == 0xFB
    assert L.oracle_f32_to_e5m2(float("nan")) == 0x7E
    assert L.oracle_f32_to_e5m2(2.0 ** -16) == 0x01      # smallest subnormal
    assert L.oracle_f32_to_e5m2(2.0 ** -17) == 0x00      # tie -> even (0)
    assert L.oracle_f32_to_e5m2(1.0) == 0x3C
    assert L.oracle_f32_to_e5m2(1.125) == 0x3C           # tie -> even mantissa
    assert L.oracle_f32_to_e5m2(1.375) == 0x3E           # tie -> even mantissa
    assert L.oracle_e5m2_to_f32(0x7C) == float("inf")
    assert L.oracle_e5m2_to_f32(0x7B) == 57344.0
    assert L.oracle_e5m2_to_f32(0x04) == 2.0 ** -14
    assert np.isnan(L.oracle_e5m2_to_f32(0xFD))
    # E5M2 is the top byte of binary16: exact f16 values with zero low byte
    h = np.arange(0, 0x7C00, 256, dtype=np.uint16)
    assert all(L.oracle_f32_to_e5m2(float(v)) == (int(b) >> 8)
               for v, b in zip(h.view(np.float16).astype(np.float32), h))


def test_f16_cast_matches_numpy():
    rng = np.random.default_rng(3)
    x = rng.integers(0, 1 << 32, size=200_000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    x = np.concatenate([x, (rng.standard_normal(100_000) * 1e-5).astype(np.float32),
                        np.array([65504, 65519.99, 65520, 1e9, -0.0], np.float32)])
    L = oracle.lib()
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([L.oracle_f32_to_f16(float(v)) for v in x[:30000]], np.uint16)
    nan = np.isnan(x[:30000])
    assert np.array_equal(got[~nan], want[:30000][~nan])
    assert np.all(got[nan] == 0x7E00)


def test_kernel_cast_source_matches_oracle(tmp_path):
    """kvx_amd/csrc/fp_convert.h (compiled into the kernels) agrees with the
    oracle's casts on every rounding boundary and on random inputs."""
    import oracle.build as ob

    ob.build_oracle()
    exe = tmp_path / "fp_convert_check"
    subprocess.run(["g++", "-std=c++17", "-O2", f"-I{REPO / 'kvx_amd' / 'csrc'}",
                    f"-I{REPO / 'oracle'}", str(REPO / "tests" / "fp_convert_check.cpp"),
                    str(ob.ORACLE_LIB), f"-Wl,-rpath,{ob.ORACLE_LIB.parent}", "-o", str(exe)],
                   check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True, check=True,
                         timeout=600).stdout
    lines = dict(l.split(" ", 1) for l in out.strip().splitlines())
    assert set(lines) == {"f32_to_e4m3", "e4m3_to_f32", "f32_to_e5m2", "e5m2_to_f32",
                          "f32_to_bf16", "f32_to_f16", "f16_to_f32"}
    for name, rest in lines.items():
        assert rest.startswith("0 of "), (name, rest)
