"""Status codes of the kvx_paged_kv.h / kvx_ext.h launch path (CPU only).

The reference launchers (kernels/kvx_paged_kv.cu) need nvcc and cannot be
built here, so each case below is one injected fault (or a pair, to pin the
check order) with the code the cited reference line returns.  Every case
returns before a kernel would be enqueued (a validation error, or an empty
batch, which the reference returns OK for without launching), so no GPU is
touched.
"""
import ctypes as C

import pytest

from kvx_amd import abi
from kvx_amd.abi import DType, Layout, Memory, ScaleGranularity, Status, TableFormat

D_ = Memory.DEVICE
FAKE = 0x20000  # never dereferenced: every case returns before a launch

INV, UNS, OK = Status.INVALID_ARGUMENT, Status.UNSUPPORTED, Status.OK


def base_write(dt=DType.BF16, io_dt=None, T=4, layout=Layout.BLOCK_NHD, v_layout=None,
               slot_dt=DType.S64, H=2, D=8, nb=4, bs=4, pack=4):
    io_dt = dt if io_dt is None else io_dt
    cache = abi.make_cache(layout, dt, D_, nb, bs, H, D, FAKE, FAKE, pack=pack,
                           v_layout=v_layout)
    w = abi.make_write(T, H, D, io_dt, D_, FAKE, FAKE, slot_dt, FAKE)
    return cache, w


def base_gather(dt=DType.BF16, io_dt=None, S=2, L=8, H=2, D=8, nb=4, bs=4,
                idx=DType.S32, lens=DType.S32, layout=Layout.BLOCK_NHD):
    io_dt = dt if io_dt is None else io_dt
    cache = abi.make_cache(layout, dt, D_, nb, bs, H, D, FAKE, FAKE)
    tb = abi.make_block_table_packed(S, 2, idx, FAKE)
    sl = abi.make_seq_lens(S, lens, FAKE)
    g = abi.make_gather(S, L, H, D, io_dt, D_, FAKE, FAKE, tb, sl)
    return cache, g


def W(lib, cache, w, fn="kvx_launch_write_kv"):
    return Status(getattr(lib, fn)(abi.ref(cache), abi.ref(w), None))


def WP(lib, cache, w, tps, fn="kvx_launch_write_kv_prefill"):
    return Status(getattr(lib, fn)(abi.ref(cache), abi.ref(w), tps, None))


def G(lib, cache, g, fn="kvx_launch_gather_kv"):
    return Status(getattr(lib, fn)(abi.ref(cache), abi.ref(g), None))


# ---------------------------------------------------------------------------
# write: kvx_paged_kv.cu:315-451 (per dtype), :472-491 (dispatch)

def test_write_dispatch(kvx_lib):
    c, w = base_write()
    assert W(kvx_lib, None, w) == INV                       # :475
    assert W(kvx_lib, c, None) == INV
    c.v.dtype = DType.F16
    assert W(kvx_lib, c, w) == INV                          # :478 k != v dtype
    for dt in (DType.U8, DType.S32, DType.INVALID):
        c, w = base_write()
        c.k.dtype = c.v.dtype = dt
        assert W(kvx_lib, c, w) == UNS, dt                  # :488
    # FP8 caches are this build's extension: with bf16 io they need scales
    for dt in (DType.F8_E4M3, DType.F8_E5M2):
        c, w = base_write(dt=dt, io_dt=DType.BF16)
        assert W(kvx_lib, c, w) == INV, dt


@pytest.mark.parametrize("fn", ["kvx_launch_write_kv", "kvx_launch_write_kv_bf16"])
def test_write_single_faults(kvx_lib, fn):
    cases = []

    def case(expect, mutate, **kw):
        c, w = base_write(**kw)
        mutate(c, w)
        cases.append((expect, c, w))

    case(INV, lambda c, w: setattr(w, "size", C.sizeof(w) - 1))             # :323
    case(INV, lambda c, w: setattr(w.io, "size", 8))                        # :326
    case(INV, lambda c, w: setattr(w.slots, "size", 0))                     # :329
    case(UNS, lambda c, w: (setattr(w.io.key, "dtype", DType.F16)))         # :335
    case(UNS, lambda c, w: (setattr(w.io.value, "dtype", DType.F32)))       # :336
    case(INV, lambda c, w: setattr(w.io, "num_kv_heads", 3))                # :339
    case(INV, lambda c, w: setattr(w.io, "head_dim", 16))                   # :340
    case(INV, lambda c, w: setattr(w.io.key, "ndim", 4))                    # :276
    case(INV, lambda c, w: w.io.key.shape.__setitem__(0, 5))                # :279
    case(UNS, lambda c, w: w.io.key.stride.__setitem__(0, 17))              # :283
    case(UNS, lambda c, w: w.io.value.stride.__setitem__(2, 2))             # :350
    case(INV, lambda c, w: setattr(w.slots, "token_count", 3))              # :357
    case(UNS, lambda c, w: setattr(c.k, "layout", 14))                      # :49
    # CUSTOM is gathered and written here (the reference: UNSUPPORTED, :49);
    # its shape must name the axes
    case(INV, lambda c, w: (setattr(c.k, "layout", Layout.BLOCK_CUSTOM),
                            setattr(c.k, "ndim", 3)))
    case(INV, lambda c, w: (setattr(c.k, "layout", Layout.BLOCK_CUSTOM),
                            c.k.shape.__setitem__(1, 5)))
    case(UNS, lambda c, w: setattr(c.v, "layout", Layout.INVALID))          # :367
    case(INV, lambda c, w: (setattr(c.k, "layout", Layout.BLOCK_HND_PACKED),
                            c.k.shape.__setitem__(4, 0)))                   # :40
    case(INV, lambda c, w: (setattr(c.k, "layout", Layout.BLOCK_HND_PACKED),
                            c.k.shape.__setitem__(4, 3)))                   # :43
    case(INV, lambda c, w: setattr(w.slots, "dtype", DType.U32))            # :443
    case(INV, lambda c, w: setattr(w.slots, "dtype", DType.S32 - 6))        # :443
    for expect, c, w in cases:
        assert W(kvx_lib, c, w, fn) == expect


def test_write_check_order(kvx_lib):
    # size checks come before dtype checks (:323 before :332)
    c, w = base_write()
    w.size = 0
    c.k.dtype = c.v.dtype = DType.F32
    assert W(kvx_lib, c, w, "kvx_launch_write_kv_bf16") == INV
    # io dtype (UNSUPPORTED) before the head check (INVALID): :335 before :339
    c, w = base_write()
    w.io.key.dtype = DType.F32
    w.io.num_kv_heads = 7
    assert W(kvx_lib, c, w) == UNS
    # key io tensor before value io tensor: INVALID shape beats UNSUPPORTED stride
    c, w = base_write()
    w.io.key.ndim = 2
    w.io.value.stride[0] = 99
    assert W(kvx_lib, c, w) == INV
    # params (UNSUPPORTED layout) before the slot dtype (INVALID): :363 before :443
    c, w = base_write()
    c.k.layout = 14
    w.slots.dtype = DType.U64
    assert W(kvx_lib, c, w) == UNS


def test_write_empty_batch_is_ok_without_launch(kvx_lib):
    # total == 0 returns OK before the slot-dtype check (:374 before :398)
    c, w = base_write(T=0)
    w.slots.dtype = DType.U32
    assert W(kvx_lib, c, w) == OK
    # mixed K/V layouts and non-canonical cache strides pass launch validation
    c, w = base_write(T=0, layout=Layout.BLOCK_HND_PACKED, v_layout=Layout.BLOCK_NHD)
    c.v.stride[0] += 64
    assert W(kvx_lib, c, w) == OK
    # ... while the strict ABI entry point rejects the mixed layouts
    c.k.memory = c.v.memory = Memory.HOST
    w.io.key.memory = w.io.value.memory = Memory.HOST
    assert Status(kvx_lib.kvx_write_kv(abi.ref(c), abi.ref(w), None)) == INV


def test_prefill_validation(kvx_lib):
    c, w = base_write()
    assert WP(kvx_lib, c, w, 0) == INV                       # :500
    assert WP(kvx_lib, c, w, -3) == INV
    # reference test run_write_prefill_invalid (kvx_kernel_test.cu:607-618)
    c0, w0 = abi.CacheDesc(), abi.WriteDesc()
    c0.k.dtype = c0.v.dtype = DType.F16
    assert WP(kvx_lib, c0, w0, 0) == INV
    # num_tokens % tps checked after sizes and before dtypes (:512)
    c, w = base_write(T=6)
    c.k.dtype = c.v.dtype = DType.F32
    assert WP(kvx_lib, c, w, 4, "kvx_launch_write_kv_prefill_bf16") == INV
    c, w = base_write(T=6)
    w.size = 1
    assert WP(kvx_lib, c, w, 4) == INV
    c, w = base_write(T=0)
    assert WP(kvx_lib, c, w, 4) == OK
    c, w = base_write(T=8)
    w.io.key.dtype = DType.F16
    assert WP(kvx_lib, c, w, 4) == UNS


def test_write_safety_checks_added_by_this_build(kvx_lib):
    """Inputs the reference would launch on and then divide by zero or fault."""
    c, w = base_write()
    c.block_size = 0
    assert W(kvx_lib, c, w) == INV
    for field in ("key", "value"):
        c, w = base_write()
        getattr(w.io, field).data = None
        assert W(kvx_lib, c, w) == INV
    c, w = base_write()
    w.slots.slots = None
    assert W(kvx_lib, c, w) == INV
    c, w = base_write()
    c.k.data = None
    assert W(kvx_lib, c, w) == INV


def test_fp8_write_validation(kvx_lib):
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    assert W(kvx_lib, c, w) == INV                           # no scale at all
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    w.k_scale_desc = abi.scale_desc(FAKE, dtype=DType.F16)
    w.v_scale = FAKE
    assert W(kvx_lib, c, w) == UNS
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    w.k_scale_desc = abi.scale_desc(FAKE, granularity=ScaleGranularity.NONE)
    w.v_scale = FAKE
    assert W(kvx_lib, c, w) == UNS
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    w.k_scale = FAKE
    w.v_scale_desc = abi.scale_desc(FAKE)
    w.v_scale_desc.size = 8
    assert W(kvx_lib, c, w) == INV
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.U8)
    assert W(kvx_lib, c, w) == UNS
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    w.io.value.dtype = DType.F16
    assert W(kvx_lib, c, w) == UNS
    # per-dtype helpers never take an FP8 cache
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16)
    assert W(kvx_lib, c, w, "kvx_launch_write_kv_bf16") == UNS
    # empty FP8 batch with valid scales
    c, w = base_write(dt=DType.F8_E4M3, io_dt=DType.BF16, T=0)
    w.k_scale = w.v_scale = FAKE
    assert W(kvx_lib, c, w) == OK
    c, w = base_write(dt=DType.F8_E5M2, io_dt=DType.F8_E5M2, T=0)
    assert W(kvx_lib, c, w) == OK                            # byte copy, no scale


# base_write / base_gather caches: 4 blocks, 2 heads
GOOD_SCALES = [(ScaleGranularity.PER_TENSOR, (1,)), (ScaleGranularity.PER_HEAD, (2,)),
               (ScaleGranularity.PER_BLOCK, (4,)), (ScaleGranularity.PER_BLOCK_HEAD, (4, 2))]
BAD_SHAPES = [(ScaleGranularity.PER_HEAD, (3,)), (ScaleGranularity.PER_HEAD, (2, 1)),
              (ScaleGranularity.PER_BLOCK, (2,)), (ScaleGranularity.PER_BLOCK_HEAD, (2, 4)),
              (ScaleGranularity.PER_BLOCK_HEAD, (4,))]


@pytest.mark.parametrize("dt", [DType.F8_E4M3, DType.F8_E5M2])
def test_fp8_scale_granularities(kvx_lib, dt):
    """Scale shapes (this build's reading of KVX_SPEC.md:190-197): accepted
    shapes resolve (empty batch -> OK, no launch), wrong shapes are
    INVALID_ARGUMENT, other granularities and dtypes UNSUPPORTED."""
    for gran, shape in GOOD_SCALES:
        c, w = base_write(dt=dt, io_dt=DType.F16, T=0)
        w.k_scale_desc = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        w.v_scale_desc = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        assert W(kvx_lib, c, w) == OK, gran
    for gran, shape in BAD_SHAPES:
        c, w = base_write(dt=dt, io_dt=DType.F16)
        w.k_scale_desc = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        w.v_scale = FAKE
        assert W(kvx_lib, c, w) == INV, (gran, shape)
    for gran in (ScaleGranularity.NONE, 7):
        c, w = base_write(dt=dt, io_dt=DType.F16)
        w.k_scale_desc = abi.scale_desc(FAKE, granularity=gran)
        w.v_scale = FAKE
        assert W(kvx_lib, c, w) == UNS, gran
    f = kvx_lib.kvx_launch_gather_kv_dequant
    for gran, shape in GOOD_SCALES:
        c, g = base_gather(dt=dt, io_dt=DType.BF16, L=0)
        k = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        assert Status(f(abi.ref(c), abi.ref(g), abi.ref(k), abi.ref(k), None)) == OK, gran
    for gran, shape in BAD_SHAPES:
        c, g = base_gather(dt=dt, io_dt=DType.BF16)
        k = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        assert Status(f(abi.ref(c), abi.ref(g), abi.ref(k), abi.ref(k), None)) == INV
    # KV_OFFSETS has no physical block ids for block-indexed scales
    for gran, shape in GOOD_SCALES[2:]:
        c, g = offsets_gather(dt=dt, io_dt=DType.BF16)
        k = abi.scale_desc(FAKE, granularity=gran, shape=shape)
        assert Status(f(abi.ref(c), abi.ref(g), abi.ref(k), abi.ref(k), None)) == UNS


# ---------------------------------------------------------------------------
# gather: kvx_paged_kv.cu:763-870 (per dtype), :891-910 (dispatch)

def test_gather_single_faults(kvx_lib):
    cases = []

    def case(expect, mutate, **kw):
        c, g = base_gather(**kw)
        mutate(c, g)
        cases.append((expect, c, g))

    case(INV, lambda c, g: setattr(g, "size", 4))                             # :771
    case(INV, lambda c, g: setattr(g.io, "size", 4))                          # :774
    case(INV, lambda c, g: setattr(g.block_table, "size", 4))                 # :777
    case(INV, lambda c, g: setattr(g.seq_lens, "size", 4))                    # :778
    case(UNS, lambda c, g: setattr(g.io.key, "dtype", DType.F32))             # :784
    # :788 rejects every non-PACKED format; this build also gathers RAGGED and
    # KV_OFFSETS (tested below), so unknown formats keep the reference code
    case(UNS, lambda c, g: setattr(g.block_table, "format", TableFormat.INVALID))
    case(UNS, lambda c, g: setattr(g.block_table, "format", 7))
    case(INV, lambda c, g: setattr(g.io, "num_kv_heads", 1))                  # :791
    case(INV, lambda c, g: setattr(g.seq_lens, "seq_count", 1))               # :795
    case(INV, lambda c, g: g.io.key.shape.__setitem__(1, 7))                  # :302
    case(UNS, lambda c, g: g.io.value.stride.__setitem__(1, 3))               # :306
    case(UNS, lambda c, g: setattr(c.k, "layout", 14))                        # :816
    case(INV, lambda c, g: (setattr(c.v, "layout", Layout.BLOCK_CUSTOM),
                            setattr(c.v, "ndim", 6)))
    case(INV, lambda c, g: setattr(g.block_table, "index_dtype", DType.S64))  # :861
    case(INV, lambda c, g: setattr(g.seq_lens, "dtype", DType.U32))           # :861
    for expect, c, g in cases:
        assert G(kvx_lib, c, g) == expect
    c, g = base_gather()
    assert G(kvx_lib, None, g) == INV
    c.v.dtype = DType.F16
    assert G(kvx_lib, c, g) == INV                                            # :897
    c, g = base_gather()
    c.k.dtype = c.v.dtype = DType.F8_E5M2
    assert G(kvx_lib, c, g) == UNS                                            # :907
    c, g = base_gather()
    assert G(kvx_lib, c, g, "kvx_launch_gather_kv_f16") == UNS               # :781


def test_gather_check_order_and_empty(kvx_lib):
    # format (UNSUPPORTED) before heads (INVALID): :788 before :791
    c, g = base_gather()
    g.block_table.format = TableFormat.INVALID
    g.io.num_kv_heads = 5
    assert G(kvx_lib, c, g) == UNS
    # total == 0 (max_seq_len 0) is OK before the index dtype check
    c, g = base_gather(L=0)
    g.block_table.index_dtype = DType.U64
    assert G(kvx_lib, c, g) == OK
    # block_table.indices_count is not checked on the launch path
    c, g = base_gather(L=0)
    g.block_table.indices_count = 12345
    assert G(kvx_lib, c, g) == OK


def test_dequant_gather_validation(kvx_lib):
    f = kvx_lib.kvx_launch_gather_kv_dequant
    ks = abi.scale_desc(FAKE)
    vs = abi.scale_desc(FAKE)

    def call(c, g, k=ks, v=vs):
        return Status(f(abi.ref(c), abi.ref(g), abi.ref(k), abi.ref(v), None))

    c, g = base_gather(dt=DType.F8_E4M3, io_dt=DType.BF16, L=0)
    assert call(c, g) == OK
    assert call(c, g, k=None) == INV
    c, g = base_gather(dt=DType.BF16)
    assert call(c, g) == UNS
    c, g = base_gather(dt=DType.F8_E4M3, io_dt=DType.F8_E4M3)
    assert call(c, g) == UNS
    c, g = base_gather(dt=DType.F8_E4M3, io_dt=DType.BF16)
    bad = abi.scale_desc(FAKE, granularity=ScaleGranularity.NONE)
    assert call(c, g, v=bad) == UNS
    bad = abi.scale_desc(None)
    assert call(c, g, k=bad) == INV
    c, g = base_gather(dt=DType.F8_E4M3, io_dt=DType.BF16)
    g.block_table.format = 9
    assert call(c, g) == UNS


def test_gather_safety_checks_added_by_this_build(kvx_lib):
    c, g = base_gather()
    c.block_size = 0
    assert G(kvx_lib, c, g) == INV
    c, g = base_gather()
    g.seq_lens.lengths = None
    assert G(kvx_lib, c, g) == INV
    c, g = base_gather()
    g.io.value.data = None
    assert G(kvx_lib, c, g) == INV


# ---------------------------------------------------------------------------
# RAGGED / KV_OFFSETS gather (this build's extension; KVX_SPEC.md:99-122).
# Their checks follow the reference's index-dtype check, so every earlier
# fault keeps the reference code.

def ragged_gather(**kw):
    c, g = base_gather(**kw)
    g.block_table.format = TableFormat.RAGGED
    g.block_table.indptr = FAKE
    g.block_table.indptr_dtype = DType.S32
    g.block_table.indptr_count = g.block_table.seq_count + 1
    return c, g


def offsets_gather(**kw):
    c, g = base_gather(**kw)
    t = g.block_table
    t.format = TableFormat.KV_OFFSETS
    t.flags = abi.TABLE_FLAG_KVCACHEINDEX
    t.indices_count = t.seq_count * 2 * t.max_blocks_per_seq
    c.pool.primary = FAKE
    c.pool.bytes_per_block = 4096
    return c, g


def test_ragged_validation(kvx_lib):
    c, g = ragged_gather(L=0)
    assert G(kvx_lib, c, g) == OK                       # empty output: no launch
    for mutate in (lambda g: setattr(g.block_table, "indptr_dtype", DType.U32),
                   lambda g: setattr(g.block_table, "indptr", None),
                   lambda g: setattr(g.block_table, "indptr_count", 2),
                   lambda g: setattr(g.block_table, "index_dtype", DType.S64),
                   lambda g: setattr(g.block_table, "indices", None)):
        c, g = ragged_gather()
        mutate(g)
        assert G(kvx_lib, c, g) == INV
    c, g = ragged_gather()
    g.io.key.dtype = DType.F32                          # earlier reference check wins
    g.block_table.indptr = None
    assert G(kvx_lib, c, g) == UNS


def test_kv_offsets_validation(kvx_lib):
    c, g = offsets_gather(L=0)
    assert G(kvx_lib, c, g) == OK
    cases = [
        (INV, lambda c, g: setattr(g.block_table, "index_dtype", DType.S64)),
        (INV, lambda c, g: setattr(g.block_table, "flags", 0)),
        (INV, lambda c, g: setattr(g.block_table, "beam_width", 0)),
        (UNS, lambda c, g: (setattr(g.block_table, "beam_width", 2),
                            setattr(g.block_table, "indices_count", g.block_table.indices_count * 2))),
        (INV, lambda c, g: setattr(c, "block_size", 6)),
        (INV, lambda c, g: setattr(c.pool, "primary", None)),
        (INV, lambda c, g: setattr(c.pool, "bytes_per_block", 0)),
        (INV, lambda c, g: setattr(c.pool, "bytes_per_block", 127)),   # block is 128 B
        (INV, lambda c, g: c.k.stride.__setitem__(1, -c.k.stride[1])),
        (INV, lambda c, g: setattr(g.block_table, "indices_count", 3)),
        (INV, lambda c, g: setattr(g.block_table, "indices", None)),
    ]
    for expect, mutate in cases:
        c, g = offsets_gather()
        mutate(c, g)
        assert G(kvx_lib, c, g) == expect
    # S64 seq_lens are accepted with S32 offsets; the pool replaces cache data
    c, g = offsets_gather(L=0, lens=DType.S64)
    c.k.data = c.v.data = None
    assert G(kvx_lib, c, g) == OK


# ---------------------------------------------------------------------------
# Grid limits: HIP allows at most 2^32 - 1 work-items per grid dimension.
# Each case below is just past that limit for the kernel its shape selects,
# so it returns UNSUPPORTED before any launch (no GPU is touched).

def big_gather(layout, S, L, H, D, bs, fmt="packed"):
    cache = abi.make_cache(layout, DType.F16, D_, 64, bs, H, D, FAKE, FAKE)
    sl = abi.make_seq_lens(S, DType.S32, FAKE)
    tb = abi.make_block_table_packed(S, (L + bs - 1) // bs, DType.S32, FAKE)
    if fmt == "ragged":
        tb.format = TableFormat.RAGGED
        tb.indptr, tb.indptr_dtype, tb.indptr_count = FAKE, DType.S32, S + 1
    return cache, abi.make_gather(S, L, H, D, DType.F16, D_, FAKE, FAKE, tb, sl)


def test_gather_grid_past_hip_limits(kvx_lib):
    # gather_rows_kernel (HND runs of 12 bytes, two heads: no LDS tile, not
    # row-major), 256 threads: 4096 x 4096 workgroups = 2^32 work-items
    assert G(kvx_lib, *big_gather(Layout.BLOCK_HND, 4096, 65536, 2, 6, 16)) == UNS
    # gather_flat_kernel (canonical NHD), 128 threads, blocks no longer
    # split, 4096 blocks per sequence taken two per workgroup: 16384 x 2048
    # workgroups = 2^32 work-items
    assert G(kvx_lib, *big_gather(Layout.BLOCK_NHD, 16384, 65536, 1, 8, 16)) == UNS
    # gather_ragged_tile_kernel, 128 threads, 16 rows per workgroup
    assert G(kvx_lib, *big_gather(Layout.BLOCK_NHD, 8192, 65536, 1, 8, 16,
                                  fmt="ragged")) == UNS


def test_pool_blocks_gather_validation(kvx_lib):
    """kvx_launch_gather_kv_pools (kvx_ext.h): its own argument checks come
    first (NULL cache / gather, a short or negative kvx_pool_blocks_t, one
    scale descriptor without the other); then it is the copy gather (no
    scales) or the dequantizing gather (both), with their codes; empty
    batches return OK without a launch."""
    f = kvx_lib.kvx_launch_gather_kv_pools
    ks, vs = abi.scale_desc(FAKE), abi.scale_desc(FAKE)

    def pb(primary=0, secondary=0, size=None):
        return abi.PoolBlocks(C.sizeof(abi.PoolBlocks) if size is None else size, 0, primary,
                              secondary)

    def call(c, g, p=None, k=None, v=None):
        return Status(f(abi.ref(c) if c is not None else None, abi.ref(g) if g is not None else None,
                        abi.ref(p) if p is not None else None, abi.ref(k) if k is not None else None,
                        abi.ref(v) if v is not None else None, None))

    assert C.sizeof(abi.PoolBlocks) == 24
    c, g = offsets_gather(L=0)
    assert call(c, g) == OK
    assert call(c, g, pb(5, 3)) == OK
    assert call(c, g, pb(0, 0)) == OK
    assert call(None, g, pb()) == INV
    assert call(c, None, pb()) == INV
    assert call(c, g, pb(size=8)) == INV
    assert call(c, g, pb(-1, 0)) == INV
    assert call(c, g, pb(0, -2)) == INV
    # copy-gather codes: a dtype the copy does not take, mismatched K / V
    c, g = offsets_gather()
    c.k.dtype = c.v.dtype = DType.S32
    assert call(c, g, pb(1, 1)) == UNS
    c, g = offsets_gather()
    c.v.dtype = DType.F16 if c.k.dtype != DType.F16 else DType.BF16
    assert call(c, g, pb(1, 1)) == INV
    # dequantizing: both scales or neither; FP8 caches only
    c, g = offsets_gather(dt=DType.F8_E4M3, io_dt=DType.BF16, L=0)
    assert call(c, g, pb(4, 2), ks, vs) == OK
    assert call(c, g, pb(4, 2), ks, None) == INV
    assert call(c, g, pb(4, 2), None, vs) == INV
    c, g = offsets_gather(dt=DType.BF16, L=0)
    assert call(c, g, pb(4, 2), ks, vs) == UNS
    # PACKED tables take the entry too (the counts are not read)
    c, g = base_gather(L=0)
    assert call(c, g, pb(1, 1)) == OK
