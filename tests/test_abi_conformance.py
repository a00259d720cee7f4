"""Status codes of the kvx_abi.h entry points (CPU only).

Three independent pins:
  1. every assert of the reference's tests/kvx_abi_test.c:190-316, restated;
  2. the reference's own kvx_abi_test.c, compiled against the reference
     kvx_abi.h and linked with libkvx_amd.so (oracle/_ref, built by
     oracle/build.py where /root/reference exists);
  3. randomized descriptor mutations compared code-for-code with the
     reference's own kvx_abi.c compiled unmodified (oracle/_ref).
All buffers are KVX_MEMORY_HOST, on which the library validates only.
"""
import ctypes as C
import random
import subprocess

import numpy as np
import pytest

from kvx_amd import abi
from kvx_amd.abi import DType, Layout, Memory, Status, TableFormat

import oracle.build as ob

H = Memory.HOST
FAKE = 0x10000  # never dereferenced on the validation-only path


def make_cache_nhd(k, v):
    """tests/kvx_abi_test.c:94-112"""
    return abi.make_cache(Layout.BLOCK_NHD, DType.F32, H, 2, 4, 2, 8, k, v)


def test_reference_asserts_restated(kvx_lib):
    L = kvx_lib
    kbuf = np.zeros(128, np.float32)
    vbuf = np.zeros(128, np.float32)
    kp, vp = kbuf.ctypes.data, vbuf.ctypes.data
    v = abi.Version()
    assert L.kvx_get_version(C.byref(v)) == Status.OK
    assert v.abi_major == 1 and v.abi_minor == 1 and v.size >= 16

    cache = make_cache_nhd(kp, vp)
    assert L.kvx_validate_cache_desc(C.byref(cache)) == Status.OK          # :217
    cache.block_size = 0
    assert L.kvx_validate_cache_desc(C.byref(cache)) == Status.INVALID_ARGUMENT
    cache = make_cache_nhd(kp, vp)
    cache.size = C.sizeof(cache) - 4
    assert L.kvx_validate_cache_desc(C.byref(cache)) == Status.INVALID_ARGUMENT
    cache = make_cache_nhd(kp, vp)
    cache.k.stride[0] += 1
    assert L.kvx_validate_cache_desc(C.byref(cache)) == Status.UNSUPPORTED
    cache = make_cache_nhd(kp, vp)
    cache.v.layout = Layout.BLOCK_HND
    assert L.kvx_validate_cache_desc(C.byref(cache)) == Status.INVALID_ARGUMENT

    # :239-251 HND_PACKED with pack 3 not dividing head_dim 8.  The shape and
    # strides are what the reference helper computes with integer division.
    pk = abi.TensorDesc()
    pk.size = C.sizeof(pk)
    pk.dtype, pk.layout, pk.memory, pk.ndim = DType.F16, Layout.BLOCK_HND_PACKED, H, 5
    for i, (n, s) in enumerate(zip((1, 2, 8 // 3, 4, 3), (2 * 2 * 4 * 3, 2 * 4 * 3, 4 * 3, 3, 1))):
        pk.shape[i], pk.stride[i] = n, s
    pk.data = kp
    pc = abi.cache_desc(1, 4, 2, 8, pk, pk)
    assert L.kvx_validate_cache_desc(C.byref(pc)) == Status.INVALID_ARGUMENT

    cache = make_cache_nhd(kp, vp)
    io_k = np.zeros(64, np.float32)
    io_v = np.zeros(64, np.float32)
    slots = np.arange(4, dtype=np.int64)
    mk = lambda s=slots.ctypes.data: abi.make_write(4, 2, 8, DType.F32, H, io_k.ctypes.data,
                                                    io_v.ctypes.data, DType.S64, s)
    w = mk()
    assert L.kvx_write_kv(C.byref(cache), C.byref(w), None) == Status.OK
    w.slots.dtype = DType.U32
    assert L.kvx_write_kv(C.byref(cache), C.byref(w), None) == Status.INVALID_ARGUMENT
    w = mk()
    w.slots.token_count = 3
    assert L.kvx_write_kv(C.byref(cache), C.byref(w), None) == Status.INVALID_ARGUMENT
    w = mk(None)
    assert L.kvx_write_kv(C.byref(cache), C.byref(w), None) == Status.INVALID_ARGUMENT
    w = mk()
    w.io.key.size = C.sizeof(abi.TensorDesc) - 4
    assert L.kvx_write_kv(C.byref(cache), C.byref(w), None) == Status.INVALID_ARGUMENT

    table = np.array([0, 1], np.int32)
    lens = np.array([4, 4], np.int32)
    gk = np.zeros(2 * 4 * 2 * 8, np.float32)
    gv = np.zeros_like(gk)
    tb = abi.make_block_table_packed(2, 1, DType.S32, table.ctypes.data)
    sl = abi.make_seq_lens(2, DType.S32, lens.ctypes.data)
    mg = lambda: abi.make_gather(2, 4, 2, 8, DType.F32, H, gk.ctypes.data, gv.ctypes.data,
                                 tb, sl)
    g = mg()
    assert L.kvx_gather_kv(C.byref(cache), C.byref(g), None) == Status.OK
    g.block_table.indices_count = 1
    assert L.kvx_gather_kv(C.byref(cache), C.byref(g), None) == Status.INVALID_ARGUMENT
    g = mg()
    g.seq_lens.seq_count = 1
    assert L.kvx_gather_kv(C.byref(cache), C.byref(g), None) == Status.INVALID_ARGUMENT
    g = mg()
    g.block_table.index_dtype = DType.U32
    assert L.kvx_gather_kv(C.byref(cache), C.byref(g), None) == Status.INVALID_ARGUMENT


@pytest.mark.parametrize("binary", [ob.REF_TEST_REF, ob.REF_TEST_OURS],
                         ids=["ref-abi", "kvx_amd"])
def test_reference_abi_test_binary(binary):
    """The reference's own kvx_abi_test.c (built from /root/reference by
    oracle/build.py); the kvx_amd variant links it with libkvx_amd.so."""
    if not binary.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    r = subprocess.run([str(binary)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stderr


# ---------------------------------------------------------------------------
# Randomized comparison with the reference kvx_abi.c.

INTS = [0, 1, 2, 3, 4, 7, 8, 16, 64, 0xFFFFFFFF]
DTYPES = list(range(0, 12))
LAYOUTS = [0, 1, 2, 3, 4, 15]
PTRS = [None, FAKE]


def _base_case(rng: random.Random):
    layout = rng.choice([Layout.BLOCK_NHD, Layout.BLOCK_HND, Layout.BLOCK_HND_PACKED])
    dt = rng.choice([DType.F16, DType.BF16, DType.F32, DType.F8_E4M3])
    nb, bs, Hh, D = rng.choice([1, 3, 8]), rng.choice([1, 4, 16]), rng.choice([1, 2, 4]), \
        rng.choice([8, 16, 64])
    pack = rng.choice([1, 2, 4, 8])
    cache = abi.make_cache(layout, dt, H, nb, bs, Hh, D, FAKE, FAKE + 64, pack=pack)
    T = rng.choice([0, 1, 5])
    w = abi.make_write(T, Hh, D, dt, H, FAKE, FAKE, rng.choice([DType.S32, DType.S64]),
                       FAKE)
    S, L = rng.choice([1, 3]), rng.choice([1, 8])
    mbps = rng.choice([1, 2, 4])
    idt = rng.choice([DType.S32, DType.S64])
    tb = abi.make_block_table_packed(S, mbps, idt, FAKE)
    sl = abi.make_seq_lens(S, idt, FAKE)
    g = abi.make_gather(S, L, Hh, D, dt, H, FAKE, FAKE, tb, sl)
    return cache, w, g


def _mutable_fields(obj, prefix=""):
    """(owner, field name, kind) for every scalar field reachable in obj."""
    out = []
    for name, typ in obj._fields_:
        val = getattr(obj, name)
        if isinstance(val, C.Structure):
            out += _mutable_fields(val, prefix + name + ".")
        elif isinstance(val, C.Array):
            for i in range(len(val)):
                out.append((val, i, "int64"))
        else:
            kind = "ptr" if typ is C.c_void_p else "int"
            out.append((obj, name, kind))
    return out


def _mutate(rng: random.Random, obj, n: int):
    fields = _mutable_fields(obj)
    for _ in range(n):
        owner, key, kind = rng.choice(fields)
        if kind == "ptr":
            value = rng.choice(PTRS)
        elif kind == "int64":
            cur = owner[key]
            value = rng.choice([0, 1, -1, cur + 1, cur - 1, cur * 2, 3])
        else:
            cur = getattr(owner, key)
            value = rng.choice(INTS + DTYPES + LAYOUTS + [cur + 1, cur - 4 if cur >= 4 else 0])
        if key in ("memory",):
            continue  # keep every buffer HOST: validation-only on both sides
        if kind == "int64":
            owner[key] = value
        else:
            try:
                setattr(owner, key, value)
            except (TypeError, OverflowError):
                pass


def test_random_mutations_match_reference_abi(kvx_lib):
    if not ob.REF_ABI_LIB.exists():
        pytest.skip("oracle/_ref not built (reference tree absent)")
    ref = abi.bind_like(C.CDLL(str(ob.REF_ABI_LIB)))
    rng = random.Random(20261201)
    checked = {"cache": 0, "write": 0, "gather": 0}
    extended = 0
    codes = set()
    for it in range(6000):
        cache, w, g = _base_case(rng)
        target = rng.choice(["cache", "write", "gather"])
        obj = {"cache": cache, "write": w, "gather": g}[target]
        _mutate(rng, obj, rng.choice([0, 1, 1, 2, 3]))
        # The reference rejects KVX_LAYOUT_BLOCK_CUSTOM as UNSUPPORTED
        # (kvx_abi.c:307-309); this build validates its shape and goes on, so
        # any later code may follow there.
        custom = Layout.BLOCK_CUSTOM in (cache.k.layout, cache.v.layout)

        def same(a, b, what):
            nonlocal extended
            if a != b and custom and a == Status.UNSUPPORTED:
                extended += 1
            else:
                assert a == b, (what, it)

        a = ref.kvx_validate_cache_desc(C.byref(cache))
        b = kvx_lib.kvx_validate_cache_desc(C.byref(cache))
        same(a, b, "validate")
        a = ref.kvx_write_kv(C.byref(cache), C.byref(w), None)
        b = kvx_lib.kvx_write_kv(C.byref(cache), C.byref(w), None)
        same(a, b, "write")
        codes.add(a)
        a = ref.kvx_gather_kv(C.byref(cache), C.byref(g), None)
        b = kvx_lib.kvx_gather_kv(C.byref(cache), C.byref(g), None)
        # The reference's last gather check rejects non-PACKED tables
        # (kvx_abi.c:462-464); this build gathers RAGGED / KV_OFFSETS, so a
        # descriptor that passed every other check is OK here.
        if (a == Status.UNSUPPORTED and b == Status.OK and
                g.block_table.format in (TableFormat.RAGGED, TableFormat.KV_OFFSETS)):
            extended += 1
        else:
            same(a, b, "gather")
        codes.add(a)
        checked[target] += 1
    # the sweep reached every code the ABI path can return
    assert {Status.OK, Status.INVALID_ARGUMENT, Status.UNSUPPORTED} <= codes
