"""GPU tests of torch.ops._C_cache_ops.reshape_and_cache_flash_kvx, the
PyTorch-ROCm op over kvx_launch_write_kv (kvx_amd/csrc/torch_ops.cpp).

Each write is checked bit for bit twice: against the CPU oracle's write
(oracle_write_kv over the cache's own strides) and against torch advanced
indexing on the cache tensor (a scatter that shares nothing with either).
Covers the reference patch's own test case (patches/vllm/kvx.patch:343-398:
8 tokens, 4 heads x 64, block 16, NHD, f16 / f32), bf16, int32 / int64 slots
with -1 entries, vLLM's HND cache (a stride-permuted [nb, bs, H, D] view),
key / value with more rows than slot_mapping, the FP8 E4M3 cache
("fp8" / "fp8_e4m3", uint8 and float8_e4m3fn storage), a non-default
stream, and the op's argument checks.
"""
import numpy as np
import pytest
import torch

import oracle
from kvx_amd import torch_ops
from kvx_amd.abi import DType, Layout

from gpu_helpers import np_bytes

pytestmark = pytest.mark.gpu
DEV = "cuda"
TDT = {torch.float16: DType.F16, torch.bfloat16: DType.BF16, torch.float32: DType.F32}
op = None


@pytest.fixture(autouse=True, scope="module")
def _load():
    global op
    torch_ops.load()
    op = torch.ops._C_cache_ops.reshape_and_cache_flash_kvx


def flat_storage(t):
    """The whole storage of `t` (storage offset 0) as a 1-D uint8 tensor."""
    n = t.untyped_storage().nbytes() // t.element_size()
    return t.as_strided((n,), (1,), 0).view(torch.uint8)


def vllm_cache(nb, bs, H, D, dtype, layout, gen):
    """vLLM's logical [nb, bs, H, D] cache, random bytes: contiguous (NHD) or
    a permuted view of [nb, H, bs, D] storage (HND)."""
    if layout == "NHD":
        t = torch.empty((nb, bs, H, D), dtype=dtype, device=DEV)
    else:
        t = torch.empty((nb, H, bs, D), dtype=dtype, device=DEV).permute(0, 2, 1, 3)
    raw = flat_storage(t)
    raw.copy_(torch.randint(0, 256, raw.shape, dtype=torch.uint8, generator=gen).to(DEV))
    return t


BITS = {1: torch.uint8, 2: torch.int16, 4: torch.int32}


def torch_scatter(cache, rows, slots, bs):
    """cache[slot // bs, slot % bs] = rows[t] for slots >= 0, in place, as bit
    patterns."""
    it = BITS[cache.element_size()]
    s = slots.long()
    ok = s >= 0
    cache.view(it)[s[ok] // bs, s[ok] % bs] = rows[: s.numel()].view(it)[ok]


def storage_bytes(t):
    return np_bytes(flat_storage(t))


def oracle_expect(cache, rows, slots, bs, nb, H, D, io_dt, cache_dt, scale=1.0):
    """The cache storage after the oracle's write of `rows` at `slots`."""
    base = storage_bytes(cache)
    g = oracle.Geometry(Layout.BLOCK_NHD, cache.stride(), 1)
    n = slots.numel()
    kb = base.copy()
    oracle.write_kv(g, g, np_bytes(rows[:n]), np_bytes(rows[:n]), kb, kb.copy(),
                    slots.cpu().numpy(), heads=H, head_dim=D, block_size=bs, num_blocks=nb,
                    io_dtype=io_dt, cache_dtype=cache_dt, k_scale=scale, v_scale=scale)
    return kb


def rand_slots(nb, bs, T, dtype, gen, invalid=0.2):
    s = torch.randperm(nb * bs, generator=gen)[:T]
    s[torch.rand(T, generator=gen) < invalid] = -1
    return s.to(dtype).to(DEV)


def run_and_check(key, value, kc, vc, slots, bs, kv_cache_dtype="auto", ks=None, vs=None):
    nb, _, H, D = kc.shape
    io_dt = TDT[key.dtype]
    fp8 = kv_cache_dtype != "auto"
    e5m2 = kv_cache_dtype == "fp8_e5m2"
    cache_dt = (DType.F8_E5M2 if e5m2 else DType.F8_E4M3) if fp8 else io_dt
    want_k = oracle_expect(kc, key, slots, bs, nb, H, D, io_dt, cache_dt,
                           ks.item() if fp8 else 1.0)
    want_v = oracle_expect(vc, value, slots, bs, nb, H, D, io_dt, cache_dt,
                           vs.item() if fp8 else 1.0)
    ref_k, ref_v = kc.clone(), vc.clone()
    if fp8:
        # torch's own cast, on the CPU (IEEE f32 division), after saturation
        f8, top = (torch.float8_e5m2, 57344.0) if e5m2 else (torch.float8_e4m3fn, 448.0)
        qk = (key.float().cpu() / ks.cpu()).clamp(-top, top).to(f8)
        qv = (value.float().cpu() / vs.cpu()).clamp(-top, top).to(f8)
        qk, qv = qk.view(torch.uint8).to(DEV), qv.view(torch.uint8).to(DEV)
        torch_scatter(ref_k, qk, slots, bs)
        torch_scatter(ref_v, qv, slots, bs)
    else:
        torch_scatter(ref_k, key, slots, bs)
        torch_scatter(ref_v, value, slots, bs)
    one = torch.ones(1, dtype=torch.float32, device=DEV)
    op(key, value, kc, vc, slots, kv_cache_dtype, one if ks is None else ks,
       one if vs is None else vs)
    torch.cuda.synchronize()
    got_k, got_v = storage_bytes(kc), storage_bytes(vc)
    assert np.array_equal(got_k, want_k)
    assert np.array_equal(got_v, want_v)
    assert np.array_equal(got_k, storage_bytes(ref_k))
    assert np.array_equal(got_v, storage_bytes(ref_v))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_reference_patch_case(dtype):
    """kvx.patch:343-398: slot_mapping = arange(8), NHD, 4 heads x 64."""
    gen = torch.Generator().manual_seed(0)
    T, H, D, bs, nb = 8, 4, 64, 16, 16
    qkv = torch.randn(T, 3, H, D, dtype=dtype, generator=gen).to(DEV)
    _, key, value = qkv.unbind(dim=1)
    key, value = key.contiguous(), value.contiguous()  # as vLLM's wrapper does
    kc = vllm_cache(nb, bs, H, D, dtype, "NHD", gen)
    vc = vllm_cache(nb, bs, H, D, dtype, "NHD", gen)
    run_and_check(key, value, kc, vc, torch.arange(T, dtype=torch.long, device=DEV), bs)


@pytest.mark.parametrize("layout", ["NHD", "HND"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("slot_dtype", [torch.int64, torch.int32])
def test_random_writes(layout, dtype, slot_dtype):
    gen = torch.Generator().manual_seed(
        ["NHD", "HND"].index(layout) * 10 + TDT[dtype] * 2 + (slot_dtype == torch.int32))
    H, D, bs, nb, T = 8, 128, 16, 40, 300
    key = torch.randn(T, H, D, generator=gen).to(dtype).to(DEV)
    value = torch.randn(T, H, D, generator=gen).to(dtype).to(DEV)
    kc = vllm_cache(nb, bs, H, D, dtype, layout, gen)
    vc = vllm_cache(nb, bs, H, D, dtype, layout, gen)
    run_and_check(key, value, kc, vc, rand_slots(nb, bs, T, slot_dtype, gen), bs)


def test_rows_past_slot_mapping_are_ignored():
    """vLLM passes padded key / value with num_actual_tokens slots."""
    gen = torch.Generator().manual_seed(3)
    H, D, bs, nb = 4, 64, 16, 8
    key = torch.randn(50, H, D, generator=gen).half().to(DEV)
    value = torch.randn(50, H, D, generator=gen).half().to(DEV)
    kc = vllm_cache(nb, bs, H, D, torch.float16, "HND", gen)
    vc = vllm_cache(nb, bs, H, D, torch.float16, "HND", gen)
    run_and_check(key, value, kc, vc, rand_slots(nb, bs, 37, torch.int64, gen), bs)


@pytest.mark.parametrize("kv_cache_dtype,storage", [
    ("fp8", torch.uint8), ("fp8", torch.float8_e4m3fn), ("fp8_e4m3", torch.uint8),
    ("fp8_e4m3", torch.float8_e4m3fn), ("fp8_e5m2", torch.uint8),
    ("fp8_e5m2", torch.float8_e5m2)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_fp8_cache(kv_cache_dtype, storage, dtype):
    gen = torch.Generator().manual_seed(5)
    H, D, bs, nb, T = 8, 128, 16, 24, 200
    key = (torch.randn(T, H, D, generator=gen) * 3).to(dtype).to(DEV)
    value = (torch.randn(T, H, D, generator=gen) * 3).to(dtype).to(DEV)
    layout = "NHD" if storage == torch.uint8 else "HND"
    kc = vllm_cache(nb, bs, H, D, storage, layout, gen)
    vc = vllm_cache(nb, bs, H, D, storage, layout, gen)
    top = 57344.0 if kv_cache_dtype == "fp8_e5m2" else 448.0
    ks = (key.float().abs().amax() / top).reshape(1)
    vs = (value.float().abs().amax() / (top * 0.7)).reshape(1)   # some values saturate
    run_and_check(key, value, kc, vc, rand_slots(nb, bs, T, torch.int64, gen), bs,
                  kv_cache_dtype, ks, vs)


def test_current_stream_is_used():
    gen = torch.Generator().manual_seed(7)
    H, D, bs, nb, T = 8, 128, 16, 64, 512
    key = torch.randn(T, H, D, generator=gen).bfloat16().to(DEV)
    value = torch.randn(T, H, D, generator=gen).bfloat16().to(DEV)
    kc = vllm_cache(nb, bs, H, D, torch.bfloat16, "NHD", gen)
    vc = vllm_cache(nb, bs, H, D, torch.bfloat16, "NHD", gen)
    slots = rand_slots(nb, bs, T, torch.int64, gen, invalid=0.0)
    ref_k = kc.clone()
    torch_scatter(ref_k, key, slots, bs)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        torch_ops.reshape_and_cache_flash_kvx(key, value, kc, vc, slots)
        done = torch.cuda.Event()
        done.record(side)
    done.synchronize()
    assert torch.equal(kc.view(torch.int16), ref_k.view(torch.int16))


def test_argument_checks():
    H, D, bs, nb, T = 4, 64, 16, 4, 8
    key = torch.zeros(T, H, D, dtype=torch.float16, device=DEV)
    kc = torch.zeros(nb, bs, H, D, dtype=torch.float16, device=DEV)
    slots = torch.arange(T, device=DEV)
    one = torch.ones(1, device=DEV)
    kc8 = torch.zeros(nb, bs, H, D, dtype=torch.uint8, device=DEV)
    cases = [
        ((key, key, kc, kc.clone(), slots, "fp8_e4m3fnuz", one, one), "kv_cache_dtype"),
        ((key, key, kc.to(torch.float8_e4m3fn), kc.to(torch.float8_e4m3fn), slots, "fp8_e5m2",
          one, one), "matching float8"),
        ((key, key.float(), kc, kc.clone(), slots, "auto", one, one), "key/value dtype mismatch"),
        ((key, key, kc, kc.float(), slots, "auto", one, one), "cache dtype mismatch"),
        ((key, key, kc.float(), kc.float(), slots, "auto", one, one),
         "key/value dtype must match cache dtype"),
        ((key, key, kc, kc.clone(), slots.float(), "auto", one, one), "int32 or int64"),
        ((key, key, kc, kc.clone(), slots.reshape(2, 4), "auto", one, one), "1D"),
        ((key.transpose(1, 2).contiguous().transpose(1, 2), key, kc, kc.clone(), slots, "auto",
          one, one), "key must be contiguous"),
        ((key, key, kc[:, :, :2], kc[:, :, :2].clone(), slots, "auto", one, one),
         "num_heads"),
        ((key, key, kc, kc[:2].clone(), slots, "auto", one, one), "cache shape mismatch"),
        ((key[:4], key[:4], kc, kc.clone(), slots, "auto", one, one), "fewer rows"),
        ((key, key, kc8, kc8.clone(), slots, "fp8", one, one.double()), "float32"),
        ((key, key, kc8, kc8.clone(), slots, "fp8", one, one.cpu()), "float32"),
    ]
    for args, msg in cases:
        with pytest.raises(RuntimeError, match=msg):
            op(*args)
