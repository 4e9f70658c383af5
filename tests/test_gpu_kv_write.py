"""GPU K/V cache-write scatter: bit-exact against the oracle's store
(store_kv.cu:20-36 / cpu_model.cpp:153-157) on every slot of the cache."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import i32, to_dev_cache

pytestmark = pytest.mark.gpu


def _run(src_bf16, cache_bf16, n_tokens, kv_dim, num_blocks, bs, seed, pad_every=0):
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    slots_total = num_blocks * bs
    slots = rng.permutation(slots_total)[:n_tokens].astype(np.int32)
    if pad_every:
        slots[::pad_every] = -1
    k = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32)
    v = rng.standard_normal((n_tokens, kv_dim), dtype=np.float32)
    if src_bf16:  # the device source is bf16; the oracle sees the same values
        k = oracle.bf16_to_f32(oracle.f32_to_bf16(k))
        v = oracle.bf16_to_f32(oracle.f32_to_bf16(v))
    cdt = np.uint16 if cache_bf16 else np.float32
    init_k = rng.integers(0, 2**16, size=(slots_total, kv_dim)).astype(cdt) if cache_bf16 else \
        rng.standard_normal((slots_total, kv_dim), dtype=np.float32)
    init_v = init_k[::-1].copy()
    ok = slots >= 0
    want_k, want_v = init_k.copy(), init_v.copy()
    oracle.store_kv(k[ok], v[ok], slots[ok], want_k, want_v)

    from llm_engine_amd import kernels
    tdt = torch.bfloat16 if src_bf16 else torch.float32
    kd = torch.from_numpy(k).to(dev).to(tdt)
    vd = torch.from_numpy(v).to(dev).to(tdt)
    kc, vc = to_dev_cache(init_k, dev), to_dev_cache(init_v, dev)
    kernels.store_kv(kd, vd, i32(slots, dev), kc, vc)
    torch.cuda.synchronize()
    got_k = kc.cpu().view(torch.int16).numpy().view(np.uint16) if cache_bf16 else kc.cpu().numpy()
    got_v = vc.cpu().view(torch.int16).numpy().view(np.uint16) if cache_bf16 else vc.cpu().numpy()
    assert np.array_equal(got_k.view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(got_v.view(np.uint8), want_v.view(np.uint8))


@pytest.mark.parametrize("src_bf16,cache_bf16", [(False, False), (False, True), (True, True), (True, False)])
def test_kv_write_config3_step(gpu, src_bf16, cache_bf16):
    """544 rows of kv_dim 128 into a fragmented 16384-block pool (config 3)."""
    _run(src_bf16, cache_bf16, 544, 128, 16384, 16, seed=1)


def test_kv_write_padding_and_shapes(gpu):
    _run(False, True, 1000, 256, 512, 16, seed=2, pad_every=7)  # TinyLlama kv_dim 256
    _run(False, False, 1, 128, 4, 16, seed=3)
    _run(True, True, 4096, 128, 4096, 16, seed=4)
