"""GPU K/V cache-write scatter: bit-exact against the oracle's store
(store_kv.cu:20-36 / cpu_model.cpp:153-157) on every slot of the cache."""
import numpy as np
import pytest
import torch

import oracle
from gpu_util import TORCH_DT, from_dev_cache, i32, random_cache, round_to, to_dev_cache

pytestmark = pytest.mark.gpu


def _run(src, cache, n_tokens, kv_dim, num_blocks, bs, seed, pad_every=0):
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    slots_total = num_blocks * bs
    slots = rng.permutation(slots_total)[:n_tokens].astype(np.int32)
    if pad_every:
        slots[::pad_every] = -1
    # the device source is `src`; the oracle sees the same values
    k = round_to(rng.standard_normal((n_tokens, kv_dim), dtype=np.float32), src)
    v = round_to(rng.standard_normal((n_tokens, kv_dim), dtype=np.float32), src)
    init_k = random_cache(rng, (slots_total, kv_dim), cache)
    init_v = init_k[::-1].copy()
    ok = slots >= 0
    want_k, want_v = init_k.copy(), init_v.copy()
    oracle.store_kv(k[ok], v[ok], slots[ok], want_k, want_v)

    from llm_engine_amd import kernels
    kd = torch.from_numpy(k).to(dev).to(TORCH_DT[src])
    vd = torch.from_numpy(v).to(dev).to(TORCH_DT[src])
    kc, vc = to_dev_cache(init_k, dev), to_dev_cache(init_v, dev)
    kernels.store_kv(kd, vd, i32(slots, dev), kc, vc)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev_cache(kc).view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(from_dev_cache(vc).view(np.uint8), want_v.view(np.uint8))


@pytest.mark.parametrize("src,cache", [(s, c) for s in ("f32", "bf16", "f16") for c in ("f32", "bf16", "f16")])
def test_kv_write_config3_step(gpu, src, cache):
    """544 rows of kv_dim 128 into a fragmented 16384-block pool (config 3),
    every source/cache type pair (fp16 is the reference's __half)."""
    _run(src, cache, 544, 128, 16384, 16, seed=1)


def test_kv_write_padding_and_shapes(gpu):
    _run("f32", "bf16", 1000, 256, 512, 16, seed=2, pad_every=7)  # TinyLlama kv_dim 256
    _run("f32", "f32", 1, 128, 4, 16, seed=3)
    _run("bf16", "bf16", 4096, 128, 4096, 16, seed=4)
    _run("f16", "f16", 777, 256, 1024, 16, seed=9, pad_every=5)


def _run_fused(act, cache, n_tokens, q_heads, kv_heads, head_dim, num_blocks, seed,
               bias=True, pad_every=0, bad_pos_every=0, stride_pad=0, max_pos=4096, theta=1e6):
    """le_rope_kv_cache_write against the oracle's own sequence: bias add
    (rounded to the activation dtype, as a separate add stores it), RoPE
    (ops.h:55-66), store_kv (store_kv.cu:20-36). Bit-exact: q, and every slot
    of both caches."""
    dev = torch.device("cuda:0")
    rng = np.random.default_rng(seed)
    bs = 16
    qd, kvd = q_heads * head_dim, kv_heads * head_dim
    row = qd + 2 * kvd + stride_pad
    slots_total = num_blocks * bs
    slots = rng.permutation(slots_total)[:n_tokens].astype(np.int32)
    pos = rng.integers(0, max_pos, size=n_tokens).astype(np.int32)
    if pad_every:
        slots[::pad_every] = -1
    if bad_pos_every:
        pos[1::bad_pos_every] = max_pos + 3
        pos[2::bad_pos_every] = -1
    qkv = rng.standard_normal((n_tokens, row), dtype=np.float32)
    b = rng.standard_normal(qd + 2 * kvd, dtype=np.float32) if bias else None
    rnd = lambda a: round_to(a, act)
    qkv = rnd(qkv)
    cos_t, sin_t = oracle.rope_tables(head_dim, max_pos, theta)

    # oracle side
    x = qkv[:, :qd + 2 * kvd].copy()
    if b is not None:
        x = rnd(x + b[None, :])
    x = np.ascontiguousarray(x)
    ok_pos = (pos >= 0) & (pos < max_pos)
    xr = x.copy()
    oracle.rope(xr, np.where(ok_pos, pos, 0), cos_t, sin_t, q_heads + kv_heads, head_dim)
    want_q = rnd(np.where(ok_pos[:, None], xr[:, :qd], 0.0).astype(np.float32))
    k_rows, v_rows = xr[:, qd:qd + kvd], x[:, qd + kvd:]
    init_k = random_cache(rng, (slots_total, kvd), cache)
    init_v = init_k[::-1].copy()
    want_k, want_v = init_k.copy(), init_v.copy()
    ok = (slots >= 0) & ok_pos
    oracle.store_kv(np.ascontiguousarray(k_rows[ok]), np.ascontiguousarray(v_rows[ok]), slots[ok], want_k, want_v)

    from llm_engine_amd import kernels
    qkv_d = torch.from_numpy(qkv).to(dev).to(TORCH_DT[act])
    kc, vc = to_dev_cache(init_k, dev), to_dev_cache(init_v, dev)
    bias_d = None if b is None else torch.from_numpy(b).to(dev)
    q = kernels.rope_store_kv(qkv_d, i32(pos, dev), i32(slots, dev), torch.from_numpy(cos_t).to(dev),
                              torch.from_numpy(sin_t).to(dev), q_heads, kv_heads, head_dim, kc, vc, bias=bias_d)
    torch.cuda.synchronize()
    got_q = q.float().cpu().numpy()
    assert np.array_equal(got_q.view(np.uint32), want_q.view(np.uint32)), \
        f"q mismatch: max|diff| {np.abs(got_q - want_q).max()}"
    assert np.array_equal(from_dev_cache(kc).view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(from_dev_cache(vc).view(np.uint8), want_v.view(np.uint8))


@pytest.mark.parametrize("act,cache", [("f32", "f32"), ("f32", "bf16"), ("bf16", "bf16"), ("f16", "f16"),
                                       ("f32", "f16")])
def test_rope_kv_write_qwen_step(gpu, act, cache):
    """Qwen2.5-0.5B shape (14/2 x 64, qkv bias), a 544-row mixed step into a
    fragmented 16384-block pool."""
    _run_fused(act, cache, 544, 14, 2, 64, 16384, seed=5)


def test_rope_kv_write_edges(gpu):
    """TinyLlama shape without bias; padding slots, out-of-range positions,
    a padded qkv row stride, a single token, head_dim 128."""
    _run_fused("bf16", "bf16", 300, 32, 4, 64, 1024, seed=6, bias=False, pad_every=5, theta=1e4, max_pos=2048)
    _run_fused("f32", "f32", 257, 14, 2, 64, 512, seed=7, bad_pos_every=9, stride_pad=8)
    _run_fused("f32", "bf16", 1, 8, 1, 128, 4, seed=8)
    _run_fused("f16", "f16", 300, 32, 4, 64, 1024, seed=10, pad_every=5, bad_pos_every=11, theta=1e4,
               max_pos=2048)
