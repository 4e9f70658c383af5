"""GPU parity with fp16 (IEEE binary16) caches and activations: the element
type of every reference launcher on this path (cuda_kernels.h:43-64 take
__half q, K/V caches and out; cuda_model.cu:76-78,276-285 keep fp16 weights
and caches). The oracle sees exactly the fp16 values the device holds,
widened to fp32 (exact), as the reference widens each element in registers.

Tolerances (max-abs against the fp32 oracle): twice the error of the host
emulation of the kernels' roundings on the same case (tests/precision.py: q
and the softmax weights rounded to fp16 before the MFMA; emulated 2.3e-4 on
config 2, where the GPU shows 2.9e-4, and 8.1e-4 on config 3, GPU 8.6e-4),
inside the north star's 2e-2 for 16-bit K/V. fp16 outputs add their own
rounding (<= 2^-11 relative, |out| < 4)."""
import numpy as np
import pytest
import torch

from cases import loguniform_ctx, make_case
from gpu_util import device_q, emulated_bar, i32, max_abs, oracle_out, poison_unused, slices_of, to_dev_cache

pytestmark = pytest.mark.gpu

OUT_ROUND = 4 * 2.0 ** -11


def run_both(case, act, dev, **plan_kw):
    """The reference-shaped entry and the ragged plan entry on one case."""
    from llm_engine_amd import kernels
    q, qh = device_q(case, act, dev)
    kc, vc = to_dev_cache(case.k_cache, dev), to_dev_cache(case.v_cache, dev)
    assert kc.dtype == torch.float16
    a = kernels.attention_decode(q, kc, vc, i32(case.tables, dev), i32(case.table_offset, dev),
                                 i32(case.token_seq, dev), i32(case.token_pos, dev), case.q_heads,
                                 case.kv_heads, case.head_dim, case.block_size, case.scale)
    plan = kernels.Plan(slices_of(case), case.q_heads, case.kv_heads, case.head_dim, case.block_size,
                        kc.dtype, **plan_kw).upload()
    b = kernels.ragged_paged_attention(q, kc, vc, plan, case.scale)
    torch.cuda.synchronize()
    assert a.dtype == act and b.dtype == act
    return a.float().cpu().numpy(), b.float().cpu().numpy(), qh, plan


@pytest.mark.parametrize("act", [torch.float16, torch.float32])
def test_config2_f16(gpu, act):
    """Config 2 at full size with fp16 K/V: 64 sequences, contexts
    log-uniform in [64, 4096], a fragmented 32768-block pool."""
    rng = np.random.default_rng(2)
    ctx = loguniform_ctx(rng, 64, 64, 4096)
    case = make_case(ctx, num_blocks=32768, seed=2, kv_f16=True)
    a, b, qh, _ = run_both(case, act, gpu)
    want = oracle_out(case, qh)
    tol = emulated_bar(case, qh, want) + (OUT_ROUND if act == torch.float16 else 0.0)
    ea, eb = max_abs(a, want), max_abs(b, want)
    print(f"config2 f16 act={act}: reference-shaped {ea:.3e} ragged {eb:.3e}")
    assert ea < tol and eb < tol


@pytest.mark.parametrize("act", [torch.float16, torch.float32])
def test_config3_f16(gpu, act):
    """Config 3 with fp16 K/V: 32 decode rows + 2 prefill chunks of 512 at
    cached offsets 0 and 1024, chunk rows on the fp16 MFMA, one launch."""
    rng = np.random.default_rng(3)
    dec_ctx = rng.integers(256, 2049, 32)
    case = make_case(list(dec_ctx) + [512, 1536], q_len=[1] * 32 + [512, 512], num_blocks=16384, seed=3,
                     kv_f16=True)
    a, b, qh, plan = run_both(case, act, gpu)
    assert plan.plan.n_tokens == 1056 and plan.plan.n_chunk_items > 0
    want = oracle_out(case, qh)
    tol = emulated_bar(case, qh, want) + (OUT_ROUND if act == torch.float16 else 0.0)
    ea, eb = max_abs(a, want), max_abs(b, want)
    print(f"config3 f16 act={act}: reference-shaped {ea:.3e} ragged {eb:.3e}")
    assert ea < tol and eb < tol


@pytest.mark.parametrize("q_heads,kv_heads,head_dim", [(32, 4, 64), (8, 8, 64), (16, 2, 128), (4, 1, 128)])
def test_f16_other_shapes(gpu, q_heads, kv_heads, head_dim):
    """GQA group 8 (TinyLlama), no grouping, head_dim 128: decode rows and
    prefill chunks (at cached offsets) in one step."""
    rng = np.random.default_rng(q_heads * 100 + head_dim + 1)
    ctx = list(loguniform_ctx(rng, 10, 1, 2500)) + [300, 700]
    q_len = [1] * 10 + [64, 45]
    case = make_case(ctx, q_len=q_len, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
                     num_blocks=4096, seed=17, kv_f16=True)
    a, b, qh, plan = run_both(case, torch.float16, gpu)
    want = oracle_out(case, qh)
    assert plan.plan.n_chunk_items > 0
    tol = emulated_bar(case, qh, want) + OUT_ROUND
    assert max_abs(a, want) < tol
    assert max_abs(b, want) < tol


@pytest.mark.parametrize("seed", range(6))
def test_f16_random_steps(gpu, seed):
    """Seeded random mixed steps: block sizes 8-32, GQA 1/4/7/8, split and
    unsplit rows and tiles, several partition sizes."""
    rng = np.random.default_rng(500 + seed)
    q_heads, kv_heads = [(14, 2), (32, 4), (8, 8), (4, 1)][seed % 4]
    head_dim = 128 if seed % 3 == 2 else 64
    bs = [8, 16, 32][seed % 3]
    S = int(rng.integers(2, 12))
    ctx = rng.integers(1, 3000, S)
    q_len = np.where(rng.random(S) < 0.3, np.minimum(ctx, rng.integers(2, 200, S)), 1)
    case = make_case(ctx, q_len=q_len, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, block_size=bs,
                     num_blocks=int(((ctx + bs - 1) // bs).sum()) + 64, seed=600 + seed, kv_f16=True)
    poison_unused(case)  # no dead cache row may reach a result
    _, b, qh, plan = run_both(case, torch.float16, gpu, partition_tokens=int(rng.choice([0, 256, 640])))
    want = oracle_out(case, qh)
    assert np.isfinite(b).all()
    err = max_abs(b, want)
    print(f"seed {seed}: {q_heads}/{kv_heads}x{head_dim} bs {bs} rows {plan.plan.n_tokens} "
          f"parts {plan.plan.n_parts}: max|err| {err:.3e}")
    assert err < emulated_bar(case, qh, want) + OUT_ROUND


def test_f16_store_then_attend(gpu):
    """le_ragged_paged_attention_store with fp16 rows and cache: on a decode
    step the store happens inside the attention launch; the cache bytes equal
    the oracle's scatter and the output the oracle's attention."""
    import oracle
    from llm_engine_amd import kernels
    rng = np.random.default_rng(23)
    ctx = loguniform_ctx(rng, 24, 20, 3000)
    case = make_case(ctx, num_blocks=8192, seed=23, kv_f16=True)
    plan = kernels.Plan(slices_of(case), case.q_heads, case.kv_heads, case.head_dim, case.block_size,
                        torch.float16).upload()
    kvd = case.kv_heads * case.head_dim
    k_new = oracle.f32_to_f16(rng.standard_normal((case.n_tokens, kvd), dtype=np.float32))
    v_new = oracle.f32_to_f16(rng.standard_normal((case.n_tokens, kvd), dtype=np.float32))
    kc, vc = to_dev_cache(case.k_cache, gpu), to_dev_cache(case.v_cache, gpu)
    oracle.store_kv(k_new.astype(np.float32), v_new.astype(np.float32), plan.host_array("slots"), case.k_cache,
                    case.v_cache)
    q, qh = device_q(case, torch.float16, gpu)
    out = kernels.ragged_paged_attention(q, kc, vc, plan, case.scale, k_new=torch.from_numpy(k_new).to(gpu),
                                         v_new=torch.from_numpy(v_new).to(gpu))
    torch.cuda.synchronize()
    assert np.array_equal(kc.cpu().numpy().view(np.uint16), case.k_cache.view(np.uint16))
    assert np.array_equal(vc.cpu().numpy().view(np.uint16), case.v_cache.view(np.uint16))
    want = oracle_out(case, qh)
    assert max_abs(out.float().cpu().numpy(), want) < emulated_bar(case, qh, want) + OUT_ROUND
