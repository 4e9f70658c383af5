"""le_ragged_paged_attention_qkv: a layer's attention straight from its
stacked QKV rows. On a decode-only step the bias, the RoPE of q and k and the
K/V store run inside the attention launch; on any other step the entry point
runs le_rope_kv_cache_write into a scratch q and then the ragged attention.
Either way the result must be bit-identical to those two calls made
separately (each pinned against the oracle by test_gpu_kv_write.py and
test_gpu_attention.py): the output, and every slot of both caches."""
import numpy as np
import pytest
import torch

import oracle
from cases import make_case
from gpu_util import TORCH_DT, max_abs, oracle_out, slices_of, to_dev_cache

pytestmark = pytest.mark.gpu


def _run(gpu, *, act, kv, bias, ctx, q_len=None, q_heads=14, kv_heads=2, head_dim=64,
         block_size=16, max_pos=4096, partition_tokens=None, stride_pad=0, seed=0, theta=1e6):
    from llm_engine_amd import kernels
    rng = np.random.default_rng(seed)
    case = make_case(ctx, q_len=q_len, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim,
                     block_size=block_size, seed=seed, kv_bf16=kv == "bf16", kv_f16=kv == "f16")
    n = len(case.token_pos)
    qd, kvd = q_heads * head_dim, kv_heads * head_dim
    tdt = TORCH_DT[act]
    qkv = torch.from_numpy(rng.standard_normal((n, qd + 2 * kvd + stride_pad), dtype=np.float32)).to(gpu).to(tdt)
    b = torch.from_numpy(rng.standard_normal(qd + 2 * kvd, dtype=np.float32)).to(gpu) if bias else None
    cos_t, sin_t = (torch.from_numpy(t).to(gpu) for t in oracle.rope_tables(head_dim, max_pos, theta))
    kw = {} if partition_tokens is None else {"partition_tokens": partition_tokens}
    kc0 = to_dev_cache(case.k_cache, gpu)
    plan = kernels.Plan(slices_of(case), q_heads, kv_heads, head_dim, block_size, kc0.dtype, **kw).upload()

    # separately: bias + RoPE + store, then attention
    kc1, vc1 = kc0.clone(), to_dev_cache(case.v_cache, gpu)
    q = kernels.rope_store_kv(qkv, plan.dev_array("positions"), plan.dev_array("slots"), cos_t, sin_t,
                              q_heads, kv_heads, head_dim, kc1.view(-1, kvd), vc1.view(-1, kvd), bias=b)
    want = kernels.ragged_paged_attention(q, kc1, vc1, plan, case.scale)
    # one call
    kc2, vc2 = kc0.clone(), to_dev_cache(case.v_cache, gpu)
    got = kernels.ragged_paged_attention_qkv(qkv, b, cos_t, sin_t, kc2, vc2, plan, case.scale)
    torch.cuda.synchronize()
    fused = plan.plan.n_tokens == plan.plan.n_seqs and plan.plan.n_chunk_items == 0
    print(f"qkv attention act={act} kv={kv} bias={bias} rows={n} "
          f"in-launch={fused} parts={plan.plan.n_parts}")
    bits = (lambda t: t.cpu().view(torch.int16)) if act != "f32" else (lambda t: t.cpu().view(torch.int32))
    assert torch.equal(bits(got), bits(want)), f"output differs: max|diff| {max_abs(got.float().cpu(), want.float().cpu())}"
    cbits = (lambda t: t.cpu().view(torch.int16)) if kv != "f32" else (lambda t: t.cpu().view(torch.int32))
    assert torch.equal(cbits(kc2), cbits(kc1)), "k cache differs"
    assert torch.equal(cbits(vc2), cbits(vc1)), "v cache differs"
    return case, q, got, kc2, vc2


@pytest.mark.parametrize("act,kv", [("f32", "f32"), ("f32", "bf16"), ("bf16", "bf16"), ("bf16", "f32"),
                                    ("f16", "f16"), ("f32", "f16")])
@pytest.mark.parametrize("bias", [False, True])
def test_qkv_decode_step(gpu, act, kv, bias):
    """Decode rows only (the in-launch path), split and unsplit rows
    (partition 256), Qwen2.5-0.5B's shape with and without its qkv bias."""
    _run(gpu, act=act, kv=kv, bias=bias, ctx=[1, 17, 300, 1500, 64, 2049, 4096],
         partition_tokens=256, seed=61)


@pytest.mark.parametrize("act,kv", [("bf16", "f32"), ("bf16", "bf16"), ("f16", "f16")])
def test_qkv_mixed_step(gpu, act, kv):
    """A prefill chunk among decode rows: the scratch-q path (chunk tiles with
    a bf16 cache, per-row decode with fp32)."""
    _run(gpu, act=act, kv=kv, bias=True, ctx=[600, 33, 1200, 5], q_len=[70, 1, 1, 5], seed=62)


def test_qkv_shapes_and_edges(gpu):
    """head_dim 128 with 8-key blocks, TinyLlama's 32/4 x 64 with 32-key
    blocks, a padded row stride, and positions past the RoPE tables (q = 0,
    nothing stored) on the in-launch path."""
    _run(gpu, act="bf16", kv="bf16", bias=False, ctx=[9, 700, 2500], q_heads=8, kv_heads=1,
         head_dim=128, block_size=8, seed=63, theta=1e4)
    _run(gpu, act="f32", kv="bf16", bias=True, ctx=[40, 1000, 3000, 1], q_heads=32, kv_heads=4,
         block_size=32, stride_pad=8, seed=64)
    _run(gpu, act="f32", kv="f32", bias=True, ctx=[100, 1500, 2100, 3000], max_pos=2048,
         partition_tokens=512, seed=65)


def test_qkv_decode_against_oracle(gpu):
    """The in-launch path against the oracle end to end: the oracle attends
    with the q the separate RoPE produced over the caches as stored (fp32
    throughout, tolerance 1e-3 max-abs as for the attention kernels)."""
    case, q, got, kc, vc = _run(gpu, act="f32", kv="f32", bias=True, ctx=[5, 333, 2048, 4000], seed=66)
    case.k_cache, case.v_cache = kc.cpu().numpy(), vc.cpu().numpy()
    err = max_abs(got.cpu().numpy(), oracle_out(case, q.cpu().numpy()))
    print(f"qkv attention vs oracle: max|err| {err:.3e}")
    assert err < 1e-3


@pytest.mark.parametrize("act", ["f32", "bf16"])
@pytest.mark.parametrize("mixed", [False, True])
@pytest.mark.parametrize("shape", [(896, 64, True), (5120, 128, False)],
                         ids=["h896-hd64-kvbf16", "h5120-hd128-kvf32"])
def test_qkv_rms_folded_norm(gpu, act, mixed, shape):
    """le_ragged_paged_attention_qkv_rms: the rows are the projection of the
    un-normalised residual stream x, and each row is scaled by
    r = 1/sqrt(mean(x^2) + eps) before its bias, on the in-launch decode path
    and on the rope/store path of a mixed step. Against the plain entry point
    on rows scaled by r on the host: with fp32 rows the two differ only by
    r's last bit; with bf16 rows by the one rounding the folded path saves
    (the host's scaled rows are rounded before the bias is added). Hidden
    5120 is longer than the decode kernel holds in registers while its row
    loads are in flight (4096 bf16 or 2048 fp32 elements): its other path."""
    from llm_engine_amd import kernels
    rng = np.random.default_rng(71 + mixed)
    hidden, head_dim, kv_bf16 = shape
    q_heads, kv_heads, eps = 14, 2, 1e-6
    ctx, q_len = ([600, 33, 1200, 5], [70, 1, 1, 5]) if mixed else ([1, 17, 300, 1500, 64, 2049], None)
    case = make_case(ctx, q_len=q_len, q_heads=q_heads, kv_heads=kv_heads, head_dim=head_dim, seed=71,
                     kv_bf16=kv_bf16)
    n = len(case.token_pos)
    qd, kvd = q_heads * head_dim, kv_heads * head_dim
    tdt = TORCH_DT[act]
    x = torch.from_numpy(rng.standard_normal((n, hidden), dtype=np.float32) * 3).to(tdt)
    xf = x.float().numpy().astype(np.float64)
    r = (1.0 / np.sqrt((xf * xf).mean(axis=1) + eps)).astype(np.float32)
    raw = torch.from_numpy(rng.standard_normal((n, qd + 2 * kvd), dtype=np.float32)).to(tdt)
    b = torch.from_numpy(rng.standard_normal(qd + 2 * kvd, dtype=np.float32)).to(gpu)
    cos_t, sin_t = (torch.from_numpy(t).to(gpu) for t in oracle.rope_tables(head_dim, 4096, 1e6))
    kc0 = to_dev_cache(case.k_cache, gpu)
    plan = kernels.Plan(slices_of(case), q_heads, kv_heads, head_dim, 16, kc0.dtype).upload()
    kc1, vc1 = kc0.clone(), to_dev_cache(case.v_cache, gpu)
    got = kernels.ragged_paged_attention_qkv(raw.to(gpu), b, cos_t, sin_t, kc1, vc1, plan, case.scale,
                                             rms_x=x.to(gpu), rms_eps=eps)
    kc2, vc2 = kc0.clone(), to_dev_cache(case.v_cache, gpu)
    scaled = (raw.float() * torch.from_numpy(r)[:, None]).to(tdt).to(gpu)
    want = kernels.ragged_paged_attention_qkv(scaled, b, cos_t, sin_t, kc2, vc2, plan, case.scale)
    torch.cuda.synchronize()
    fused = plan.plan.n_tokens == plan.plan.n_seqs and plan.plan.n_chunk_items == 0
    assert fused != mixed
    g, w = got.float().cpu().numpy(), want.float().cpu().numpy()
    err = max_abs(g, w)
    kerr = max_abs(kc1.float().cpu(), kc2.float().cpu())
    verr = max_abs(vc1.float().cpu(), vc2.float().cpu())
    print(f"qkv rms act={act} mixed={mixed} shape={shape}: max|out diff| {err:.2e}, cache diffs {kerr:.2e} {verr:.2e}")
    # cache entries: one bf16 step of the largest written value at most
    vmax = float(max(kc2.float().abs().max(), vc2.float().abs().max()))
    assert kerr <= vmax * 2 ** -7 and verr <= vmax * 2 ** -7
    assert err <= (2e-3 if act == "f32" else 3e-2)
    # a row scale that is not applied would move outputs by far more
    assert float(np.abs(r - 1).max()) > 0.3
