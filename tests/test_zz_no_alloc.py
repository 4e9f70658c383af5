"""le_ragged_paged_attention_noalloc (the entry point that allocates nothing:
its workspace is a static device array) against le_ragged_paged_attention on
the same plans: bit-identical outputs, on two calls in a row, the second
with a smaller step, for a mixed bf16 step and an fp32 decode step. Called
through the C ABI (ctypes)."""
import ctypes

import numpy as np
import pytest
import torch

from cases import loguniform_ctx, make_case
from gpu_util import device_q, slices_of, to_dev_cache

pytestmark = pytest.mark.gpu


def _noalloc(q, kc, vc, plan, scale):
    from llm_engine_amd import _lib
    from llm_engine_amd.kernels import _dt, _p, _stream
    out = torch.full_like(q, float("nan"))
    cfg = plan.plan.cfg
    num_blocks = kc.numel() // (cfg.block_size * cfg.kv_heads * cfg.head_dim)
    st = _lib.load().le_ragged_paged_attention_noalloc(
        _p(q), _dt(q), _p(kc), _p(vc), _dt(kc), num_blocks, ctypes.byref(plan.plan), float(scale), _p(out),
        _stream(None))
    _lib.check("le_ragged_paged_attention_noalloc", st)
    return out


def _case_pair(kind):
    if kind == "mixed_bf16":
        rng = np.random.default_rng(3)
        big = make_case(list(rng.integers(256, 2049, 32)) + [512, 1536], q_len=[1] * 32 + [512, 512],
                        num_blocks=16384, seed=3, kv_bf16=True)
        small = make_case([700, 90, 2000], q_len=[1, 40, 1], num_blocks=1024, seed=4, kv_bf16=True)
    else:
        rng = np.random.default_rng(2)
        big = make_case(loguniform_ctx(rng, 64, 64, 4096), num_blocks=32768, seed=2)
        small = make_case([1, 3000, 17], num_blocks=512, seed=5)
    return big, small


@pytest.mark.parametrize("kind", ["mixed_bf16", "decode_f32"])
def test_noalloc_equals_workspace_entry(gpu, kind):
    from llm_engine_amd import kernels
    for case in _case_pair(kind):  # the second call's step is smaller
        q, _ = device_q(case, torch.float32, gpu)
        kc, vc = to_dev_cache(case.k_cache, gpu), to_dev_cache(case.v_cache, gpu)
        plan = kernels.Plan(slices_of(case), case.q_heads, case.kv_heads, case.head_dim, case.block_size,
                            kc.dtype, partition_tokens=256, chunk_partition_tokens=256).upload()
        assert plan.plan.n_parts > 0  # split rows: the scratch holds partials and counters
        want = kernels.ragged_paged_attention(q, kc, vc, plan, case.scale)
        got = _noalloc(q, kc, vc, plan, case.scale)
        again = _noalloc(q, kc, vc, plan, case.scale)
        torch.cuda.synchronize()
        print(f"{kind}: rows {plan.plan.n_tokens} parts {plan.plan.n_parts} "
              f"workspace {plan.workspace_size()} bytes")
        assert torch.equal(got.view(torch.int32), want.view(torch.int32))
        assert torch.equal(again.view(torch.int32), want.view(torch.int32))
