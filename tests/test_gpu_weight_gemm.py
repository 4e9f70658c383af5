"""GPU numerics of le_weight_gemm (the decode-step projections) against a
plain PyTorch fp32 reference on the same bf16 operands.

Bar: |got - ref| <= 2^-8 |ref| + 2^-16 (|x| . |w|^T) per element. The first
term is the output's own bf16 rounding (2^-9 relative, doubled); the second
bounds fp32 accumulation in another order (k <= 5632 terms, each product
exact in fp32, 2^-24 per addition; 2^-16 leaves a margin of 2^8 over
k * 2^-24). For fp32 outputs only the second term applies. The SiLU epilogue
is compared with silu(round_bf16(g)) * round_bf16(u) from the fp32 products;
a product within one bf16 step of a rounding boundary may round the other
way, so that bar is 2^-6 relative."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

# (k, n, silu): TinyLlama-1.1B and Qwen2.5-0.5B projections (qkv, o, gate|up, down, lm head)
SHAPES = [(2048, 2560, False), (2048, 2048, False), (2048, 11264, True), (5632, 2048, False),
          (896, 1152, False), (896, 896, False), (896, 9728, True), (4864, 896, False)]


def _ops(m, k, n, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(m, k, generator=g).to(torch.bfloat16)
    w = (torch.randn(n, k, generator=g) * 0.02).to(torch.bfloat16)
    return x, w


def _ref(x, w):
    xf, wf = x.float(), w.float()
    return xf @ wf.t(), xf.abs() @ wf.abs().t()


@pytest.mark.parametrize("k,n,silu", SHAPES)
@pytest.mark.parametrize("m", [1, 7, 16, 33, 64])
def test_weight_gemm_matches_fp32(gpu, m, k, n, silu):
    from llm_engine_amd import kernels
    x, w = _ops(m, k, n, seed=m * 7919 + n)
    ref, mag = _ref(x, w)
    got = kernels.weight_gemm(x.to(gpu), w.to(gpu), silu=silu).float().cpu()
    if silu:
        I = n // 2
        rb = lambda t: t.to(torch.bfloat16).float()
        gg, uu = rb(ref[:, :I]), rb(ref[:, I:])
        want = gg / (1.0 + torch.exp(-gg)) * uu
        bar = 2.0 ** -6 * want.abs() + 2.0 ** -16 * (mag[:, :I] + mag[:, I:])
    else:
        want = ref
        bar = 2.0 ** -8 * want.abs() + 2.0 ** -16 * mag
    err = (got - want).abs()
    print(f"m={m} k={k} n={n} silu={silu}: max|err| {err.max().item():.3e}, max err/bar "
          f"{(err / bar).max().item():.3f}")
    assert bool((err <= bar).all())


@pytest.mark.parametrize("m", [1, 64])
def test_weight_gemm_fp32_logits(gpu, m):
    """The lm head writes fp32 logits (TinyLlama vocab 32000)."""
    from llm_engine_amd import kernels
    x, w = _ops(m, 2048, 32000, seed=5 + m)
    ref, mag = _ref(x, w)
    got = kernels.weight_gemm(x.to(gpu), w.to(gpu), out_dtype=torch.float32).cpu()
    err = (got - ref).abs()
    print(f"lm head m={m}: max|err| {err.max().item():.3e}")
    assert bool((err <= 2.0 ** -16 * mag).all())


def test_weight_gemm_split_is_deterministic_and_leaves_counters_zero(gpu):
    """Split-k partials are summed in split order: two runs are bit-identical,
    and the shared workspace's counters are back at zero after each."""
    from llm_engine_amd import kernels
    x, w = _ops(64, 5632, 2048, seed=11)
    x, w = x.to(gpu), w.to(gpu)
    need = kernels.weight_gemm_workspace_size(64, 5632, 2048)
    assert need > 0  # this shape splits k
    ws = torch.zeros(need, dtype=torch.uint8, device=gpu)
    a = kernels.weight_gemm(x, w, workspace=ws)
    b = kernels.weight_gemm(x, w, workspace=ws)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
    assert int(ws[:256].count_nonzero().item()) == 0  # the 32 block counters


def test_weight_gemm_rejects_unsupported_shapes(gpu):
    from llm_engine_amd import kernels
    from llm_engine_amd._lib import LeError
    x, w = _ops(65, 256, 64, seed=1)
    with pytest.raises(LeError):
        kernels.weight_gemm(x.to(gpu), w.to(gpu))        # m > 64
    x, w = _ops(8, 200, 64, seed=1)
    with pytest.raises(LeError):
        kernels.weight_gemm(x.to(gpu), w.to(gpu))        # k % 128 != 0
