"""The layer ops behind the reference's small launchers (le_embedding,
le_rmsnorm, le_silu_mul, le_rope, le_add_inplace, le_add_bias; the
kernels of cuda_kernels.h:17-40) on the GPU, for fp32, bf16 and fp16
elements, against the oracle's ops (ops.h) on the values the device holds.

Bit-exact: embedding, residual add, bias add and RoPE (each one fp32
operation, or a*c - b*s without contraction, then one rounding). RMSNorm and
SiLU: within the output type's rounding (2^-24 fp32, 2^-8 bf16, 2^-11 fp16,
relative; 2^-25 absolute for fp16 subnormals) plus 1e-6 relative for the different order of the sum of squares
and expf's last bits. Ragged shapes (odd column counts, n not a multiple of 8)
take the scalar paths, the others the 16-byte paths."""
import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DT = {"f32": (0, torch.float32, 2.0 ** -24), "bf16": (1, torch.bfloat16, 2.0 ** -8),
      "f16": (2, torch.float16, 2.0 ** -11)}


def L():
    from llm_engine_amd import _lib
    return _lib.load()


def p(t):
    return ctypes.c_void_p(t.data_ptr())


def stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def held(x: np.ndarray, dt: str, dev):
    """Device tensor of x in dt, and the fp32 values it holds."""
    t = torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(dev).to(DT[dt][1])
    return t, t.float().cpu().numpy()


def as_f32(t):
    return t.float().cpu().numpy()


def rounded(x: np.ndarray, dt: str) -> np.ndarray:
    """fp32 values rounded to dt by the oracle's rules (tensor.h:20-56)."""
    if dt == "bf16":
        return oracle.bf16_to_f32(oracle.f32_to_bf16(x))
    if dt == "f16":
        return oracle.f32_to_f16(x).astype(np.float32)
    return np.asarray(x, np.float32)


def within_rounding(got, want, dt):
    # relative rounding, plus half of fp16's smallest subnormal step
    bar = np.abs(want) * (DT[dt][2] + 1e-6) + (2.0 ** -25 if dt == "f16" else 1e-38)
    worst = float(np.max(np.abs(got.astype(np.float64) - want) / bar))
    assert worst <= 1.0, worst
    return worst


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("hidden", [896, 67])
def test_embedding(gpu, dt, hidden):
    rng = np.random.default_rng(1)
    table, table_h = held(rng.standard_normal((300, hidden)), dt, gpu)
    ids = rng.integers(0, 300, 77).astype(np.int32)
    out = torch.empty((77, hidden), dtype=DT[dt][1], device=gpu)
    assert L().le_embedding(p(table), DT[dt][0], p(torch.from_numpy(ids).to(gpu)), p(out), 77, hidden, stream()) == 0
    assert np.array_equal(as_f32(out), table_h[ids])


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("rows,cols", [(64, 896), (5, 2048), (3, 131)])
def test_rmsnorm(gpu, dt, rows, cols):
    rng = np.random.default_rng(2)
    x, xh = held(rng.standard_normal((rows, cols)) * 3, dt, gpu)
    w = (1 + 0.1 * rng.standard_normal(cols)).astype(np.float32)
    out = torch.empty_like(x)
    assert L().le_rmsnorm(p(x), DT[dt][0], p(torch.from_numpy(w).to(gpu)), p(out), rows, cols,
                          ctypes.c_float(1e-6), stream()) == 0
    want = oracle.rmsnorm(xh, w, 1e-6)
    print(f"rmsnorm {dt} {rows}x{cols}: {within_rounding(as_f32(out), want, dt):.3f} of the bar")


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("n", [64 * 4864, 1001])
def test_silu_mul(gpu, dt, n):
    rng = np.random.default_rng(3)
    g, gh = held(rng.standard_normal(n) * 2, dt, gpu)
    u, uh = held(rng.standard_normal(n), dt, gpu)
    assert L().le_silu_mul(p(g), p(u), DT[dt][0], n, stream()) == 0
    want = gh.copy()
    oracle.lib().orc_silu_mul(oracle.ptr(want), oracle.ptr(np.ascontiguousarray(uh)), n)
    print(f"silu {dt} n={n}: {within_rounding(as_f32(g), want, dt):.3f} of the bar")


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("n", [64 * 896, 1003])
def test_add_inplace(gpu, dt, n):
    rng = np.random.default_rng(4)
    x, xh = held(rng.standard_normal(n), dt, gpu)
    y, yh = held(rng.standard_normal(n), dt, gpu)
    assert L().le_add_inplace(p(x), p(y), DT[dt][0], n, stream()) == 0
    assert np.array_equal(as_f32(x), rounded(xh + yh, dt))


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("rows,cols", [(64, 1152), (7, 131)])
def test_add_bias(gpu, dt, rows, cols):
    rng = np.random.default_rng(5)
    x, xh = held(rng.standard_normal((rows, cols)), dt, gpu)
    b = rng.standard_normal(cols).astype(np.float32)
    assert L().le_add_bias(p(x), DT[dt][0], p(torch.from_numpy(b).to(gpu)), rows, cols, stream()) == 0
    assert np.array_equal(as_f32(x), rounded(xh + b[None, :], dt))


@pytest.mark.parametrize("dt", list(DT))
@pytest.mark.parametrize("heads,hd,stride", [(14, 64, 14 * 64), (2, 64, 1152), (4, 128, 4 * 128)])
def test_rope(gpu, dt, heads, hd, stride):
    """In place on the first `heads` heads of each row; the rest of the row
    (the k and v parts of a stacked row) is untouched. A token past the
    tables' end is left unchanged when max_pos bounds them."""
    rng = np.random.default_rng(6)
    n, max_pos = 50, 4096
    x, xh = held(rng.standard_normal((n, stride)), dt, gpu)
    pos = rng.integers(0, max_pos, n).astype(np.int32)
    pos[7] = max_pos + 3
    cos_t, sin_t = oracle.rope_tables(hd, max_pos, 1e6)
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(gpu)  # noqa: E731
    assert L().le_rope(p(x), DT[dt][0], p(dev(pos)), p(dev(cos_t)), p(dev(sin_t)), max_pos, n, heads, hd,
                       stride, stream()) == 0
    want = xh.copy()
    for t in range(n):
        if pos[t] < max_pos:
            row = np.ascontiguousarray(want[t])
            oracle.lib().orc_rope_inplace(oracle.ptr(row), heads, hd, int(pos[t]), oracle.ptr(cos_t), oracle.ptr(sin_t))
            want[t] = rounded(row, dt)
    assert np.array_equal(as_f32(x), want)


def test_rejected_arguments(gpu):
    nul = ctypes.c_void_p(0)
    assert L().le_rmsnorm(nul, 7, nul, nul, 1, 1, ctypes.c_float(1e-6), nul) < 0  # bad dtype
    assert L().le_rope(nul, 0, nul, nul, nul, 0, 1, 1, 63, 63, nul) < 0           # odd head_dim
    assert L().le_embedding(nul, 0, nul, nul, 0, 8, nul) == 0                      # nothing to do
    assert L().le_add_bias(nul, 0, nul, 3, 8, nul) < 0                            # null pointers
