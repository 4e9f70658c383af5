"""The 16-bit attention kernels' error, stated without a GPU: the host
emulation of their roundings (tests/precision.py: q, or in the chunk tile
q * scale * log2(e), and the softmax weights rounded to the cache type before
the MFMA) on configs 2 and 3, against the
fp32 oracle. The GPU parity tests hold each 16-bit case to twice its own
emulated error (gpu_util.emulated_bar); here the emulated errors of the
benchmark configs are stated and kept under half the north star's 2e-2, so
those bars stay inside it."""
import numpy as np
import pytest

from cases import loguniform_ctx, make_case
from gpu_util import oracle_out
from precision import emulate

NORTH_STAR = 2e-2  # max-abs bound for 16-bit K/V
# the emulated max-abs error, decode rows and prefill-chunk rows, within 20 %
STATED = {"config2": {"bf16": 1.66e-3, "f16": 2.29e-4},
          "config3": {"bf16": (1.12e-3, 5.79e-3), "f16": (1.27e-4, 8.74e-4)}}


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_config2_emulated_error_under_half_the_bar(dt):
    rng = np.random.default_rng(2)
    case = make_case(loguniform_ctx(rng, 64, 64, 4096), num_blocks=32768, seed=2, kv_bf16=dt == "bf16",
                     kv_f16=dt == "f16")
    err = float(np.abs(emulate(case, case.q, dt) - oracle_out(case, case.q)).max())
    print(f"config2 {dt}: emulated max|err| {err:.3e}")
    assert 2 * err < NORTH_STAR
    assert abs(err / STATED["config2"][dt] - 1) < 0.2


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_config3_emulated_error_under_half_the_bar(dt):
    rng = np.random.default_rng(3)
    case = make_case(list(rng.integers(256, 2049, 32)) + [512, 1536], q_len=[1] * 32 + [512, 512],
                     num_blocks=16384, seed=3, kv_bf16=dt == "bf16", kv_f16=dt == "f16")
    chunk = np.array([case.seq_qlen[s] > 1 for s in case.token_seq])
    e = np.abs(emulate(case, case.q, dt, chunk) - oracle_out(case, case.q))
    print(f"config3 {dt}: emulated max|err| decode rows {e[~chunk].max():.3e}, chunk rows {e[chunk].max():.3e}")
    assert 2 * e.max() < NORTH_STAR
    d, c = STATED["config3"][dt]
    assert abs(e[~chunk].max() / d - 1) < 0.2 and abs(e[chunk].max() / c - 1) < 0.2


def test_error_attribution_bf16():
    """Which rounding costs what (config 3, bf16): q alone and the softmax
    weights alone, each a sizeable share of the total."""
    rng = np.random.default_rng(3)
    case = make_case(list(rng.integers(256, 2049, 32)) + [512, 1536], q_len=[1] * 32 + [512, 512],
                     num_blocks=16384, seed=3, kv_bf16=True)
    chunk = np.array([case.seq_qlen[s] > 1 for s in case.token_seq])
    want = oracle_out(case, case.q)
    only_q = float(np.abs(emulate(case, case.q, "bf16", chunk, round_p=False) - want).max())
    only_p = float(np.abs(emulate(case, case.q, "bf16", chunk, round_q=False) - want).max())
    both = float(np.abs(emulate(case, case.q, "bf16", chunk) - want).max())
    print(f"config3 bf16: q only {only_q:.3e}, weights only {only_p:.3e}, both {both:.3e}")
    assert only_q > 0.2 * both and only_p > 0.2 * both
