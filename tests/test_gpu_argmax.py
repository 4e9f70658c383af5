"""Device greedy selection (le_argmax_rows) against the oracle's first-maximum
rule (oracle.c:orc_argmax, restating sampler.cpp:9-13, pinned to the compiled
reference): bit-exact token ids, including ties, NaNs and all -inf rows."""
import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _check(logits: np.ndarray):
    from llm_engine_amd import kernels
    got = kernels.argmax_rows(torch.from_numpy(logits).cuda()).cpu().numpy()
    want = np.array([oracle.argmax(r) for r in logits], dtype=np.int32)
    assert np.array_equal(got, want), (got, want)


@pytest.mark.parametrize("vocab", [32000, 151936, 1001, 7])
def test_argmax_random_rows(gpu, vocab):
    rng = np.random.default_rng(vocab)
    _check(rng.standard_normal((65, vocab), dtype=np.float32))


def test_argmax_ties_nans_and_empty_rows(gpu):
    rng = np.random.default_rng(5)
    x = rng.standard_normal((9, 32000), dtype=np.float32)
    x[0, [17, 4000, 31999]] = 50.0            # tie: lowest index wins
    x[1, :] = 1.0                             # all equal: index 0
    x[2, ::3] = np.nan                        # NaNs never win
    x[2, 30000] = 9.0
    x[3, :] = -np.inf                         # no finite value: the first element (0)
    x[4, :] = np.nan                          # nothing but NaN: 0
    x[5, 31998:] = 100.0                      # tie at the tail
    x[6, 0] = np.nan; x[6, 1] = -np.inf       # leading NaN then -inf
    x[7, 12345] = np.inf; x[7, 23456] = np.inf
    x[8, 4 * 777 + 1] = 30.0; x[8, 4 * 777 + 3] = 30.0  # tie inside one 16-byte piece
    _check(x)
