"""The oracle's whole forward (oracle.c:orc_forward, restating
cpu_model.cpp:98-214) against Hugging Face's Qwen2 and Llama in fp32.

tests/golden/forward_ref.npz holds, per prompt, the residual stream after
the embedding and after every layer, the last position's logits and the
greedy continuation, written by tests/golden/make_forward_ref.py from
transformers' own model classes on the weights of
tests/golden/forward_models.py. The bars are the reference's
(test_cpu_model.cpp:112-129): per layer max|diff| <= 2e-3 * max(1, max|ref|),
logits max|diff| < 1e-2, and the argmax of the last position equal; and
the greedy continuation through the scheduler (test_cpu_model.cpp:152-176)
equal to HF's, up to the first step whose HF top-2 margin is <= 1e-3.

The oracle runs each prompt through a fragmented block table (a random
permutation of a 96-block pool, block 16), so the paging is part of what is
checked. The last tests show the check has teeth: the same comparison fails
when the oracle is fed the plausible mistakes (the two norms of a layer
swapped, the q/k/v biases dropped or on q alone, gate and up swapped, the
head tied or untied wrongly, the RoPE theta or the norm eps wrong).
"""
import ctypes
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "golden"))
import forward_models as fm  # noqa: E402

REF = np.load(ROOT / "golden" / "forward_ref.npz")
POOL = 96
BS = 16


def _slice(key, ids, blocks):
    from llm_engine_amd._lib import StepSlice
    b = np.ascontiguousarray(blocks, np.int32)
    t = np.ascontiguousarray(ids, np.int32)
    s = StepSlice(key, 0, len(ids), 1, len(b), b.ctypes.data, t.ctypes.data)
    s._keep = (b, t)
    return s


def _run_prompt(w, ids, seed):
    """One prefill step of the whole prompt through a fragmented table."""
    from e2e_util import OracleModel
    m = OracleModel(w, POOL, BS, threads=2)
    rng = np.random.default_rng(seed)
    nb = (len(ids) + BS - 1) // BS
    blocks = rng.permutation(POOL)[:nb]
    logits, resid = m.trace([_slice(7, ids, blocks)])
    return logits[0], resid


def _compare(w, name, pi):
    logits, resid = _run_prompt(w, REF[f"{name}.p{pi}.ids"], seed=pi)
    want = REF[f"{name}.p{pi}.resid"]
    assert resid.shape == want.shape
    worst = 0.0
    for l in range(want.shape[0]):
        d = float(np.max(np.abs(resid[l] - want[l])))
        bar = 2e-3 * max(1.0, float(np.max(np.abs(want[l]))))
        worst = max(worst, d / bar)
    dl = float(np.max(np.abs(logits - REF[f"{name}.p{pi}.logits"])))
    return worst, dl, logits


@pytest.mark.parametrize("name", list(fm.ARCHS))
@pytest.mark.parametrize("pi", range(len(fm.PROMPT_LENS)))
def test_forward_matches_hf(name, pi):
    w = fm.weights(name)
    worst, dl, logits = _compare(w, name, pi)
    assert worst <= 1.0, f"residual off by {worst:.3g}x the bar"
    assert dl < 1e-2, dl
    # Both restate the same fp32 arithmetic, so the measured agreement is far
    # inside the reference's bars (worst residual 0.07 % of the bar, logits
    # 4e-6); the tight bars catch mistakes too small for the reference's.
    assert worst <= 0.02, worst
    assert dl < 5e-5, dl
    import oracle
    assert oracle.argmax(logits) == int(REF[f"{name}.p{pi}.gen"][0])


@pytest.mark.parametrize("name", list(fm.ARCHS))
def test_greedy_through_scheduler_matches_hf(name):
    """All prompts at once, prefill chunks of 16 tokens, a fragmented pool:
    the oracle's greedy tokens equal HF generate's."""
    from e2e_util import OracleModel
    from llm_engine_amd.engine import greedy_loop, sched_config
    w = fm.weights(name)
    prompts = [REF[f"{name}.p{i}.ids"].tolist() for i in range(len(fm.PROMPT_LENS))]
    m = OracleModel(w, POOL, BS, threads=2)
    got = greedy_loop(m.forward, prompts, [fm.GEN_TOKENS] * len(prompts), POOL, BS,
                      sched_config(prefill_chunk_size=16), fragment_blocks=12)
    checked = 0
    for i, g in enumerate(got):
        want = REF[f"{name}.p{i}.gen"]
        margin = REF[f"{name}.p{i}.margin"]
        for j, tok in enumerate(want):
            assert g[j] == int(tok), (i, j, g, want)
            checked += 1
            if margin[j] <= 1e-3:
                break
    assert checked >= len(prompts) * fm.GEN_TOKENS // 2


def _mutated(name, how):
    w = fm.weights(name)
    for L in w.layers:
        if how == "swap_norms":
            L["in_norm"], L["post_norm"] = L["post_norm"], L["in_norm"]
        elif how == "drop_bias":
            for k in ("bq", "bk", "bv"):
                L[k] = np.zeros_like(L[k])
        elif how == "bias_on_q_only":
            L["bk"] = np.zeros_like(L["bk"])
        elif how == "gate_up_swapped":
            L["wgate"], L["wup"] = L["wup"], L["wgate"]
    if how == "tie_head":
        w.arch = dict(w.arch, tie=True)
    if how == "theta_1e4":
        w.arch = dict(w.arch, theta=1e4)
    if how == "eps_1e-2":
        w.arch = dict(w.arch, eps=1e-2)
    if how == "untie_with_embed_t":
        w.arch = dict(w.arch, tie=False)
        w.lm_head = np.ascontiguousarray(np.roll(w.embed, 1, axis=0))
    return w


@pytest.mark.parametrize("name,how", [("qwen2_tiny", "swap_norms"), ("llama_tiny", "swap_norms"),
                                      ("qwen2_tiny", "drop_bias"), ("qwen2_tiny", "bias_on_q_only"),
                                      ("llama_tiny", "tie_head"),
                                      ("qwen2_tiny", "untie_with_embed_t"),
                                      ("llama_tiny", "gate_up_swapped"), ("qwen2_tiny", "theta_1e4"),
                                      ("llama_tiny", "eps_1e-2")])
def test_comparison_catches_plausible_mistakes(name, how):
    w = _mutated(name, how)
    pi = 3
    worst, dl, _ = _compare(w, name, pi)
    assert worst > 1.0 or dl >= 1e-2, (how, worst, dl)
