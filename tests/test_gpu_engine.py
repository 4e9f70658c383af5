"""End-to-end parity on the GPU: the device model (GEMMs + this path's kernels)
driven by the scheduler against the CPU oracle model, token for token on the
fp32 path. Mirrors the reference's CUDA parity cases
(test_cuda_model.cpp:116-235, test_cuda_invariance.cpp:156-344): greedy equality,
a fragmented pool, several sequences in one fragmented pool (table_offset),
chunked prefill, preemption with recompute, prefix caching, a second
architecture (GQA group 8, untied head, no qkv bias)."""
import json
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLD = Path(__file__).resolve().parent / "golden"


def qwen_small(layers=2, seed=7):
    from llm_engine_amd.engine import synthetic_weights
    return synthetic_weights("qwen2.5-0.5b", seed, layers=layers)


def prompts_of(seed, lens, vocab):
    rng = np.random.default_rng(seed)
    return [rng.integers(0, vocab, n).astype(np.int32).tolist() for n in lens]


def run_both(w, prompts, max_tokens, num_blocks, cfg=None, prefix=False, frag=0, kv="f32"):
    from e2e_util import OracleModel
    from llm_engine_amd.engine import Model, greedy_loop
    m = Model(w, num_blocks, 16, dtype="f32", kv_dtype=kv)
    gpu, stats = m.run_greedy(prompts, max_tokens, cfg, prefix, frag)
    m.close()
    o = OracleModel(w, num_blocks, kv_bf16=(kv == "bf16"))
    cpu = greedy_loop(o.forward, prompts, max_tokens, num_blocks, 16, cfg, prefix, frag)
    return gpu, cpu, stats


def test_config1_matches_oracle_token_for_token(gpu):
    """Qwen2.5-0.5B (24 layers) random-init fp32, 8 prompts of
    16..512 tokens, 32 greedy tokens, fragmented 4096-block pool."""
    from llm_engine_amd.engine import Model, sched_config, synthetic_weights
    import sys
    sys.path.insert(0, str(GOLD))
    from make_config1 import weight_digest
    fx = json.loads((GOLD / "config1_tokens.json").read_text())
    w = synthetic_weights(fx["arch"], fx["weight_seed"])
    assert weight_digest(w) == fx["weight_digest"], "weight generator changed; regenerate the fixture"
    m = Model(w, fx["num_blocks"], 16, dtype="f32")
    toks, stats = m.run_greedy(fx["prompts"], [fx["gen"]] * len(fx["prompts"]),
                               sched_config(max_num_batched_tokens=fx["max_num_batched_tokens"]),
                               fragment_blocks=fx["fragment_blocks"])
    m.close()
    print(f"config1: {stats.steps} steps, {stats.decode_tokens} tokens in {stats.seconds:.2f}s; "
          f"oracle min top-2 margins {fx['min_margin']}")
    assert toks == fx["tokens"]


@pytest.mark.parametrize("case", ["fragmented_multi", "chunked16", "preempt", "prefix"])
def test_small_model_matches_oracle(gpu, case):
    from llm_engine_amd.engine import sched_config
    w = qwen_small()
    V = w.arch["vocab"]
    if case == "fragmented_multi":
        prompts = prompts_of(1, (20, 150, 300, 47), V)
        gpu_t, cpu_t, _ = run_both(w, prompts, [8] * 4, 256, frag=40)
    elif case == "chunked16":
        prompts = prompts_of(2, (40, 200, 90), V)
        gpu_t, cpu_t, _ = run_both(w, prompts, [6] * 3, 256, sched_config(prefill_chunk_size=16))
    elif case == "preempt":
        prompts = prompts_of(3, (30, 120, 64, 99, 40, 75, 110, 33), V)
        gpu_t, cpu_t, st = run_both(w, prompts, [24] * 8, 48, sched_config(max_num_seqs=8))
        print(f"preemptions: {st.preemptions}")
        assert st.preemptions > 0
    else:
        base = prompts_of(4, (20, 37, 50, 9), V)
        prompts = [[1234] * 96 + p for p in base]
        gpu_t, cpu_t, _ = run_both(w, prompts, [8] * 4, 256, prefix=True)
        off, _, _ = run_both(w, prompts, [8] * 4, 256, prefix=False)
        assert off == gpu_t
    assert gpu_t == cpu_t


def test_second_architecture_group8(gpu):
    """TinyLlama-1.1B shape (GQA 32/4 = 8, untied head, no qkv bias), 2 layers."""
    from llm_engine_amd.engine import synthetic_weights
    w = synthetic_weights("tinyllama-1.1b", 11, layers=2)
    prompts = prompts_of(5, (33, 180, 64), w.arch["vocab"])
    gpu_t, cpu_t, _ = run_both(w, prompts, [8] * 3, 256, frag=40)
    assert gpu_t == cpu_t


def test_bf16_kv_cache_matches_bf16_oracle(gpu):
    """fp32 model with a bf16 K/V cache against the oracle storing K/V as bf16
    (same rounding); attention runs on MFMA with bf16 operands here, so equality
    is expected except at near ties, which the margins show."""
    w = qwen_small(seed=9)
    prompts = prompts_of(6, (60, 200, 17), w.arch["vocab"])
    gpu_t, cpu_t, _ = run_both(w, prompts, [8] * 3, 256, kv="bf16")
    agree = sum(a == b for g, c in zip(gpu_t, cpu_t) for a, b in zip(g, c))
    total = sum(len(c) for c in cpu_t)
    print(f"bf16 KV: {agree}/{total} tokens agree")
    assert gpu_t[0][0] == cpu_t[0][0]
    assert agree >= 0.9 * total


def test_first_step_logits_close(gpu):
    """Logits of one mixed step (prefill chunk + decode rows) against the oracle:
    fp32 GEMM reordering only."""
    from e2e_util import OracleModel
    from llm_engine_amd.engine import Model, Scheduler, sched_config
    w = qwen_small(seed=3)
    prompts = prompts_of(7, (70, 20), w.arch["vocab"])
    m = Model(w, 128, 16, dtype="f32")
    o = OracleModel(w, 128)
    sch = Scheduler(128, 16, sched_config(), fragment_blocks=10)
    for i, p in enumerate(prompts):
        sch.add(i, p, 4)
    for _ in range(3):
        sl = sch.step()
        n = sum(int(s.needs_logits) for s in sl)
        toks, lg = m.forward(sl, n, want_logits=True)
        want = o.logits(sl)
        err = float(np.max(np.abs(lg - want)))
        print(f"step logits max|err| {err:.2e}, max|logit| {np.abs(want).max():.2f}")
        assert err < 1e-3
        sch.done(toks)
    m.close()


def _round_weights_bf16(w):
    """The same model with every weight rounded to bf16 (round to nearest
    even), held in fp32: what the bf16 device model computes with."""
    import oracle
    r = lambda a: oracle.bf16_to_f32(oracle.f32_to_bf16(a)).reshape(a.shape)
    w.embed = r(w.embed)
    if w.lm_head is not None:
        w.lm_head = r(w.lm_head)
    for L in w.layers:
        for k in ("wq", "wk", "wv", "wo", "wgate", "wup", "wdown"):
            L[k] = r(L[k])
    return w


@pytest.mark.parametrize("arch", ["qwen2.5-0.5b", "tinyllama-1.1b"])
def test_bf16_model_logits_close(gpu, arch):
    """bf16 weights, activations and K/V (the config-4 precision) against the
    fp32 oracle run on the same bf16-rounded weights with a bf16 K/V cache:
    the difference is the rounding of activations between ops, so the
    tolerance is relative to the logit scale: max|err| <= 5 % of max|logit|
    over three steps (mixed prefill + decode), and the greedy tokens agree
    wherever the oracle's top-2 margin exceeds twice that error."""
    from e2e_util import OracleModel, top2_margin
    from llm_engine_amd.engine import Model, Scheduler, sched_config, synthetic_weights
    w = _round_weights_bf16(synthetic_weights(arch, 21, layers=2))
    prompts = prompts_of(8, (90, 33, 260), w.arch["vocab"])
    m = Model(w, 128, 16, dtype="bf16", kv_dtype="bf16")
    o = OracleModel(w, 128, kv_bf16=True)
    sch = Scheduler(128, 16, sched_config(max_num_batched_tokens=256), fragment_blocks=12)
    for i, p in enumerate(prompts):
        sch.add(i, p, 6)
    checked = 0
    for _ in range(5):
        if not sch.has_work():
            break
        sl = sch.step()
        n = sum(int(s.needs_logits) for s in sl)
        toks, lg = m.forward(sl, n, want_logits=True)
        want = o.logits(sl)
        err = float(np.max(np.abs(lg - want))) if n else 0.0
        scale = float(np.abs(want).max()) if n else 1.0
        print(f"{arch} bf16 step: {n} rows, max|err| {err:.3e}, max|logit| {scale:.3f}")
        assert err <= 0.05 * scale
        for r in range(n):
            if top2_margin(want[r]) > 2 * err:
                assert toks[r] == int(np.argmax(want[r]))
                checked += 1
        # both models continue from the device's tokens
        sch.done(toks)
    m.close()
    print(f"{arch}: {checked} greedy tokens checked against clear oracle margins")


@pytest.mark.parametrize("kv", ["f32", "bf16"])
def test_config5_shared_prefix_preemption(gpu, kv):
    """Config 5 at a size the oracle finishes in seconds: 128 sequences share a
    512-token prefix (32 refcounted blocks, prefix caching on) plus unique
    suffixes, in a pool small enough that the scheduler preempts and
    recomputes. Qwen2.5-0.5B attention shape (14/2 x 64), 2 layers, vocab cut
    to 8192 to keep the oracle's LM head cheap. Token for token against the
    oracle driven by the same scheduler (fp32 path: exact; bf16 K/V: the
    oracle stores bf16 too, agreement >= 90 %)."""
    from llm_engine_amd.engine import ARCHS, sched_config, synthetic_weights
    arch = dict(ARCHS["qwen2.5-0.5b"], vocab=8192)
    w = synthetic_weights(arch, 31, layers=2)
    rng = np.random.default_rng(12)
    prefix = rng.integers(0, 8192, 512).tolist()
    prompts = [prefix + rng.integers(0, 8192, int(n)).tolist() for n in rng.integers(16, 129, 128)]
    cfg = sched_config(max_num_seqs=128, max_num_batched_tokens=2048)
    gpu_t, cpu_t, st = run_both(w, prompts, [24] * 128, 200, cfg, prefix=True, kv=kv)
    print(f"config5 small ({kv}): {st.steps} steps, {st.preemptions} preemptions, "
          f"{st.prompt_tokens} prompt tokens computed")
    assert st.preemptions > 0
    assert all(len(t) == 24 for t in gpu_t)
    if kv == "f32":
        assert gpu_t == cpu_t
    else:
        agree = sum(a == b for g, c in zip(gpu_t, cpu_t) for a, b in zip(g, c))
        print(f"bf16 K/V: {agree}/{24 * 128} tokens agree")
        assert agree >= 0.9 * 24 * 128
