"""Host engine checks (no GPU): the C++ scheduler + block allocator reproduce
the reference's own Scheduler/KVCacheManager step for step
(tests/golden/schedule_ref.npz, written from the reference compiled from
source), through both the trace entry point and the steppable API; and the
CPU oracle model keeps the reference's invariances (batch composition and
prefill chunking do not change greedy tokens, cpu/test_cpu_model.cpp:160-316)."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

from cases import parse_trace

ROOT = Path(__file__).resolve().parent.parent
TR = np.load(ROOT / "tests" / "golden" / "schedule_ref.npz")
NAMES = sorted({k.split(".")[0] for k in TR.files})


def cfg_of(c):
    from llm_engine_amd.engine import sched_config
    nb, bs, prefix, ms, mbt, chunk, wm, frag, n, cont, look, starve = (int(v) for v in c)
    return nb, bs, prefix, frag, sched_config(max_num_seqs=ms, max_num_batched_tokens=mbt,
                                              prefill_chunk_size=chunk, watermark_blocks=wm,
                                              continuous=bool(cont), admission_lookahead=look,
                                              starvation_wait_steps=starve)


@pytest.mark.parametrize("name", NAMES)
def test_scheduler_trace_matches_reference(name):
    from llm_engine_amd import _lib
    nb, bs, prefix, frag, cfg = cfg_of(TR[f"{name}.config"])
    lens, flat, mt = TR[f"{name}.prompt_lens"], TR[f"{name}.prompts"], TR[f"{name}.max_tokens"]
    out = np.zeros(1 << 22, dtype=np.int32)
    got = _lib.load().le_sched_trace(nb, bs, prefix, ctypes.byref(cfg), frag, len(lens), lens.ctypes.data,
                                     flat.ctypes.data, mt.ctypes.data, 100000, out.ctypes.data, out.size)
    want = TR[f"{name}.trace"]
    assert got == len(want)
    assert np.array_equal(out[:got], want)


@pytest.mark.parametrize("name", NAMES)
def test_steppable_scheduler_matches_reference(name):
    """Same traces, driving le_sched_* from Python with the fake model's tokens."""
    from llm_engine_amd.engine import Scheduler
    nb, bs, prefix, frag, cfg = cfg_of(TR[f"{name}.config"])
    steps, toks = parse_trace(TR[f"{name}.trace"])
    lens, flat, mt = TR[f"{name}.prompt_lens"], TR[f"{name}.prompts"], TR[f"{name}.max_tokens"]
    sch = Scheduler(nb, bs, cfg, bool(prefix), frag)
    o = 0
    for i, l in enumerate(lens):
        sch.add(i, flat[o:o + l], int(mt[i]))
        o += l
    nxt = 1000
    for want in steps:
        sl = sch.step()
        got = [(s.seq_key, s.start, s.len, s.needs_logits) for s in sl]
        assert got == [(w[0], w[1], w[2], w[3]) for w in want]
        for s, w in zip(sl, want):
            blocks = np.ctypeslib.as_array(ctypes.cast(s.blocks, ctypes.POINTER(ctypes.c_int32)), (s.num_blocks,))
            assert np.array_equal(blocks, w[5])
        n = sum(w[3] for w in want)
        sch.done(np.arange(nxt, nxt + n, dtype=np.int32))
        nxt += n
    assert not sch.has_work()
    for i, t in enumerate(toks):
        assert sch.generated(i) == t[int(lens[i]):].tolist()


def tiny_model(seed=0, **kw):
    from llm_engine_amd.engine import synthetic_weights
    arch = dict(hidden=64, inter=160, layers=2, q_heads=4, kv_heads=2, head_dim=16, vocab=300,
                max_pos=1024, eps=1e-6, theta=1e4, tie=True, qkv_bias=True)
    arch.update(kw)
    return synthetic_weights(arch, seed)


def test_oracle_greedy_invariances():
    """Chunked prefill and batch composition leave the oracle's tokens
    bit-identical (its arithmetic is per token)."""
    from e2e_util import OracleModel
    from llm_engine_amd.engine import greedy_loop, sched_config
    w = tiny_model(1)
    rng = np.random.default_rng(0)
    prompts = [rng.integers(0, 300, n).tolist() for n in (5, 40, 77)]

    def run(chunk, ps, frag=0):
        m = OracleModel(w, 64, threads=2)
        return greedy_loop(m.forward, ps, [6] * len(ps), 64, 16,
                           sched_config(prefill_chunk_size=chunk), fragment_blocks=frag)

    whole = run(4096, prompts)
    assert run(16, prompts) == whole
    assert run(7, prompts, frag=10) == whole
    for i, p in enumerate(prompts):
        assert run(4096, [p])[0] == whole[i]


def test_shuffled_pool_hands_out_a_seeded_permutation():
    """POOL_SHUFFLED | seed: the tables of the admitted sequences hold distinct
    blocks of the pool, in an order fixed by the seed (the same on every run,
    different for another seed) and far from the default low-ids-first order."""
    from llm_engine_amd.engine import POOL_SHUFFLED, Scheduler, sched_config

    def tables(seed):
        sch = Scheduler(64, 16, sched_config(max_num_batched_tokens=4096), False, POOL_SHUFFLED | seed)
        for i in range(4):
            sch.add(i, np.arange(16 * 16 - 1, dtype=np.int32) + 1, 1)  # 16 blocks each
        sl = sch.step()
        out = [np.ctypeslib.as_array(ctypes.cast(s.blocks, ctypes.POINTER(ctypes.c_int32)), (s.num_blocks,)).copy()
               for s in sl]
        sch.close()
        return np.concatenate(out)

    a, b, c = tables(7), tables(7), tables(8)
    assert len(a) >= 32 and len(set(a.tolist())) == len(a) and a.min() >= 0 and a.max() < 64
    assert np.array_equal(a, b)
    assert not np.array_equal(a, c)
    assert np.count_nonzero(np.diff(a) == 1) < 16  # not runs of consecutive ids
