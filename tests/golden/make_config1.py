"""Greedy tokens of BASELINE config 1 from the CPU oracle (oracle.c, the fp32
reference forward), for the GPU end-to-end test:

  Qwen2.5-0.5B architecture, random-init fp32 weights (engine.synthetic_weights,
  seed 1234), 8 sequences of random token ids with prompt lengths uniform in
  [16, 512], 32 greedy tokens each, block size 16, 4096-block pool whose free
  list is a seeded random permutation (POOL_SHUFFLED | POOL_SEED), so every
  block table is drawn from a random permutation of the pool, scheduled by the
  engine's scheduler (which reproduces the reference scheduler,
  tests/test_engine_host.py).

    python tests/golden/make_config1.py   # ~ minutes on 8 cores

Writes config1_tokens.json: inputs (seeds, prompts), expected tokens, and per
step and logits row the oracle's top-1 and top-2 (index, logit) pairs, with
the smallest top-1/top-2 margin per sequence (near ties are where a reordered
fp32 sum could legitimately flip a token; the GPU test compares the device
logits at those indices against these values)."""
from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
for p in (ROOT / "llm-engine_amd", ROOT / "oracle", ROOT / "tests"):
    sys.path.insert(0, str(p))

from e2e_util import OracleModel, top2_margin  # noqa: E402
from llm_engine_amd.engine import POOL_SHUFFLED, greedy_loop, sched_config, synthetic_weights  # noqa: E402

WEIGHT_SEED, PROMPT_SEED = 1234, 1
N_SEQS, GEN, NUM_BLOCKS, POOL_SEED = 8, 32, 4096, 4242
FRAGMENT = POOL_SHUFFLED | POOL_SEED


def prompts_config1(vocab):
    rng = np.random.default_rng(PROMPT_SEED)
    lens = rng.integers(16, 513, size=N_SEQS)
    return [rng.integers(0, vocab, size=int(n)).astype(np.int32).tolist() for n in lens]


def weight_digest(w) -> str:
    h = hashlib.sha256()
    h.update(w.embed[:64].tobytes())
    h.update(w.layers[-1]["wdown"][-64:].tobytes())
    return h.hexdigest()[:16]


def main():
    t0 = time.time()
    w = synthetic_weights("qwen2.5-0.5b", WEIGHT_SEED)
    prompts = prompts_config1(w.arch["vocab"])
    m = OracleModel(w, NUM_BLOCKS)
    margins = {}
    top2 = []  # per step: [seq_key, i1, v1, i2, v2] per logits row

    def top_two(r):
        i1 = int(np.argmax(r == r.max()))
        rr = r.copy()
        rr[i1] = -np.inf
        i2 = int(np.argmax(rr == rr.max()))
        return [i1, float(r[i1]), i2, float(r[i2])]

    def fwd(slices, n_logits):
        lg = m.logits(slices)
        toks = np.array([int(np.argmax(r == r.max())) for r in lg], dtype=np.int32)  # first max
        k = 0
        rows = []
        for s in slices:
            if s.needs_logits:
                margins.setdefault(int(s.seq_key), []).append(top2_margin(lg[k]))
                rows.append([int(s.seq_key)] + top_two(lg[k]))
                k += 1
        top2.append(rows)
        print(f"  step: {len(slices)} slices, {time.time() - t0:.0f}s", flush=True)
        return toks

    toks = greedy_loop(fwd, prompts, [GEN] * N_SEQS, NUM_BLOCKS, 16,
                       sched_config(max_num_batched_tokens=4096), fragment_blocks=FRAGMENT)
    out = {"arch": "qwen2.5-0.5b", "weight_seed": WEIGHT_SEED, "prompt_seed": PROMPT_SEED,
           "weight_digest": weight_digest(w), "num_blocks": NUM_BLOCKS, "fragment_blocks": FRAGMENT,
           "max_num_batched_tokens": 4096, "gen": GEN, "prompts": prompts, "tokens": toks,
           "min_margin": [min(margins[i]) for i in range(N_SEQS)], "top2": top2,
           "seconds": round(time.time() - t0, 1)}
    (HERE / "config1_tokens.json").write_text(json.dumps(out))
    print("done", out["min_margin"], out["seconds"])


if __name__ == "__main__":
    main()
