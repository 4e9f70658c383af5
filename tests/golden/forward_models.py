"""Two small models for pinning the oracle's whole forward (oracle.c:
orc_forward, restating cpu_model.cpp:98-214) against Hugging Face's own
Qwen2 and Llama implementations.

Shared by make_forward_ref.py (which runs transformers in fp32 and writes
forward_ref.npz) and tests/test_oracle_forward.py (which feeds the same
weights to the oracle). Weights come from a seeded numpy generator, so the
fixture holds only inputs and outputs.

The two shapes differ in every way a forward could get wrong silently,
as the reference's own second-architecture test chooses them
(test_cpu_model.cpp:138-150): q/k/v bias or none, tied or untied head,
GQA 7 or 8, eps 1e-6 or 1e-5, theta 1e6 or 1e4. Norm weights are
1 + N(0, 0.1) and different in every norm, and the biases are N(0, 0.02),
so swapping the two norms of a layer, dropping a bias or putting it on the
wrong projection, or using the wrong head changes the outputs.
"""
from __future__ import annotations

from types import SimpleNamespace

import numpy as np

ARCHS = {
    "qwen2_tiny": dict(kind="qwen2", hidden=112, inter=304, layers=3, q_heads=14, kv_heads=2,
                       head_dim=8, vocab=512, max_pos=512, eps=1e-6, theta=1e6, tie=True,
                       qkv_bias=True),
    "llama_tiny": dict(kind="llama", hidden=128, inter=344, layers=3, q_heads=16, kv_heads=2,
                       head_dim=8, vocab=512, max_pos=512, eps=1e-5, theta=1e4, tie=False,
                       qkv_bias=False),
}
SEEDS = {"qwen2_tiny": 11, "llama_tiny": 12}
# Prompt lengths: one token, shorter than a block, several blocks (block 16).
PROMPT_LENS = (1, 6, 19, 33, 64)
GEN_TOKENS = 12
# Linear/embedding std. Larger than the usual 0.02 so that random-init
# logits have top-2 margins well above the 1e-3 the greedy check needs.
STD = 0.08


def weights(name: str):
    """Weights in the oracle's layout ([out][in] matrices), as a namespace with
    the fields OracleModel reads (arch, embed, final_norm, lm_head, layers)."""
    a = dict(ARCHS[name])
    rng = np.random.default_rng(SEEDS[name])
    H, I, V = a["hidden"], a["inter"], a["vocab"]
    QD, KVD = a["q_heads"] * a["head_dim"], a["kv_heads"] * a["head_dim"]

    def normal(*shape, std=STD):
        return (rng.standard_normal(shape) * std).astype(np.float32)

    def norm_w():
        return (1.0 + rng.standard_normal(H) * 0.1).astype(np.float32)

    embed = normal(V, H)
    lm_head = None if a["tie"] else normal(V, H)
    final_norm = norm_w()
    layers = []
    for _ in range(a["layers"]):
        L = dict(wq=normal(QD, H), wk=normal(KVD, H), wv=normal(KVD, H), wo=normal(H, QD),
                 wgate=normal(I, H), wup=normal(I, H), wdown=normal(H, I),
                 in_norm=norm_w(), post_norm=norm_w())
        if a["qkv_bias"]:
            L.update(bq=normal(QD, std=0.02), bk=normal(KVD, std=0.02), bv=normal(KVD, std=0.02))
        layers.append(L)
    return SimpleNamespace(arch=a, embed=embed, final_norm=final_norm, lm_head=lm_head,
                           layers=layers)


def prompts(name: str):
    rng = np.random.default_rng(SEEDS[name] + 100)
    V = ARCHS[name]["vocab"]
    return [rng.integers(0, V, n).astype(np.int32) for n in PROMPT_LENS]
