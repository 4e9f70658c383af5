#!/usr/bin/env python3
"""Writes tests/golden/forward_ref.npz: Hugging Face fp32 outputs for the two
small models of forward_models.py, the ground truth that pins the oracle's
whole forward (oracle.c:orc_forward).

It records what the reference's own ground-truth dumper records
(reference/dump_logits.py:1-24, read by test_cpu_model.cpp:80-129): for
each prompt the residual stream after the embedding and after every layer,
the last position's logits, and the greedy continuation, plus each
continuation step's top-2 logit margin.

Run in the build container only (it needs transformers, which the GPU box
does not use); the fixture it writes is data and travels with the tests.
    python tests/golden/make_forward_ref.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE))
import forward_models as fm  # noqa: E402


def hf_model(name: str, w):
    from transformers import LlamaConfig, LlamaForCausalLM, Qwen2Config, Qwen2ForCausalLM
    a = w.arch
    common = dict(vocab_size=a["vocab"], hidden_size=a["hidden"], intermediate_size=a["inter"],
                  num_hidden_layers=a["layers"], num_attention_heads=a["q_heads"],
                  num_key_value_heads=a["kv_heads"], head_dim=a["head_dim"],
                  max_position_embeddings=a["max_pos"], rms_norm_eps=a["eps"],
                  rope_parameters={"rope_type": "default", "rope_theta": a["theta"]},
                  tie_word_embeddings=a["tie"], hidden_act="silu")
    if a["kind"] == "qwen2":
        cfg = Qwen2Config(use_sliding_window=False, **common)
        cls = Qwen2ForCausalLM
    else:
        cfg = LlamaConfig(attention_bias=False, mlp_bias=False, **common)
        cls = LlamaForCausalLM
    cfg._attn_implementation = "eager"
    m = cls(cfg).eval().to(torch.float32)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x))  # noqa: E731
    sd = {"model.embed_tokens.weight": t(w.embed), "model.norm.weight": t(w.final_norm)}
    if not a["tie"]:
        sd["lm_head.weight"] = t(w.lm_head)
    for i, L in enumerate(w.layers):
        p = f"model.layers.{i}."
        sd.update({p + "self_attn.q_proj.weight": t(L["wq"]), p + "self_attn.k_proj.weight": t(L["wk"]),
                   p + "self_attn.v_proj.weight": t(L["wv"]), p + "self_attn.o_proj.weight": t(L["wo"]),
                   p + "mlp.gate_proj.weight": t(L["wgate"]), p + "mlp.up_proj.weight": t(L["wup"]),
                   p + "mlp.down_proj.weight": t(L["wdown"]),
                   p + "input_layernorm.weight": t(L["in_norm"]),
                   p + "post_attention_layernorm.weight": t(L["post_norm"])})
        if a["qkv_bias"]:
            sd.update({p + "self_attn.q_proj.bias": t(L["bq"]), p + "self_attn.k_proj.bias": t(L["bk"]),
                       p + "self_attn.v_proj.bias": t(L["bv"])})
    missing, unexpected = m.load_state_dict(sd, strict=False)
    # Only derived buffers (rotary inv_freq) and a tied head may be absent.
    assert not unexpected, unexpected
    assert all("rotary" in k or (a["tie"] and k == "lm_head.weight") for k in missing), missing
    if a["tie"]:
        assert torch.equal(m.lm_head.weight, m.model.embed_tokens.weight)
    return m


def main():
    out = {}
    torch.manual_seed(0)
    for name in fm.ARCHS:
        w = fm.weights(name)
        m = hf_model(name, w)
        resid = []
        hooks = [m.model.embed_tokens.register_forward_hook(
            lambda mod, i, o: resid.append(o.detach()[0].clone()))]
        for layer in m.model.layers:
            hooks.append(layer.register_forward_hook(
                lambda mod, i, o: resid.append((o[0] if isinstance(o, tuple) else o).detach()[0].clone())))
        with torch.no_grad():
            for pi, ids in enumerate(fm.prompts(name)):
                resid.clear()
                logits = m(torch.from_numpy(ids.astype(np.int64))[None]).logits[0]
                assert len(resid) == w.arch["layers"] + 1
                out[f"{name}.p{pi}.ids"] = ids
                out[f"{name}.p{pi}.resid"] = torch.stack(resid).numpy().astype(np.float32)
                out[f"{name}.p{pi}.logits"] = logits[-1].numpy().astype(np.float32)
                # Greedy continuation, recomputing the whole sequence each step.
                seq = ids.astype(np.int64).tolist()
                gen, margins = [], []
                for _ in range(fm.GEN_TOKENS):
                    lg = m(torch.tensor([seq])).logits[0, -1]
                    top = torch.topk(lg, 2).values
                    tok = int(torch.argmax(lg))
                    gen.append(tok)
                    margins.append(float(top[0] - top[1]))
                    seq.append(tok)
                out[f"{name}.p{pi}.gen"] = np.array(gen, np.int32)
                out[f"{name}.p{pi}.margin"] = np.array(margins, np.float32)
        for h in hooks:
            h.remove()
    import transformers
    out["meta.transformers"] = np.array(transformers.__version__)
    out["meta.torch"] = np.array(torch.__version__)
    np.savez_compressed(HERE / "forward_ref.npz", **out)
    print("wrote", HERE / "forward_ref.npz")


if __name__ == "__main__":
    main()
