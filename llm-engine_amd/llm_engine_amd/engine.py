"""End-to-end engine over the hot path: device model, scheduler, greedy loop.

The model architectures are the ones the benchmark configs name, with
random-init weights from a seed (there is no network for checkpoints):
linear and embedding weights N(0, 0.02), RMSNorm weights 1, biases 0 (the
Hugging Face initialisation convention).
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass, field

import numpy as np

from . import _lib
from ._lib import LE_BF16, LE_F16, LE_F32, ModelDesc, RunStats, SchedConfig, StepSlice, check

ARCHS = {
    # Qwen2.5-0.5B: qkv bias, tied embeddings
    "qwen2.5-0.5b": dict(hidden=896, inter=4864, layers=24, q_heads=14, kv_heads=2, head_dim=64,
                         vocab=151936, max_pos=32768, eps=1e-6, theta=1e6, tie=True, qkv_bias=True),
    # TinyLlama-1.1B: no qkv bias, untied head
    "tinyllama-1.1b": dict(hidden=2048, inter=5632, layers=22, q_heads=32, kv_heads=4, head_dim=64,
                           vocab=32000, max_pos=2048, eps=1e-5, theta=1e4, tie=False, qkv_bias=False),
}


@dataclass
class Weights:
    arch: dict
    embed: np.ndarray
    final_norm: np.ndarray
    lm_head: np.ndarray | None
    layers: list = field(default_factory=list)  # dicts of per-layer arrays


def synthetic_weights(arch: str | dict, seed: int, layers: int | None = None) -> Weights:
    """Random-init weights in a fixed generation order (embedding, head, then
    per layer q, k, v, o, gate, up, down), so a seed names one model."""
    a = dict(ARCHS[arch] if isinstance(arch, str) else arch)
    if layers is not None:
        a["layers"] = layers
    rng = np.random.default_rng(seed)
    H, I, V = a["hidden"], a["inter"], a["vocab"]
    QD, KVD = a["q_heads"] * a["head_dim"], a["kv_heads"] * a["head_dim"]
    s = np.float32(0.02)

    def normal(*shape):
        x = rng.standard_normal(shape, dtype=np.float32)
        x *= s
        return x

    embed = normal(V, H)
    lm_head = None if a["tie"] else normal(V, H)
    w = Weights(a, embed, np.ones(H, np.float32), lm_head)
    for _ in range(a["layers"]):
        L = dict(wq=normal(QD, H), wk=normal(KVD, H), wv=normal(KVD, H), wo=normal(H, QD),
                 wgate=normal(I, H), wup=normal(I, H), wdown=normal(H, I),
                 in_norm=np.ones(H, np.float32), post_norm=np.ones(H, np.float32))
        if a["qkv_bias"]:
            L.update(bq=np.zeros(QD, np.float32), bk=np.zeros(KVD, np.float32), bv=np.zeros(KVD, np.float32))
        w.layers.append(L)
    return w


def sched_config(max_num_seqs=32, max_num_batched_tokens=4096, prefill_chunk_size=512,
                 continuous=True, watermark_blocks=-1, admission_lookahead=1,
                 starvation_wait_steps=64, max_queue_wait_seconds=0.0) -> SchedConfig:
    return SchedConfig(int(continuous), max_num_seqs, max_num_batched_tokens, prefill_chunk_size,
                       admission_lookahead, starvation_wait_steps, watermark_blocks, 0,
                       max_queue_wait_seconds)


class Model:
    """The device model (le_model_create): weights uploaded once, one K/V cache
    pair per layer of num_blocks * block_size slots."""

    DTYPES = {"f32": LE_F32, "bf16": LE_BF16, "f16": LE_F16}

    def __init__(self, w: Weights, num_blocks: int, block_size: int = 16, dtype: str = "f32",
                 kv_dtype: str | None = None, attention: str = "ragged", decode_graph: bool = False,
                 unfused_norms: bool = False):
        """attention: "ragged" (le_ragged_paged_attention_qkv over the packed
        step) or "reference" (the reference-shaped le_attention_decode).
        decode_graph: replay decode steps from captured HIP graphs
        (le_model_set_decode_graph). unfused_norms: a bf16 model keeps its
        RMSNorm launches instead of folding them into the GEMMs."""
        a = w.arch
        self.arch = a
        self.num_blocks, self.block_size = num_blocks, block_size
        dt = self.DTYPES[dtype]
        kvdt = dt if kv_dtype is None else self.DTYPES[kv_dtype]
        attn = {"ragged": 0, "reference": 1}[attention]
        n = a["layers"]

        def arr(key):
            if key in ("bq", "bk", "bv") and not a["qkv_bias"]:
                return None
            return (ctypes.c_void_p * n)(*[L[key].ctypes.data for L in w.layers])

        self._keep = {k: arr(k) for k in ("in_norm", "post_norm", "wq", "wk", "wv", "wo", "bq", "bk",
                                          "bv", "wgate", "wup", "wdown")}
        d = ModelDesc(a["hidden"], a["inter"], n, a["q_heads"], a["kv_heads"], a["head_dim"],
                      a["vocab"], a["max_pos"], a["eps"], a["theta"], int(a["tie"]), dt, kvdt, attn,
                      w.embed.ctypes.data, w.final_norm.ctypes.data,
                      None if w.lm_head is None else w.lm_head.ctypes.data)
        for k, v in self._keep.items():
            setattr(d, k, ctypes.cast(v, ctypes.POINTER(ctypes.c_void_p)) if v is not None else None)
        d.unfused_norms = int(unfused_norms)
        st = ctypes.c_int(0)
        self._h = _lib.load().le_model_create(ctypes.byref(d), num_blocks, block_size, ctypes.byref(st))
        if not self._h:
            raise _lib.LeError("le_model_create", st.value or _lib.LE_EINVAL)
        self._keep = None  # weights are on the device now
        if decode_graph:
            check("le_model_set_decode_graph", _lib.load().le_model_set_decode_graph(self._h, 1))

    @property
    def graph_replays(self) -> int:
        return int(_lib.load().le_model_graph_replays(self._h))

    def set_plan_flags(self, flags: int) -> None:
        """le_plan_config.flags for the model's plans (le_model_set_plan_flags)."""
        check("le_model_set_plan_flags", _lib.load().le_model_set_plan_flags(self._h, int(flags)))

    @property
    def eager_fallbacks(self) -> int:
        """Decode steps run eagerly although graph replay is on (le_model_eager_fallbacks)."""
        return int(_lib.load().le_model_eager_fallbacks(self._h))

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().le_model_destroy(self._h)
            self._h = None

    __del__ = close

    def forward(self, slices, n_logits: int, want_logits: bool = False):
        """slices: ctypes StepSlice array (as le_sched_step returns them)."""
        toks = np.zeros(max(n_logits, 1), dtype=np.int32)
        logits = np.zeros((max(n_logits, 1), self.arch["vocab"]), dtype=np.float32) if want_logits else None
        check("le_model_forward", _lib.load().le_model_forward(
            self._h, slices, len(slices), toks.ctypes.data,
            None if logits is None else logits.ctypes.data))
        return toks[:n_logits], (None if logits is None else logits[:n_logits])

    def run_greedy(self, prompts, max_tokens, cfg: SchedConfig | None = None, prefix_caching=False,
                   fragment_blocks=0, arrival_s=None):
        """Greedy generation through the C++ scheduler loop (le_run_greedy)."""
        cfg = cfg or sched_config()
        lens = np.array([len(p) for p in prompts], dtype=np.int32)
        flat = np.concatenate([np.asarray(p, dtype=np.int32) for p in prompts]).astype(np.int32)
        mt = np.asarray(max_tokens, dtype=np.int32)
        out = np.full(int(mt.sum()), -1, dtype=np.int32)
        arr = None if arrival_s is None else np.asarray(arrival_s, dtype=np.float64)
        stats = RunStats()
        check("le_run_greedy", _lib.load().le_run_greedy(
            self._h, ctypes.byref(cfg), int(prefix_caching), fragment_blocks, len(prompts),
            lens.ctypes.data, flat.ctypes.data, mt.ctypes.data,
            None if arr is None else arr.ctypes.data, out.ctypes.data, ctypes.byref(stats)))
        res, o = [], 0
        for m in mt:
            g = out[o:o + m]
            res.append(g[g >= 0].tolist())
            o += m
        return res, stats


class Scheduler:
    """The steppable scheduler (le_sched_*), for loops that run their own model."""

    def __init__(self, num_blocks, block_size=16, cfg: SchedConfig | None = None,
                 prefix_caching=False, fragment_blocks=0):
        self._cfg = cfg or sched_config()
        self._h = _lib.load().le_sched_create(num_blocks, block_size, int(prefix_caching),
                                              ctypes.byref(self._cfg), fragment_blocks)
        if not self._h:
            raise _lib.LeError("le_sched_create", _lib.LE_EINVAL)
        self._buf = (StepSlice * 1024)()

    def close(self):
        if getattr(self, "_h", None):
            _lib.load().le_sched_destroy(self._h)
            self._h = None

    __del__ = close

    def add(self, seq_id, prompt, max_tokens):
        p = np.ascontiguousarray(prompt, dtype=np.int32)
        check("le_sched_add", _lib.load().le_sched_add(self._h, seq_id, p.ctypes.data, p.size, max_tokens))

    def has_work(self) -> bool:
        return bool(_lib.load().le_sched_has_work(self._h))

    def step(self):
        n = ctypes.c_int(0)
        st = _lib.load().le_sched_step(self._h, self._buf, len(self._buf), ctypes.byref(n))
        if st == _lib.LE_ENOSPACE:
            self._buf = (StepSlice * (2 * n.value))()
            raise RuntimeError("step larger than the slice buffer; retry")
        check("le_sched_step", st)
        return (StepSlice * n.value).from_buffer(self._buf) if n.value else []

    def done(self, sampled):
        s = np.ascontiguousarray(sampled, dtype=np.int32)
        check("le_sched_done", _lib.load().le_sched_done(self._h, s.ctypes.data if s.size else None, s.size))

    def generated(self, seq_id, cap=1 << 16):
        out = np.zeros(cap, dtype=np.int32)
        n = _lib.load().le_sched_generated(self._h, seq_id, out.ctypes.data, cap)
        return out[:min(n, cap)].tolist()


# Pool preparation code for fragment_blocks (LE_POOL_SHUFFLED in le_engine.h):
# POOL_SHUFFLED | seed puts the whole free list in a seeded random order.
POOL_SHUFFLED = 1 << 30


def greedy_loop(forward, prompts, max_tokens, num_blocks, block_size=16, cfg=None,
                prefix_caching=False, fragment_blocks=0, max_steps=100000, on_step=None):
    """The reference's greedy_run (test_cuda_invariance.cpp:90-143) with any
    model: forward(slices, n_logits) -> greedy token per logits row."""
    sch = Scheduler(num_blocks, block_size, cfg, prefix_caching, fragment_blocks)
    for i, (p, m) in enumerate(zip(prompts, max_tokens)):
        sch.add(i, p, m)
    for _ in range(max_steps):
        if not sch.has_work():
            break
        sl = sch.step()
        if not len(sl):
            break
        n_logits = sum(int(s.needs_logits) for s in sl)
        toks = forward(sl, n_logits)
        if on_step:
            on_step(sl, toks)
        sch.done(toks)
    out = [sch.generated(i) for i in range(len(prompts))]
    sch.close()
    return out
