"""End-to-end helpers for the tests: the CPU oracle model (oracle.c:orc_forward,
restating cpu_model.cpp:98-214) behind the same forward(slices) interface as
the device model, so one greedy loop drives both."""
from __future__ import annotations

import ctypes

import numpy as np

import oracle


class OracleModel:
    def __init__(self, w, num_blocks, block_size=16, kv_bf16=False, threads=None):
        a = w.arch
        self.a, self.bs, self.kv_bf16 = a, block_size, kv_bf16
        self.threads = threads or oracle.threads_default()
        n = a["layers"]
        slots = num_blocks * block_size
        kvd = a["kv_heads"] * a["head_dim"]
        dt = np.uint16 if kv_bf16 else np.float32
        self.kc = [np.zeros((slots, kvd), dt) for _ in range(n)]
        self.vc = [np.zeros((slots, kvd), dt) for _ in range(n)]
        self.cos, self.sin = oracle.rope_tables(a["head_dim"], a["max_pos"], a["theta"])
        P = ctypes.c_void_p

        def arr(key):
            if key in ("bq", "bk", "bv") and not a["qkv_bias"]:
                return None
            return (P * n)(*[L[key].ctypes.data for L in w.layers])

        self._w = w
        self._arrs = {k: arr(k) for k in ("in_norm", "post_norm", "wq", "wk", "wv", "wo", "bq", "bk",
                                          "bv", "wgate", "wup", "wdown")}

        class M(ctypes.Structure):
            _fields_ = [(x, ctypes.c_int) for x in ("hidden", "inter", "layers", "q_heads", "kv_heads",
                                                     "head_dim", "vocab", "max_pos")] + [
                ("eps", ctypes.c_float), ("theta", ctypes.c_float), ("tie", ctypes.c_int),
                ("embed", P), ("final_norm", P), ("lm_head", P)] + [
                (k, P) for k in ("in_norm", "post_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv",
                                 "wgate", "wup", "wdown")]

        self.m = M(a["hidden"], a["inter"], n, a["q_heads"], a["kv_heads"], a["head_dim"], a["vocab"],
                   a["max_pos"], a["eps"], a["theta"], int(a["tie"]), w.embed.ctypes.data,
                   w.final_norm.ctypes.data, None if w.lm_head is None else w.lm_head.ctypes.data,
                   *[ctypes.cast(v, P) if v is not None else None for v in self._arrs.values()])
        self.kp = (P * n)(*[c.ctypes.data for c in self.kc])
        self.vp = (P * n)(*[c.ctypes.data for c in self.vc])

    def logits(self, slices):
        return self.trace(slices, resid=False)[0]

    def trace(self, slices, resid=True):
        """Logits of the step's logit rows and, with resid, the residual
        stream [layers+1][tokens][hidden] (orc_forward_trace)."""
        pk = oracle.pack_step([(s.seq_key, s.start, s.len, s.needs_logits,
                                np.ctypeslib.as_array(ctypes.cast(s.blocks, ctypes.POINTER(ctypes.c_int32)), (s.num_blocks,)),
                                np.ctypeslib.as_array(ctypes.cast(s.tokens, ctypes.POINTER(ctypes.c_int32)), (s.start + s.len,)))
                               for s in slices], self.bs)
        R = len(pk.logit_rows)
        out = np.zeros((max(R, 1), self.a["vocab"]), np.float32)
        pt = oracle.ptr
        N = len(pk.token_ids)
        res = np.zeros((self.a["layers"] + 1, N, self.a["hidden"]), np.float32) if resid else None
        oracle.lib().orc_forward_trace(ctypes.byref(self.m), pt(self.cos), pt(self.sin), self.kp, self.vp,
                                       int(self.kv_bf16), pt(pk.token_ids), pt(pk.positions), pt(pk.slots),
                                       pt(pk.token_seq), pt(pk.tables), pt(pk.table_offset), N,
                                       pt(pk.logit_rows), R, self.bs, pt(out), self.threads,
                                       None if res is None else pt(res))
        return out[:R], res

    def forward(self, slices, n_logits):
        lg = self.logits(slices)
        return np.array([oracle.argmax(r) for r in lg], dtype=np.int32)


def top2_margin(logits_row: np.ndarray) -> float:
    t = np.partition(logits_row, -2)[-2:]
    return float(t[1] - t[0])


def poisson_arrival_steps(n: int, rate_per_s: float, step_s: float, seed: int) -> list[int]:
    """Poisson arrivals (exponential gaps at rate_per_s, seeded) on a step
    clock: request i joins before step floor(t_i / step_s). The step clock
    makes the schedule independent of how fast either model runs, so the
    device and the oracle see the same batches."""
    rng = np.random.default_rng(seed)
    t = np.cumsum(rng.exponential(1.0 / rate_per_s, n))
    return [int(x) for x in np.floor(t / step_s)]


def lockstep(device, oracle_model, prompts, max_tokens, num_blocks, cfg=None, prefix_caching=False,
             fragment_blocks=0, arrival_steps=None, block_size=16, max_steps=100000):
    """One scheduler drives the device model and the oracle model over the
    same steps (the reference's greedy_run, test_cuda_invariance.cpp:90-143,
    with both models in the loop). Each step the device's greedy tokens and
    logits are compared with the oracle's logits on the same slices; both
    continue from the device's tokens. Returns the generated tokens, per
    logits row (device token, oracle argmax, oracle top-2 margin, the step's
    max |device - oracle| logit difference, max |oracle logit|, sequence id),
    and the most slices any step held."""
    from llm_engine_amd.engine import Scheduler
    sch = Scheduler(num_blocks, block_size, cfg, prefix_caching, fragment_blocks)
    order = sorted(range(len(prompts)), key=lambda i: (arrival_steps[i] if arrival_steps else 0, i))
    nxt = 0
    rows = []
    max_running = 0
    for step in range(max_steps):
        while nxt < len(order) and (arrival_steps is None or arrival_steps[order[nxt]] <= step):
            i = order[nxt]
            sch.add(i, prompts[i], max_tokens[i])
            nxt += 1
        if not sch.has_work():
            if nxt >= len(order):
                break
            continue
        sl = sch.step()
        if not len(sl):
            continue
        n = sum(int(s.needs_logits) for s in sl)
        max_running = max(max_running, len(sl))
        toks, lg = device.forward(sl, n, want_logits=True)
        want = oracle_model.logits(sl)
        if n:
            err = float(np.max(np.abs(lg - want)))
            scale = float(np.abs(want).max())
            ids = [int(s.seq_key) for s in sl if s.needs_logits]
            for r in range(n):
                rows.append((int(toks[r]), int(oracle.argmax(want[r])), top2_margin(want[r]), err, scale, ids[r]))
        sch.done(toks)
    out = [sch.generated(i) for i in range(len(prompts))]
    sch.close()
    return out, rows, max_running


def check_rows(rows, exact: bool):
    """Greedy tokens against the oracle: every row when `exact` (the fp32
    path), else every row whose oracle top-2 margin exceeds twice the step's
    measured logit difference. Returns (rows checked, rows total)."""
    checked = 0
    for dev_tok, want_tok, margin, err, _, _ in rows:
        if exact or margin > 2 * err:
            assert dev_tok == want_tok, (dev_tok, want_tok, margin, err)
            checked += 1
    return checked, len(rows)
