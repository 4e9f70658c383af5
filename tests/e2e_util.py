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
        pk = oracle.pack_step([(s.seq_key, s.start, s.len, s.needs_logits,
                                np.ctypeslib.as_array(ctypes.cast(s.blocks, ctypes.POINTER(ctypes.c_int32)), (s.num_blocks,)),
                                np.ctypeslib.as_array(ctypes.cast(s.tokens, ctypes.POINTER(ctypes.c_int32)), (s.start + s.len,)))
                               for s in slices], self.bs)
        R = len(pk.logit_rows)
        out = np.zeros((max(R, 1), self.a["vocab"]), np.float32)
        pt = oracle.ptr
        oracle.lib().orc_forward(ctypes.byref(self.m), pt(self.cos), pt(self.sin), self.kp, self.vp,
                                 int(self.kv_bf16), pt(pk.token_ids), pt(pk.positions), pt(pk.slots),
                                 pt(pk.token_seq), pt(pk.tables), pt(pk.table_offset),
                                 len(pk.token_ids), pt(pk.logit_rows), R, self.bs, pt(out), self.threads)
        return out[:R]

    def forward(self, slices, n_logits):
        lg = self.logits(slices)
        return np.array([oracle.argmax(r) for r in lg], dtype=np.int32)


def top2_margin(logits_row: np.ndarray) -> float:
    t = np.partition(logits_row, -2)[-2:]
    return float(t[1] - t[0])
