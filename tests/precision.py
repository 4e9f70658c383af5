"""CPU emulation of the roundings the 16-bit attention kernels make, to state
and bound their error against the fp32 oracle without a GPU.

With a 16-bit cache (bf16 or fp16) the MFMA tiles take 16-bit operands: the
query is rounded to the cache type before S = q.K^T (the decode tile rounds q;
the chunk tile rounds q * scale * log2(e), the softmax scale folded in, with
scale_log2 formed in fp32 as the host code forms it), and the softmax weights
P = exp2(s - m) (each <= 1) are rounded to the cache type before O = P.V.
Accumulation is fp32. The decode tile sums l from the unrounded weights; the
chunk tile sums l on the MFMA from the rounded ones (a row of ones beside V).
This emulation applies those roundings with the row's global maximum as m
(the kernels use running maxima, which round the same magnitudes at other
points), so it reproduces the size of the error, not its exact bits."""
from __future__ import annotations

import numpy as np

import oracle


def _round(a: np.ndarray, dt: str) -> np.ndarray:
    a = np.asarray(a, dtype=np.float32)
    if dt == "bf16":
        return oracle.bf16_to_f32(oracle.f32_to_bf16(a))
    if dt == "f16":
        return oracle.f32_to_f16(a).astype(np.float32)
    return a


def _widen(c: np.ndarray) -> np.ndarray:
    if c.dtype == np.uint16:
        return oracle.bf16_to_f32(c)
    return c.astype(np.float32)


def emulate(case, q: np.ndarray, dt: str, chunk_rows: np.ndarray | None = None, round_q: bool = True,
            round_p: bool = True) -> np.ndarray:
    """Output of the 16-bit kernels as emulated on the host, fp64 elsewhere.
    chunk_rows: boolean per query row, True where the row runs on the chunk
    tile (l from rounded weights). round_q / round_p switch each rounding off,
    to attribute the error."""
    kc, vc = _widen(case.k_cache), _widen(case.v_cache)
    G = case.q_heads // case.kv_heads
    hd = case.head_dim
    qr = (_round(q, dt) if round_q else np.asarray(q, np.float32)).astype(np.float64)
    if round_q and chunk_rows is not None and chunk_rows.any():
        # chunk rows: q * scale_log2 rounded, then taken back to q's units
        c = np.float32(case.scale) * np.float32(1.4426950408889634)
        qc = _round(np.asarray(q, np.float32) * c, dt).astype(np.float64) / np.float64(c)
        qr[chunk_rows] = qc[chunk_rows]
    out = np.zeros((q.shape[0], case.q_heads * hd), dtype=np.float64)
    bs = case.block_size
    for t in range(q.shape[0]):
        s_ = int(case.token_seq[t])
        pos = int(case.token_pos[t])
        blocks = case.tables[case.table_offset[s_]:]
        p = np.arange(pos + 1)
        slots = blocks[p // bs].astype(np.int64) * bs + p % bs
        for kvh in range(case.kv_heads):
            K = kc[slots, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            V = vc[slots, kvh * hd:(kvh + 1) * hd].astype(np.float64)
            qh = qr[t].reshape(case.q_heads, hd)[kvh * G:(kvh + 1) * G]
            s = (qh @ K.T) * case.scale
            w = np.exp(s - s.max(axis=1, keepdims=True))
            wr = _round(w.astype(np.float32), dt).astype(np.float64) if round_p else w
            l = wr.sum(axis=1) if chunk_rows is not None and chunk_rows[t] else w.sum(axis=1)
            out[t].reshape(case.q_heads, hd)[kvh * G:(kvh + 1) * G] = (wr @ V) / l[:, None]
    return out
