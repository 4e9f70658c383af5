"""Seeded synthetic inputs for the paged-attention path (shared by the tests,
bench.py and the fixture writer). Shapes follow the configs the benchmark is
quoted on: Qwen2.5-0.5B GQA (14 q heads, 2 kv heads, head_dim 64), block 16,
block tables drawn from a random permutation of a large pool (fragmented)."""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass
class AttnCase:
    q_heads: int
    kv_heads: int
    head_dim: int
    block_size: int
    num_blocks: int
    q: np.ndarray            # [N, q_heads*head_dim] f32
    k_cache: np.ndarray      # [num_blocks*bs, kv_heads*head_dim] f32, uint16 (bf16 bits) or float16
    v_cache: np.ndarray
    tables: np.ndarray       # concatenated block tables (int32)
    table_offset: np.ndarray  # [S]
    table_len: np.ndarray    # [S]
    token_seq: np.ndarray    # [N]
    token_pos: np.ndarray    # [N]
    seq_start: np.ndarray    # [S] first position of each sequence's rows
    seq_qlen: np.ndarray     # [S] rows per sequence (1 = decode)

    @property
    def n_tokens(self) -> int:
        return int(self.q.shape[0])

    @property
    def scale(self) -> float:
        return float(np.float32(1.0) / np.sqrt(np.float32(self.head_dim)))

    def blocks_of(self, s: int) -> np.ndarray:
        o = int(self.table_offset[s])
        return self.tables[o:o + int(self.table_len[s])]


def loguniform_ctx(rng: np.random.Generator, n: int, lo: int, hi: int) -> np.ndarray:
    return np.rint(np.exp(rng.uniform(np.log(lo), np.log(hi), size=n))).astype(np.int64)


def make_case(ctx, q_heads=14, kv_heads=2, head_dim=64, block_size=16, num_blocks=None,
              q_len=None, seed=0, kv_bf16=False, fill="normal", kv_f16=False) -> AttnCase:
    """ctx[s] = context length of sequence s after this step; q_len[s] = rows of
    sequence s in the step (1 = decode row; >1 = the last q_len positions, a
    prefill chunk). Tables are a random permutation of the pool, so no two
    consecutive logical blocks are physically adjacent by construction."""
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx, dtype=np.int64)
    S = len(ctx)
    q_len = np.ones(S, dtype=np.int64) if q_len is None else np.asarray(q_len, dtype=np.int64)
    assert np.all(q_len >= 1) and np.all(q_len <= ctx)
    nblk = (ctx + block_size - 1) // block_size
    need = int(nblk.sum())
    if num_blocks is None:
        num_blocks = max(need, 64)
    assert need <= num_blocks, "pool too small"
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = perm[:need].copy()
    table_offset = np.concatenate([[0], np.cumsum(nblk)[:-1]]).astype(np.int32)
    kv_dim = kv_heads * head_dim
    slots = num_blocks * block_size
    if fill == "normal":
        k = rng.standard_normal((slots, kv_dim), dtype=np.float32)
        v = rng.standard_normal((slots, kv_dim), dtype=np.float32)
    else:  # tables and q only; the caller provides the caches
        k = v = np.zeros((0, kv_dim), dtype=np.float32)
    N = int(q_len.sum())
    q = rng.standard_normal((N, q_heads * head_dim), dtype=np.float32)
    token_seq = np.repeat(np.arange(S, dtype=np.int32), q_len)
    seq_start = (ctx - q_len).astype(np.int32)
    token_pos = np.concatenate([np.arange(seq_start[s], ctx[s]) for s in range(S)]).astype(np.int32)
    if kv_bf16 and fill == "normal":
        import oracle  # test infrastructure: host RNE rounding identical to tensor.h
        k = oracle.f32_to_bf16(k)
        v = oracle.f32_to_bf16(v)
    elif kv_f16 and fill == "normal":
        import oracle
        k = oracle.f32_to_f16(k)
        v = oracle.f32_to_f16(v)
    return AttnCase(q_heads, kv_heads, head_dim, block_size, num_blocks, q, k, v, tables,
                    table_offset, nblk.astype(np.int32), token_seq, token_pos, seq_start,
                    q_len.astype(np.int32))


def make_shared_prefix_case(suffix, prefix_blocks=32, q_len=None, num_blocks=16384, seed=0,
                            kv_bf16=False, q_heads=14, kv_heads=2, head_dim=64, block_size=16) -> AttnCase:
    """Config 5's cache state: every sequence's table starts with the same
    prefix_blocks refcounted blocks (one shared prefix), then suffix[s] tokens
    in blocks of its own, all drawn from a random permutation of the pool
    (fragmented). Rows as make_case: the last q_len[s] positions."""
    rng = np.random.default_rng(seed)
    suffix = np.asarray(suffix, dtype=np.int64)
    S = len(suffix)
    ctx = prefix_blocks * block_size + suffix
    q_len = np.ones(S, dtype=np.int64) if q_len is None else np.asarray(q_len, dtype=np.int64)
    assert np.all(q_len >= 1) and np.all(q_len <= ctx)
    own = (suffix + block_size - 1) // block_size
    assert prefix_blocks + int(own.sum()) <= num_blocks, "pool too small"
    perm = rng.permutation(num_blocks).astype(np.int32)
    shared, rest = perm[:prefix_blocks], perm[prefix_blocks:]
    tables, o = [], 0
    for s in range(S):
        tables.append(np.concatenate([shared, rest[o:o + int(own[s])]]))
        o += int(own[s])
    table_len = np.array([len(t) for t in tables], dtype=np.int32)
    table_offset = np.concatenate([[0], np.cumsum(table_len)[:-1]]).astype(np.int32)
    kv_dim = kv_heads * head_dim
    k = rng.standard_normal((num_blocks * block_size, kv_dim), dtype=np.float32)
    v = rng.standard_normal((num_blocks * block_size, kv_dim), dtype=np.float32)
    if kv_bf16:
        import oracle  # test infrastructure: host RNE rounding identical to tensor.h
        k, v = oracle.f32_to_bf16(k), oracle.f32_to_bf16(v)
    N = int(q_len.sum())
    q = rng.standard_normal((N, q_heads * head_dim), dtype=np.float32)
    token_seq = np.repeat(np.arange(S, dtype=np.int32), q_len)
    seq_start = (ctx - q_len).astype(np.int32)
    token_pos = np.concatenate([np.arange(seq_start[s], ctx[s]) for s in range(S)]).astype(np.int32)
    return AttnCase(q_heads, kv_heads, head_dim, block_size, num_blocks, q, k, v,
                    np.concatenate(tables).astype(np.int32), table_offset, table_len, token_seq, token_pos,
                    seq_start, q_len.astype(np.int32))


def fragment_like_reference(num_blocks: int, n_single: int = 40):
    """Free-list order after the reference's fragmentation recipe
    (test_cuda_invariance.cpp:98-105): allocate n_single one-block sequences
    from a fresh pool (free list hands out low ids first,
    block_allocator.cpp:13), then free every other one. Returns the free list
    as the allocator would pop it (last element first)."""
    free = list(range(num_blocks - 1, -1, -1))
    held = [free.pop() for _ in range(n_single)]
    for i in range(0, len(held), 2):
        free.append(held[i])  # release_block pushes back onto the free list
    return free


def parse_trace(trace: np.ndarray):
    """-> (steps, tokens): steps = list of list of (seq_id, start, len,
    needs_logits, is_prefill, blocks); tokens[seq_id] = final token list."""
    i, steps = 0, []
    while trace[i] != -1:
        ns = int(trace[i]); i += 1
        sl = []
        for _ in range(ns):
            sid, start, ln, nl, pf, nbk = (int(v) for v in trace[i:i + 6]); i += 6
            sl.append((sid, start, ln, nl, pf, trace[i:i + nbk].copy())); i += nbk
        steps.append(sl)
    i += 1
    toks = []
    while i < len(trace):
        n = int(trace[i]); i += 1
        toks.append(trace[i:i + n].copy()); i += n
    return steps, toks
