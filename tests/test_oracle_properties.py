"""What the mathematics fixes about paged attention, checked on the oracle
(so a dropped term, a wrong index or a transposed operand fails here even
without the reference): closed forms, a float64 brute force, and the
invariances the reference's own model tests rely on."""
import numpy as np
import pytest

import oracle
from cases import make_case


def brute(case):
    """softmax(q K^T * scale) V in float64, straight from the definition."""
    qh, kvh, hd, bs = case.q_heads, case.kv_heads, case.head_dim, case.block_size
    g = qh // kvh
    out = np.zeros(case.q.shape, dtype=np.float64)
    k = case.k_cache.astype(np.float64)
    v = case.v_cache.astype(np.float64)
    for t in range(case.n_tokens):
        blocks = case.blocks_of(int(case.token_seq[t]))
        pos = int(case.token_pos[t])
        slots = np.array([blocks[p // bs] * bs + p % bs for p in range(pos + 1)])
        for h in range(qh):
            kvhead = h // g
            K = k[slots, kvhead * hd:(kvhead + 1) * hd]
            V = v[slots, kvhead * hd:(kvhead + 1) * hd]
            s = K @ case.q[t, h * hd:(h + 1) * hd].astype(np.float64) * case.scale
            p = np.exp(s - s.max())
            out[t, h * hd:(h + 1) * hd] = (p / p.sum()) @ V
    return out


def run(case):
    return oracle.paged_attention(case.q, case.k_cache, case.v_cache, case.tables,
                                  case.table_offset, case.token_seq, case.token_pos, case.q_heads,
                                  case.kv_heads, case.head_dim, case.block_size, case.scale, threads=2)


@pytest.mark.parametrize("qh,kvh,hd,bs", [(14, 2, 64, 16), (32, 4, 64, 16), (4, 4, 128, 8)])
def test_matches_float64_brute_force(qh, kvh, hd, bs):
    case = make_case([1, 33, 160], q_len=[1, 5, 1], q_heads=qh, kv_heads=kvh, head_dim=hd,
                     block_size=bs, seed=qh + hd)
    assert np.max(np.abs(run(case) - brute(case))) < 2e-6


def test_single_position_returns_v0():
    case = make_case([1, 1], seed=3)
    out = run(case)
    for s in range(2):
        slot = case.blocks_of(s)[0] * 16
        for h in range(14):
            kvh = h // 7
            np.testing.assert_array_equal(out[s, h * 64:(h + 1) * 64], case.v_cache[slot, kvh * 64:(kvh + 1) * 64])


def test_zero_query_is_mean_of_values():
    case = make_case([200], seed=4)
    case.q[:] = 0
    out = run(case)
    blocks = case.blocks_of(0)
    slots = [blocks[p // 16] * 16 + p % 16 for p in range(200)]
    mean = case.v_cache[slots].astype(np.float64).mean(axis=0)
    for h in range(14):
        kvh = h // 7
        assert np.max(np.abs(out[0, h * 64:(h + 1) * 64] - mean[kvh * 64:(kvh + 1) * 64])) < 1e-5


def test_one_dominant_key_selects_its_value():
    case = make_case([100], seed=5)
    blocks = case.blocks_of(0)
    slot = blocks[37 // 16] * 16 + 37 % 16
    case.k_cache[slot, :64] = case.q[0, :64] * 1000.0  # huge score for q head 0, kv head 0
    out = run(case)
    np.testing.assert_allclose(out[0, :64], case.v_cache[slot, :64], atol=1e-6)


def test_block_permutation_invariance():
    """Moving blocks to other physical ids, with their K/V, changes nothing."""
    case = make_case([90, 250], q_len=[1, 3], seed=6, num_blocks=64)
    base = run(case)
    rng = np.random.default_rng(0)
    perm = rng.permutation(case.num_blocks).astype(np.int32)
    k2 = np.zeros_like(case.k_cache)
    v2 = np.zeros_like(case.v_cache)
    for b in range(case.num_blocks):
        k2[perm[b] * 16:(perm[b] + 1) * 16] = case.k_cache[b * 16:(b + 1) * 16]
        v2[perm[b] * 16:(perm[b] + 1) * 16] = case.v_cache[b * 16:(b + 1) * 16]
    case.k_cache, case.v_cache, case.tables = k2, v2, perm[case.tables]
    assert np.array_equal(run(case), base)


def test_row_independent_of_batch_mates():
    """A token's output does not depend on the other rows of the step
    (test_cpu_model.cpp:160-266 batching invariance)."""
    case = make_case([50, 300, 7], seed=8)
    full = run(case)
    for s in range(3):
        sub = make_case([50, 300, 7], seed=8)
        keep = [s]
        sub.q = sub.q[keep]
        sub.token_seq = sub.token_seq[keep]
        sub.token_pos = sub.token_pos[keep]
        assert np.array_equal(run(sub)[0], full[s])


def test_linear_matches_numpy_and_keeps_order():
    rng = np.random.default_rng(1)
    a = rng.standard_normal((37, 96), dtype=np.float32)
    b = rng.standard_normal((53, 96), dtype=np.float32)
    bias = rng.standard_normal(53).astype(np.float32)
    c = oracle.linear(a, b, bias, threads=3)
    np.testing.assert_allclose(c, a.astype(np.float64) @ b.T.astype(np.float64) + bias, atol=1e-4)
    # bit-identical to the naive triple loop of cpu_model.cpp:30-36 (float accumulator, t ascending)
    i, j = 5, 17
    s = np.float32(0)
    for t in range(96):
        s = np.float32(s + np.float32(a[i, t] * b[j, t]))
    assert np.float32(s + bias[j]) == c[i, j]
    # thread count does not change the bits
    assert np.array_equal(c, oracle.linear(a, b, bias, threads=1))


def test_argmax_first_maximum_wins():
    """sampler.cpp:9-13 / test_sampler.cpp:20-26."""
    assert oracle.argmax(np.array([-1, 5, 2, 5], np.float32)) == 1
    assert oracle.argmax(np.array([3], np.float32)) == 0
    assert oracle.argmax(np.array([-9, -8, -100], np.float32)) == 1


def test_pack_step_closed_forms():
    """orc_pack_step's non-slot arrays against closed forms of the reference's
    packing (cuda_model.cu:434-491): token_seq = rank of the slice's sequence
    in first-seen order; tables = the distinct sequences' tables back to back,
    table_offset their exclusive prefix sums; logit_rows = the last row of
    each slice with needs_logits (cu_seqlens[i+1] - 1); token_ids and
    positions = tokens[start:start+len] and arange(start, start+len)."""
    rng = np.random.default_rng(11)
    for trial in range(20):
        n_seq = int(rng.integers(1, 9))
        tabs = [rng.permutation(500)[:int(rng.integers(1, 20))].astype(np.int32) for _ in range(n_seq)]
        toks = [rng.integers(0, 32000, t.size * 16).astype(np.int32) for t in tabs]
        keys = rng.permutation(10 ** 6)[:n_seq] * 7 + 3  # arbitrary, unordered keys
        # one slice per sequence (a step holds each sequence once), in a random order
        order = rng.permutation(n_seq)
        slices = []
        for s in order:
            cap = tabs[s].size * 16
            start = int(rng.integers(0, cap))
            ln = int(rng.integers(1, cap - start + 1))
            slices.append((int(keys[s]), start, ln, bool(rng.integers(0, 2)), tabs[s], toks[s]))
        got = oracle.pack_step(slices, 16)
        lens = np.array([sl[2] for sl in slices])
        cu = np.concatenate([[0], np.cumsum(lens)])
        # distinct sequences in first-seen order: here every slice is a new one
        rank = np.arange(len(slices))
        assert np.array_equal(got.token_seq, np.repeat(rank, lens))
        sizes = np.array([sl[4].size for sl in slices])
        assert np.array_equal(got.table_offset, np.concatenate([[0], np.cumsum(sizes)[:-1]]))
        assert np.array_equal(got.tables, np.concatenate([sl[4] for sl in slices]))
        nl = np.array([sl[3] for sl in slices], dtype=bool)
        assert np.array_equal(got.logit_rows, (cu[1:] - 1)[nl])
        assert np.array_equal(got.positions, np.concatenate([np.arange(s, s + l) for _, s, l, *_ in slices]))
        assert np.array_equal(got.token_ids, np.concatenate([t[s:s + l] for _, s, l, _, _, t in slices]))


def test_pack_step_repeated_sequence_shares_one_table():
    """Two slices of one sequence (a key seen twice): one table, one rank."""
    t = np.arange(5, dtype=np.int32) + 40
    u = np.arange(3, dtype=np.int32) + 90
    toks = np.zeros(80, np.int32)
    got = oracle.pack_step([(9, 0, 3, False, t, toks), (4, 2, 2, True, u, toks), (9, 3, 1, True, t, toks)], 16)
    assert list(got.token_seq) == [0, 0, 0, 1, 1, 0]
    assert list(got.tables) == list(t) + list(u)
    assert list(got.table_offset) == [0, 5]
    assert list(got.logit_rows) == [4, 5]


def _bf16_rne(x):
    """fp32 -> bf16 bits from the format's definition: round to nearest,
    ties to even, on the top 16 bits; NaN stays NaN (quiet bit set)."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(x)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


@pytest.mark.parametrize("cache", ["f32", "bf16"])
def test_store_kv_closed_form(cache):
    """store_kv.cu:20-36: row t of k and v lands at row slots[t] of the
    caches, tokens in order (a repeated slot keeps the last token's row),
    and no other row changes. bf16 rows are the round-to-nearest-even of
    the fp32 rows, computed here from the bit pattern."""
    rng = np.random.default_rng(5)
    n, kv_dim, slots_total = 40, 24, 128
    k = rng.standard_normal((n, kv_dim)).astype(np.float32)
    v = rng.standard_normal((n, kv_dim)).astype(np.float32)
    k[0, :4] = [np.inf, -np.inf, 0.0, -0.0]
    k[1, 0] = np.float32(1.0 + 2.0 ** -8)  # a tie between two bf16 values: rounds to even
    k[1, 1] = np.float32(1.0 + 3 * 2.0 ** -8)  # a tie that rounds up
    slots = rng.choice(slots_total, n, replace=False).astype(np.int32)
    slots[-1] = slots[3]  # a repeated slot: the later token wins
    dt = np.float32 if cache == "f32" else np.uint16
    kc = np.full((slots_total, kv_dim), 7, dt)
    vc = np.full((slots_total, kv_dim), 9, dt)
    oracle.store_kv(k, v, slots, kc, vc)
    conv = (lambda x: x) if cache == "f32" else _bf16_rne
    want_k = np.full_like(kc, 7)
    want_v = np.full_like(vc, 9)
    for t in range(n):
        want_k[slots[t]] = conv(k[t])
        want_v[slots[t]] = conv(v[t])
    assert np.array_equal(kc.view(np.uint8), want_k.view(np.uint8))
    assert np.array_equal(vc.view(np.uint8), want_v.view(np.uint8))
    if cache == "bf16":
        assert kc[slots[1], 0] == 0x3F80 and kc[slots[1], 1] == 0x3F82
