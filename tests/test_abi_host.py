"""Host-side checks of the C ABI (no GPU needed): the library loads and
exports exactly what include/llm_engine_amd.h declares, argument validation
returns the documented codes without launching anything, and the step packer
(le_plan_step) reproduces the reference's packing bit for bit on steps the
reference's own scheduler produced (tests/golden/schedule_ref.npz)."""
import ctypes
import re
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from cases import parse_trace

ROOT = Path(__file__).resolve().parent.parent


def declared_symbols():
    syms = set()
    # the C ABI headers; le_cuda_kernels.h (C++, the reference's launcher
    # names, in the bridge library) is checked by test_bridge_exports_reference_signatures
    for h in (ROOT / "include").glob("*.h"):
        if h.name == "le_cuda_kernels.h":
            continue
        text = re.sub(r"/\*.*?\*/", "", h.read_text(), flags=re.S)
        for m in re.finditer(r"^\s*(?!static)[A-Za-z_][\w\s\*]*?\b(le_\w+)\s*\(", text, flags=re.M):
            syms.add(m.group(1))
    return syms


def test_library_exports_every_declared_symbol():
    from llm_engine_amd import _lib
    lib = _lib.load()
    syms = declared_symbols()
    assert {"le_kv_cache_write", "le_attention_decode", "le_plan_step",
            "le_ragged_paged_attention"} <= syms
    for s in sorted(syms):
        assert hasattr(lib, s), s
    assert set(_lib.SIGNATURES) == syms
    assert b"gfx950" in lib.le_version()


def test_validation_codes_without_launch():
    from llm_engine_amd import _lib
    L = _lib.load()
    nul = ctypes.c_void_p(0)
    assert L.le_kv_cache_write(nul, nul, 0, nul, nul, nul, 0, 0, 128, 10, nul) == _lib.LE_OK
    assert L.le_kv_cache_write(nul, nul, 0, nul, nul, nul, 0, 4, 100, 10, nul) == _lib.LE_EUNSUPPORTED
    assert L.le_kv_cache_write(nul, nul, 0, nul, nul, nul, 0, 4, 128, 10, nul) == _lib.LE_EINVAL
    assert L.le_kv_cache_write(nul, nul, 7, nul, nul, nul, 0, 4, 128, 10, nul) == _lib.LE_EINVAL
    args = lambda qh, kvh, hd, bs: (nul, 0, nul, nul, 0, nul, nul, nul, nul, nul, 3, qh, kvh, hd, bs,
                                    0.125, 100, nul, 0, nul)
    assert L.le_attention_decode(*args(14, 2, 64, 16)) == _lib.LE_EINVAL          # null pointers
    assert L.le_attention_decode(*args(14, 3, 64, 16)) == _lib.LE_EINVAL          # heads not divisible
    assert L.le_attention_decode(*args(18, 2, 64, 16)) == _lib.LE_EUNSUPPORTED    # group 9
    assert L.le_attention_decode(*args(14, 2, 96, 16)) == _lib.LE_EUNSUPPORTED    # head_dim 96
    assert L.le_attention_decode(*args(14, 2, 64, 12)) == _lib.LE_EUNSUPPORTED    # block 12
    assert L.le_status_string(_lib.LE_ENOSPACE) == b"buffer too small"


def _plan(slices, kv=torch.bfloat16, **kw):
    from llm_engine_amd import kernels
    return kernels.Plan(slices, 14, 2, 64, 16, kv, device="cpu", pin=False, **kw)


def _items(plan, kind):
    P = plan.plan
    n, w, off = {"decode": (P.n_decode_items, 8, P.off_decode_items),
                 "chunk": (P.n_chunk_items, 9, P.off_chunk_items)}[kind]
    return plan.host.numpy()[off:off + 4 * n * w].view(np.int32).reshape(n, w)


def check_work_lists(plan, slices, bs=16):
    P = plan.plan
    dec, chk = _items(plan, "decode"), _items(plan, "chunk")
    pos = plan.host_array("positions")
    toff = plan.host_array("table_offset")
    tseq = plan.host_array("token_seq")
    # decode items: per row, [blk_begin, blk_end) ranges tile [0, pos/bs] exactly once
    rows = {}
    lengths = []
    row_bins = {}
    placed = bool(P.xcd_local) and any(int(it[5]) >= 0 for it in dec)
    for k, it in enumerate(dec):
        token, p, to, b0, b1, part, pb, npart = (int(x) for x in it)
        if npart == 0:  # padding of the fixed layout, or of the XCD placement
            assert token == -1 and b0 == b1 and (P.cfg.table_capacity > 0 or placed)
            continue
        assert p == pos[token] and to == toff[tseq[token]]
        rows.setdefault(token, []).append((b0, b1, part, pb, npart))
        lengths.append(b1 - b0)
        if part >= 0:
            row_bins.setdefault(token, set()).add(k % 8)
    if placed:  # LE_PLAN_XCD_LOCAL: a split row's partitions at indices equal modulo 8
        assert P.cfg.table_capacity == 0 and len(dec) % 8 == 0
        assert all(len(b) == 1 for b in row_bins.values())
    else:  # longest items first (the critical path starts first)
        assert lengths == sorted(lengths, reverse=True)
    for token, items in rows.items():
        items.sort()
        assert items[0][0] == 0 and items[-1][1] == pos[token] // bs + 1
        for a, b in zip(items, items[1:]):
            assert a[1] == b[0]
        npart = items[0][4]
        assert len(items) == npart
        if npart == 1:
            assert items[0][2] == -1
        else:
            assert sorted(i[2] for i in items) == list(range(items[0][3], items[0][3] + npart))
    # chunk items: each tile's partitions tile the keys up to its last row,
    # numbered 0..J-1 in key order, with part0 = base + j
    tiles, tile_bins = {}, {}
    for k, it in enumerate(chk):
        tb, nq, b0, b1, p0, stride, seq, part, live = (int(x) for x in it)
        if nq == 0:  # padding that keeps split tiles on one XCD
            assert b0 == b1 and p0 == -1
            continue
        assert 1 <= nq <= 32 and all(pos[tb + r] == pos[tb] + r for r in range(nq))
        # live keys from the partition's first key: whole blocks, except that
        # the partition holding the tile's last position stops just past it
        assert live == min((b1 - b0) * bs, pos[tb + nq - 1] + 1 - b0 * bs) and live >= 1
        tiles.setdefault(tb, []).append((b0, b1, p0, stride, nq, part))
        if p0 >= 0:  # a split tile's partitions sit at indices equal modulo 8 (one XCD)
            tile_bins.setdefault(tb, set()).add(k % 8)
    assert all(len(b) == 1 for b in tile_bins.values())
    if tile_bins:
        assert len(chk) % 8 == 0
    for tb, items in tiles.items():
        items.sort()
        nq, J = items[0][4], items[0][3]
        assert items[0][0] == 0 and items[-1][1] == pos[tb + nq - 1] // bs + 1
        for a, b in zip(items, items[1:]):
            assert a[1] == b[0]
        assert [i[5] for i in items] == list(range(len(items)))
        if len(items) == 1:
            assert items[0][2] == -1
        else:
            assert J == len(items) and len({i[2] - i[5] for i in items}) == 1
    # every work item's block ids, at the shared stride: decode items, then chunk items
    stride = P.decode_ids_stride
    ids = plan.host.numpy()[P.off_decode_ids:P.off_decode_ids + 4 * (len(dec) + len(chk)) * stride]
    ids = ids.view(np.int32).reshape(len(dec) + len(chk), stride)
    tables = plan.host_array("tables")
    for k, it in enumerate(dec):
        b0, b1, to = int(it[3]), int(it[4]), int(it[2])
        assert list(ids[k, :b1 - b0]) == list(tables[to + b0:to + b1]) and (ids[k, b1 - b0:] == -1).all()
    for k, it in enumerate(chk):
        b0, b1, seq = int(it[2]), int(it[3]), int(it[6])
        to = int(toff[seq])
        row = ids[len(dec) + k]
        assert list(row[:b1 - b0]) == list(tables[to + b0:to + b1]) and (row[b1 - b0:] == -1).all()
    assert P.n_combine_items == 0
    # every partial index is owned exactly once
    owned = []
    for it in dec:
        if it[5] >= 0:
            owned.append(int(it[5]))
    for it in chk:
        if it[4] >= 0:
            owned += [int(it[4]) + r * int(it[5]) for r in range(int(it[1]))]
    if P.cfg.table_capacity > 0:  # fixed layout: each row owns a fixed slot range, some unused
        assert len(set(owned)) == len(owned) and all(0 <= o < P.n_parts for o in owned)
    else:
        assert sorted(owned) == list(range(P.n_parts))


TRACES = np.load(ROOT / "tests" / "golden" / "schedule_ref.npz")
TRACE_NAMES = sorted({k.split(".")[0] for k in TRACES.files})


@pytest.mark.parametrize("name", TRACE_NAMES)
@pytest.mark.parametrize("kv", [torch.bfloat16, torch.float32])
def test_packer_matches_reference_on_scheduler_steps(name, kv):
    """Every step the reference Scheduler built (fragmented pool, chunked
    prefill, preemption, token budget, prefix caching): token ids, positions,
    int32 slots, token->sequence, concatenated tables + offsets and logit rows
    equal the reference packing (restated in the oracle, cuda_model.cu:434-491);
    cu_seqlens/seq_lens and the work lists are consistent."""
    from llm_engine_amd.kernels import Slice
    steps, toks = parse_trace(TRACES[f"{name}.trace"])
    assert len(steps) > 3
    for st in steps:
        slices = [Slice(sid, start, ln, bool(nl), blocks, toks[sid]) for sid, start, ln, nl, pf, blocks in st]
        plan = _plan(slices, kv=kv)
        want = oracle.pack_step([(s.seq_key, s.start, s.len, s.needs_logits, s.blocks, s.tokens)
                                 for s in slices], 16)
        for f in ("token_ids", "positions", "slots", "token_seq", "tables", "table_offset", "logit_rows"):
            assert np.array_equal(plan.host_array(f), getattr(want, f)), (name, f)
        cu = plan.host_array("cu_seqlens_q")
        assert np.array_equal(np.diff(cu), [s.len for s in slices])
        assert np.array_equal(plan.host_array("seq_lens_k"), [s.start + s.len for s in slices])
        check_work_lists(plan, slices)


@pytest.mark.parametrize("name", TRACE_NAMES[:6])
def test_xcd_local_placement_on_scheduler_steps(name):
    """LE_PLAN_XCD_LOCAL: the same steps with every split row's and tile's
    partitions placed at item indices equal modulo 8 (one XCD), the work
    lists otherwise as without the flag; ignored by fixed layouts."""
    from llm_engine_amd._lib import LE_PLAN_XCD_LOCAL
    from llm_engine_amd.kernels import Slice
    steps, toks = parse_trace(TRACES[f"{name}.trace"])
    seen_split = False
    for st in steps:
        slices = [Slice(sid, start, ln, bool(nl), blocks, toks[sid]) for sid, start, ln, nl, pf, blocks in st]
        for part in (0, 64):  # the planner's partitions, and 64-token ones (many split rows)
            plan = _plan(slices, flags=LE_PLAN_XCD_LOCAL, partition_tokens=part)
            assert plan.plan.xcd_local == 1
            check_work_lists(plan, slices)
            seen_split |= plan.plan.n_parts > 0
    assert seen_split
    dec = [Slice(i, 300 + 50 * i, 1, True, np.arange(40 * i, 40 * i + 40, dtype=np.int32),
                 np.zeros(640, np.int32)) for i in range(6)]
    fixed = _plan(dec, flags=LE_PLAN_XCD_LOCAL, partition_tokens=128, table_capacity=64)
    assert fixed.plan.xcd_local == 0


def test_slot_closed_form_and_fragmentation():
    """kv_cache.h:29-31 on a fragmented table (test_block_allocator.cpp:39)."""
    from llm_engine_amd.kernels import Slice
    rng = np.random.default_rng(3)
    blocks = rng.permutation(4096)[:40].astype(np.int32)
    toks = np.arange(640, dtype=np.int32)
    plan = _plan([Slice(1, 0, 640, True, blocks, toks)], kv=torch.float32)
    p = np.arange(640)
    assert np.array_equal(plan.host_array("slots"), blocks[p // 16] * 16 + p % 16)


def test_plan_errors():
    from llm_engine_amd import _lib
    from llm_engine_amd.kernels import Slice
    with pytest.raises(ValueError):  # position 32 has no block
        _plan([Slice(1, 0, 33, True, np.array([3, 4], np.int32), np.zeros(33, np.int32))])
    # an empty step packs to an empty plan
    plan = _plan([])
    assert plan.plan.n_tokens == 0 and plan.plan.n_decode_items == 0


def test_plan_rejects_slices_outgrowing_their_sequence_table():
    """Slices that share a sequence key share the first slice's table (one
    Sequence, one table). A later slice whose positions need more blocks than
    that table holds is rejected (its slots would otherwise be read past the
    table), whatever table it carries itself."""
    from llm_engine_amd.kernels import Slice
    toks = np.zeros(200, np.int32)
    short = np.array([5], np.int32)
    long = np.arange(10, dtype=np.int32)
    with pytest.raises(ValueError):
        _plan([Slice(7, 0, 1, False, short, toks), Slice(7, 150, 1, True, long, toks)])
    # the same two slices under distinct keys are fine
    plan = _plan([Slice(7, 0, 1, False, short, toks), Slice(8, 150, 1, True, long, toks)])
    assert plan.plan.n_seqs == 2
    assert list(plan.host_array("slots")) == [5 * 16, 9 * 16 + 150 % 16]


def test_bridge_exports_reference_signatures():
    """libllm_engine_amd_bridge.so exports all nine of the reference's
    launcher names with its argument lists (cuda_kernels.h:17-64, __half
    buffers, fp32 weights/bias/tables, hipStream_t), plus the registration
    calls declared in include/le_cuda_kernels.h."""
    import subprocess
    lib = ROOT / "llm-engine_amd" / "lib" / "libllm_engine_amd_bridge.so"
    ctypes.CDLL(str(lib))
    syms = subprocess.run(["nm", "-DC", str(lib)], capture_output=True, text=True, check=True).stdout
    h = "__half const*"
    want = [
        f"engine::launch_store_kv({h}, {h}, int const*, __half*, __half*, int, int, ihipStream_t*)",
        f"engine::launch_attention_decode({h}, {h}, {h}, int const*, int const*, int const*, int const*, "
        "__half*, int, int, int, int, int, float, ihipStream_t*)",
        f"engine::launch_attention_decode_gqa({h}, {h}, {h}, int const*, int const*, int const*, int const*, "
        "__half*, int, int, int, int, int, float, ihipStream_t*)",
        "engine::le_bridge_set_workspace(void*, unsigned long)",
        "engine::le_bridge_set_cache_slots(long)",
        "engine::le_bridge_set_rope_positions(int)",
        f"engine::launch_embedding({h}, int const*, __half*, int, int, ihipStream_t*)",
        f"engine::launch_rmsnorm({h}, float const*, __half*, int, int, float, ihipStream_t*)",
        f"engine::launch_silu_mul(__half*, {h}, unsigned long, ihipStream_t*)",
        "engine::launch_rope(__half*, int const*, float const*, float const*, int, int, int, int, ihipStream_t*)",
        f"engine::launch_add_inplace(__half*, {h}, unsigned long, ihipStream_t*)",
        "engine::launch_add_bias(__half*, float const*, int, int, ihipStream_t*)",
    ]
    for w in want:
        assert w in syms, w


def test_noalloc_rejects_steps_beyond_its_scratch():
    """A step whose workspace exceeds the static scratch is rejected before
    anything runs (LE_ETOOLARGE); an empty step is a no-op."""
    from llm_engine_amd import _lib
    from llm_engine_amd.kernels import Plan, Slice
    L = _lib.load()
    cap = int(L.le_noalloc_scratch_bytes())
    assert cap == 32 << 20
    # 512 rows of 8192 keys in 128-token partitions: 64 partials per row
    rng = np.random.default_rng(1)
    sl = [Slice(i, 8191, 1, True, rng.permutation(100000)[:512].astype(np.int32), np.zeros(8192, np.int32))
          for i in range(512)]
    plan = Plan(sl, 32, 4, 128, 16, torch.bfloat16, partition_tokens=128, device="cpu", pin=False)
    assert plan.workspace_size() > cap
    nul = ctypes.c_void_p(0)
    assert L.le_ragged_paged_attention_noalloc(nul, 0, nul, nul, 1, 100000, ctypes.byref(plan.plan), 0.125,
                                               nul, nul) == _lib.LE_ETOOLARGE
    empty = Plan([], 14, 2, 64, 16, torch.bfloat16, device="cpu", pin=False)
    assert L.le_ragged_paged_attention_noalloc(nul, 0, nul, nul, 1, 100, ctypes.byref(empty.plan), 0.125,
                                               nul, nul) == _lib.LE_OK


def test_fixed_layout_is_constant_across_decode_steps():
    """table_capacity > 0: a decode step's plan has one layout for a given row
    count (every array offset, the item and partial counts, the id stride),
    however the contexts grow, so launches captured in a HIP graph replay
    for later steps; the values are still the reference packing's."""
    from llm_engine_amd.kernels import Slice
    rng = np.random.default_rng(7)
    cap, n = 128, 24
    blocks = [rng.permutation(5000)[:cap].astype(np.int32) for _ in range(n)]
    ctx = rng.integers(1, 1500, n)
    layout = None
    for step in range(40):
        c = ctx + step * 13  # crosses block and partition boundaries
        sl = [Slice(100 + i, int(c[i]) - 1, 1, True, blocks[i][:(int(c[i]) + 15) // 16],
                    np.arange(int(c[i]), dtype=np.int32)) for i in range(n)]
        plan = _plan(sl, partition_tokens=512, table_capacity=cap)
        P = plan.plan
        key = (P.bytes, P.n_decode_items, P.n_parts, P.decode_ids_stride, P.n_table) + tuple(
            getattr(P, f) for f, _ in type(P)._fields_ if f.startswith("off_"))
        layout = layout or key
        assert key == layout, step
        want = oracle.pack_step([(s.seq_key, s.start, s.len, s.needs_logits, s.blocks, s.tokens) for s in sl], 16)
        for f in ("token_ids", "positions", "slots", "token_seq", "logit_rows"):
            assert np.array_equal(plan.host_array(f), getattr(want, f)), f
        tab = plan.host_array("tables").reshape(n, cap)
        for i, s in enumerate(sl):
            assert np.array_equal(tab[i, :len(s.blocks)], s.blocks) and (tab[i, len(s.blocks):] == -1).all()
        assert list(plan.host_array("table_offset")) == [i * cap for i in range(n)]
        check_work_lists(plan, sl)
    with pytest.raises(ValueError):  # prefill chunks have no fixed layout
        _plan([Slice(1, 0, 5, True, blocks[0][:1], np.zeros(5, np.int32))], partition_tokens=512, table_capacity=cap)


def test_fixed_layout_accepts_skewed_decode_batches():
    """Decode steps with a few full-length rows among many short ones (the
    engine's graph-replay layout: partitions of 1024 tokens, block 16) plan
    in the fixed layout for every table capacity and partition size: the
    item list is rows * partitions-per-row long, so no mix of lengths can
    overflow it. Seeded random batches as well."""
    from llm_engine_amd.kernels import Slice
    rng = np.random.default_rng(11)

    def step(lens, cap):
        return [Slice(100 + i, int(c) - 1, 1, True, rng.permutation(20000)[:(int(c) + 15) // 16].astype(np.int32),
                      np.arange(int(c), dtype=np.int32)) for i, c in enumerate(lens)]

    cases = [([128 * 16] * 7 + [6] * 16, 128, 1024)]  # the reported batch: 7 full rows, 16 at pos 5
    for _ in range(60):
        cap = int(rng.choice([32, 64, 128, 256]))
        part = int(rng.choice([256, 512, 640, 1024, 2048]))
        n = int(rng.integers(1, 80))
        n_long = int(rng.integers(0, n + 1))
        lens = [cap * 16 if i < n_long else int(rng.integers(1, 40)) for i in range(n)]
        rng.shuffle(lens)
        cases.append((lens, cap, part))
    for lens, cap, part in cases:
        sl = step(lens, cap)
        plan = _plan(sl, partition_tokens=part, table_capacity=cap)
        check_work_lists(plan, sl)
        parts_cap = -(-cap // -(-part // 16))
        assert plan.plan.n_decode_items == len(lens) * min(parts_cap, 1024 // 7)


@pytest.mark.parametrize("bs", [8, 16, 32])
def test_plan_fuzz_accepts_exactly_the_valid_steps(bs):
    """Random steps, valid and not: sequences whose keys repeat across
    slices, tables shorter than a slice's positions, empty tables, negative
    starts and lengths, chunk and decode slices mixed. le_plan_step accepts
    exactly the steps whose every slice has a block for each of its positions
    in its own table and in its sequence's first table (one table per
    sequence), and rejects the rest with LE_EINVAL, never reading past a
    table; every accepted step packs as the oracle packer does (slots by the
    closed form of kv_cache.h:29-31 through the first slice's table) with
    consistent work lists."""
    from llm_engine_amd.kernels import Slice
    rng = np.random.default_rng(1000 + bs)
    toks = rng.integers(0, 32000, size=4096).astype(np.int32)
    n_ok = n_bad = 0
    for case in range(300):
        n_keys = int(rng.integers(1, 6))
        tables = {k: rng.permutation(2048)[:int(rng.integers(0, 12))].astype(np.int32) for k in range(n_keys)}
        slices, first_nb, valid = [], {}, True
        for _ in range(int(rng.integers(1, 8))):
            key = int(rng.integers(0, n_keys))
            nb = tables[key].size
            # a table of its own that sometimes differs from the first slice's
            own = tables[key] if rng.random() < 0.8 else rng.permutation(2048)[:int(rng.integers(0, 14))].astype(np.int32)
            cap = max(own.size * bs, 1)
            ln = 1 if rng.random() < 0.5 else int(rng.integers(-1, min(cap, 200) + 2))
            start = int(rng.integers(-1, cap + 2)) if rng.random() < 0.1 else int(rng.integers(0, max(cap - max(ln, 1), 0) + 2))
            if ln <= 0 or start < 0:
                valid = False
            else:
                last = start + ln - 1
                if last // bs >= own.size:
                    valid = False
                if key in first_nb and last // bs >= first_nb[key]:
                    valid = False
            first_nb.setdefault(key, own.size)
            slices.append(Slice(key, start, ln, bool(rng.random() < 0.7), own, toks))
        try:
            plan = kernels_plan(slices, bs)
        except ValueError:
            assert not valid, (case, [(s.seq_key, s.start, s.len, s.blocks.size) for s in slices])
            n_bad += 1
            continue
        assert valid, (case, [(s.seq_key, s.start, s.len, s.blocks.size) for s in slices])
        n_ok += 1
        want = oracle.pack_step([(s.seq_key, s.start, s.len, s.needs_logits, s.blocks, s.tokens)
                                 for s in slices], bs)
        for f in ("token_ids", "positions", "slots", "token_seq", "tables", "table_offset", "logit_rows"):
            assert np.array_equal(plan.host_array(f), getattr(want, f)), (case, f)
        # slots by the closed form, through each sequence's first table
        firsts = {}
        for s in slices:
            firsts.setdefault(s.seq_key, s.blocks)
        slots = np.concatenate([firsts[s.seq_key][(s.start + np.arange(s.len)) // bs] * bs
                                + (s.start + np.arange(s.len)) % bs for s in slices])
        assert np.array_equal(plan.host_array("slots"), slots)
        check_work_lists(plan, slices, bs=bs)
    assert n_ok > 50 and n_bad > 50


def kernels_plan(slices, bs):
    from llm_engine_amd import kernels
    return kernels.Plan(slices, 14, 2, 64, bs, torch.bfloat16, device="cpu", pin=False)


def test_auto_partition_fits_one_round_at_two_per_cu():
    """The automatic decode partition (partition_tokens 0): at least 640 keys
    and a multiple of 128, grown until the step's workgroups (items x kv
    heads, placement padding aside) fit 512, two per CU, unless it reaches
    4096; and never grown past the first size that fits."""
    from llm_engine_amd import kernels
    from llm_engine_amd.kernels import Slice
    rng = np.random.default_rng(11)
    for trial in range(40):
        qh, kvh = [(14, 2), (32, 4), (32, 8), (16, 16)][trial % 4]
        n = int(rng.integers(1, 200))
        lens = rng.integers(1, int(rng.choice([600, 1400, 5000, 20000])), size=n)
        blocks = [np.arange((l + 15) // 16, dtype=np.int32) for l in lens]
        sl = [Slice(i, int(l) - 1, 1, True, blocks[i], np.zeros(int(l), np.int32)) for i, l in enumerate(lens)]
        plan = kernels.Plan(sl, qh, kvh, 64, 16, torch.bfloat16, device="cpu", pin=False)
        part = plan.plan.cfg.partition_tokens
        assert part >= 640 and part % 128 == 0 and part <= 4096

        def items(pt):
            pb = (pt + 15) // 16
            return sum(min(-(-((int(l) - 1) // 16 + 1) // pb), max(1, 1024 // (qh // kvh))) for l in lens)
        assert plan.plan.n_decode_items == items(part)
        if part < 4096:
            assert items(part) * kvh <= 512
        if part > 640 and items(part - 128) * kvh <= 512:
            # grown only past sizes that did not fit: the first rule's size
            ctx = int(lens.sum())
            first = max(640, -(-(-(-ctx // max(1, 512 // kvh))) // 128) * 128)
            assert part == min(first, 4096)
