"""Benchmark of the ragged paged-attention hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--kv bf16|f32]
                    [--workload config2|target|config3] [--no-cpu-baseline]
                    [--e2e decode64|config4|config5|all|none]

A step is one decode pass of the hot path over one ragged batch, for every
layer of the model: the packed step metadata is uploaded once (one async
copy), then per layer the new K/V rows are scattered into that layer's paged
cache and ragged paged attention runs over the batch -- one launch per layer
(le_ragged_paged_attention_store; --separate-scatter runs le_kv_cache_write
then the attention). Each layer has its own KV pool, so a step touches 24
distinct caches (>> the 256 MB Infinity Cache). The step is captured once as
a HIP graph and replayed (the engine replays its decode steps the same way);
--eager-step launches it from Python instead (about 5 % slower on config 2,
the host's launch cost).

Workloads (Qwen2.5-0.5B GQA: 14 q heads, 2 kv heads, head_dim 64, block 16):
  config2  64 seqs, context log-uniform in [64, 4096], tables from a
           32768-block pool (benchmark config 2) -- the default
  target   64 seqs x 4096 context (the >= 60 % of HBM peak target point)
  config3  32 decode rows + 2 prefill chunks of 512 (MFMA chunk rows)

After the attention measurement, an end-to-end leg runs the whole engine
(scheduler, packing, device model, greedy) on TinyLlama-1.1B with bf16
weights and K/V (benchmark config 4 shape) and reports decode tok/s at
64 sequences under "e2e_decode64"; --e2e config4 / config5 / all run the
Poisson serving workload and the shared-prefix + preemption stress instead
or as well.

A config2 run also measures the target point (bf16 and fp32 K/V) and
config3 the same way (fewer steps) and reports them under "target",
"target_f32" and "config3", each with its own roofline ("config3" adds the
chunk rows' MFMA flops and utilisation).
"plan.pack_us" is the steady-state host cost of le_plan_step on the step
(sizing + packing call); the e2e legs report "plan_us_per_step", the C++
engine's own timing of le_plan_step + le_plan_upload per step.

Prints ONE JSON line. `value` is algorithmic HBM bytes per step / step time:
K/V of each kv head once (the GQA-shared minimum), q, out, block tables and
per-row metadata, plus the K/V rows written by the scatter.
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "llm-engine_amd", ROOT / "tests", ROOT / "oracle"):
    sys.path.insert(0, str(p))

METRIC = "ragged paged-attn HBM GB/s (% of peak); decode tok/s at 64 seqs, 1 GPU"
HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
Q_HEADS, KV_HEADS, HEAD_DIM, BS = 14, 2, 64, 16
LAYERS = 24


def workload_shape(name: str):
    rng = np.random.default_rng(2)
    if name == "config2":
        from cases import loguniform_ctx
        ctx = loguniform_ctx(rng, 64, 64, 4096)
        return ctx, np.ones(64, dtype=np.int64), 32768
    if name == "target":
        return np.full(64, 4096, dtype=np.int64), np.ones(64, dtype=np.int64), 32768
    if name == "config3":
        dec = np.random.default_rng(3).integers(256, 2049, size=32)
        ctx = np.array([512, 1536] + list(dec), dtype=np.int64)
        return ctx, np.array([512, 512] + [1] * 32, dtype=np.int64), 16384
    raise SystemExit(f"unknown workload {name}")


def algorithmic_bytes(ctx, q_len, kv_size, act_size):
    """HBM bytes one layer of the step must move at minimum."""
    n = int(q_len.sum())
    kv = int(ctx.sum()) * KV_HEADS * HEAD_DIM * 2 * kv_size          # K and V, once per kv head
    qo = n * Q_HEADS * HEAD_DIM * act_size * 2                         # q in, out
    tables = int(((ctx + BS - 1) // BS).sum()) * 4
    meta = n * 4 * 2 + len(ctx) * 4                                    # token pos/seq, table offsets
    attn = kv + qo + tables + meta
    write = n * KV_HEADS * HEAD_DIM * 2 * (act_size + kv_size) + n * 4  # scatter: read rows, write cache
    return attn, write


def chunk_flops(ctx, q_len):
    f = 0
    for c, ql in zip(ctx, q_len):
        if ql > 1:
            keys = np.arange(c - ql, c) + 1
            f += int(keys.sum())
    return 4 * Q_HEADS * HEAD_DIM * f


def measured_traffic(workload: str, kv: str):
    """HBM bytes per attention launch from the committed rocprofv3 PMC summary
    (profiles/traffic.json: FETCH_SIZE and WRITE_SIZE of the decode kernel,
    scaled by the factors a plain copy of known size gives), or None."""
    f = ROOT / "profiles" / "traffic.json"
    if not f.exists():
        return None
    d = json.loads(f.read_text()).get(f"{workload}/{kv}")
    return None if d is None else int(d["traffic_bytes"])


def cpu_baseline(ctx, q_len, kv_bf16: bool, budget_s: float):
    """The oracle's (token, head) loop (cpu_model.cpp:160-185) on the host
    cores, on one layer of the same batch, repeated until budget_s elapses."""
    import oracle
    from cases import make_case
    case = make_case(ctx, q_len=q_len, num_blocks=int(((ctx + BS - 1) // BS).sum()) + 64,
                     seed=21, kv_bf16=kv_bf16)
    threads = oracle.threads_default()
    attn_bytes, _ = algorithmic_bytes(ctx, q_len, 2 if kv_bf16 else 4, 4)

    def rate(n_threads, budget):
        reps, t0 = 0, time.perf_counter()
        while True:
            oracle.paged_attention(case.q, case.k_cache, case.v_cache, case.tables, case.table_offset,
                                   case.token_seq, case.token_pos, Q_HEADS, KV_HEADS, HEAD_DIM, BS,
                                   case.scale, threads=n_threads)
            reps += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return attn_bytes * reps / el / 1e9, reps, el

    value, reps, el = rate(threads, budget_s)
    one, reps1, el1 = rate(1, budget_s / 4)  # the same loop on one thread
    return {"value": round(value, 3), "unit": "GB/s", "cores": threads,
            "kind": "port", "value_1_thread": round(one, 3),
            "sample": f"{reps} layer(s) of the same batch (one layer's attention, "
                      f"{'bf16' if kv_bf16 else 'fp32'} K/V), {el:.1f} s, oracle.c "
                      f"(token, head) loop on {threads} threads; then {reps1} layer(s) "
                      f"in {el1:.1f} s on 1 thread (value_1_thread)"}


def cpu_e2e_decode_baseline(budget_s: float = 3.0):
    """End-to-end decode on the host cores: the oracle's model forward (a
    restatement of the reference CPU backend, cpu_model.cpp:98-214, naive
    threaded GEMMs, bf16 K/V) on one 64-row decode step of the decode64 leg's
    shape (TinyLlama-1.1B, contexts = prompts U[128, 1024] plus up to 256
    generated tokens, block 16). Its caches are filled directly (no CPU
    prefill); a bounded sample times the step with 1 and with 4 layers, and
    the 22-layer step is the 1-layer step plus 21 times the per-layer
    difference. The
    weights' and caches' values do not change the time of naive GEMMs and the
    attention loop, so both are filled from a small random block (N(0, 0.02)
    weights, N(0, 1) bf16 K/V) rather than drawn in full."""
    import oracle
    from e2e_util import OracleModel
    from llm_engine_amd import _lib
    from llm_engine_amd.engine import ARCHS, Weights
    rng = np.random.default_rng(9)
    wtile = (rng.standard_normal(1 << 20, dtype=np.float32) * np.float32(0.02))

    def filled(*shape):
        return np.resize(wtile, shape).astype(np.float32)

    def weights(nl):
        a = dict(ARCHS["tinyllama-1.1b"], layers=nl)
        H, I, V = a["hidden"], a["inter"], a["vocab"]
        QD, KVD = a["q_heads"] * a["head_dim"], a["kv_heads"] * a["head_dim"]
        w = Weights(a, filled(V, H), np.ones(H, np.float32), None if a["tie"] else filled(V, H))
        for _ in range(nl):
            L = dict(wq=filled(QD, H), wk=filled(KVD, H), wv=filled(KVD, H), wo=filled(H, QD),
                     wgate=filled(I, H), wup=filled(I, H), wdown=filled(H, I),
                     in_norm=np.ones(H, np.float32), post_norm=np.ones(H, np.float32))
            if a["qkv_bias"]:
                L.update(bq=np.zeros(QD, np.float32), bk=np.zeros(KVD, np.float32), bv=np.zeros(KVD, np.float32))
            w.layers.append(L)
        return w

    S = 64
    ctx = rng.integers(128, 1025, S) + rng.integers(0, 257, S)
    nb = (ctx + BS - 1) // BS
    pool = int(nb.sum()) + 64
    perm = rng.permutation(pool).astype(np.int32)
    tables = np.split(perm[:int(nb.sum())], np.cumsum(nb)[:-1])
    tables = [np.ascontiguousarray(t) for t in tables]
    toks = [rng.integers(0, 32000, int(c)).astype(np.int32) for c in ctx]
    step = [_lib.StepSlice(s, int(ctx[s]) - 1, 1, 1, int(nb[s]), tables[s].ctypes.data, toks[s].ctypes.data)
            for s in range(S)]
    tile = oracle.f32_to_bf16(rng.standard_normal(1 << 20, dtype=np.float32))
    per_step = {}
    for nl in (1, 4):
        om = OracleModel(weights(nl), pool, BS, kv_bf16=True)
        for c in om.kc + om.vc:
            c.reshape(-1)[:] = np.resize(tile, c.size)
        om.logits(step)  # warm-up
        reps, t0 = 0, time.perf_counter()
        while reps < 2 or time.perf_counter() - t0 < budget_s / 2:
            om.logits(step)
            reps += 1
        per_step[nl] = ((time.perf_counter() - t0) / reps, reps)
        del om
    t1, t4 = per_step[1][0], per_step[4][0]
    t22 = t1 + 21 * (t4 - t1) / 3
    threads = oracle.threads_default()
    return {"decode_tok_per_s": round(S / t22, 2), "unit": "tok/s", "cores": threads, "kind": "port",
            "sample": f"64-row decode steps at contexts {int(ctx.min())}-{int(ctx.max())}, oracle.c model forward "
                      f"on {threads} threads: 1 layer {t1:.3f} s/step ({per_step[1][1]} steps), 4 layers "
                      f"{t4:.3f} s/step ({per_step[4][1]} steps); 22 layers estimated {t22:.2f} s/step"}


def pack_cost_us(slices, kv_dt, reps=200):
    """Steady-state host cost of le_plan_step on a step's slices (the
    sized call and the packing call, as the engine makes them each step),
    timed over `reps` calls through ctypes into a pinned buffer."""
    import ctypes
    from llm_engine_amd import _lib, kernels
    plan = kernels.Plan(slices, Q_HEADS, KV_HEADS, HEAD_DIM, BS, kv_dt)
    L = _lib.load()
    arr = (_lib.StepSlice * max(1, len(slices)))()
    keep = []
    for i, s in enumerate(slices):
        b = np.ascontiguousarray(s.blocks, dtype=np.int32)
        tk = np.ascontiguousarray(s.tokens, dtype=np.int32)
        keep += [b, tk]
        arr[i] = _lib.StepSlice(s.seq_key, s.start, s.len, int(s.needs_logits), b.size, b.ctypes.data, tk.ctypes.data)
    P = _lib.StepPlan()
    buf = ctypes.c_void_p(plan.host.data_ptr())
    t0 = time.perf_counter()
    for _ in range(reps):
        L.le_plan_step(arr, len(slices), ctypes.byref(plan.cfg), None, 0, ctypes.byref(P))
        L.le_plan_step(arr, len(slices), ctypes.byref(plan.cfg), buf, int(plan.plan.bytes), ctypes.byref(P))
    return (time.perf_counter() - t0) / reps * 1e6


_ARENA = {}


def kv_arena(nbytes: int, dev):
    """One byte buffer per device for the legs' K/V pools, grown (reallocated)
    only when a leg needs more than any before it (main sizes it for the
    largest leg of the run before the first one)."""
    import torch
    a = _ARENA.get(str(dev))
    if a is None or a.numel() < nbytes:
        _ARENA.pop(str(dev), None)
        a = _ARENA[str(dev)] = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    return a


def attention_leg(workload, kv, L, steps, warmup, partition=0, chunk_partition=0, graph=False,
                  separate_scatter=False, flags=0, step_graph=True):
    """The hot path over one workload for L layers per step (see the module
    docstring); returns the fields of the JSON line for it. The step is
    replayed from a captured HIP graph (step_graph, as the engine replays its
    decode steps; eagerly launched otherwise), and the attention-only loop
    behind `roofline` is launched eagerly unless `graph`, which replays it
    from a graph as well."""
    import torch
    from llm_engine_amd import kernels
    from gpu_util import slices_of
    from cases import make_case

    dev = torch.device("cuda:0")
    kv_dt = torch.bfloat16 if kv == "bf16" else torch.float32
    act_dt = torch.float32
    ctx, q_len, pool = workload_shape(workload)
    case = make_case(ctx, q_len=q_len, num_blocks=pool, seed=2, fill="none")  # tables and rows only
    kv_dim = KV_HEADS * HEAD_DIM
    n = int(q_len.sum())
    g = torch.Generator(device=dev)
    g.manual_seed(1234)
    # The K/V pools live in one arena allocated once per process and reused by
    # every leg, as the engine's model allocates its pools at start-up (one
    # allocation for all layers). With a pair of allocations per layer and
    # leg, a leg that allocated after an earlier leg freed its pools measured
    # up to 3.5 % slower (64 x 4096: 29.5 against 28.5 us per launch); the
    # arena also runs that point at 28.0 us.
    pool_elems = pool * BS * kv_dim
    esz = torch.empty((), dtype=kv_dt).element_size()
    arena = kv_arena(2 * L * pool_elems * esz, dev)
    pools = arena[:2 * L * pool_elems * esz].view(kv_dt).view(2 * L, pool * BS, kv_dim)
    for i in range(2 * L):
        pools[i].normal_(generator=g)
    kc = [pools[2 * l] for l in range(L)]
    vc = [pools[2 * l + 1] for l in range(L)]
    qs = [torch.randn(n, Q_HEADS * HEAD_DIM, device=dev, generator=g).to(act_dt) for _ in range(L)]
    knew = [torch.randn(n, kv_dim, device=dev, generator=g).to(act_dt) for _ in range(L)]
    vnew = [torch.randn(n, kv_dim, device=dev, generator=g).to(act_dt) for _ in range(L)]
    outs = [torch.empty_like(qs[0]) for _ in range(L)]

    slices = slices_of(case)
    plan = kernels.Plan(slices, Q_HEADS, KV_HEADS, HEAD_DIM, BS, kv_dt,
                        partition_tokens=partition, chunk_partition_tokens=chunk_partition, flags=flags)
    pack_us = pack_cost_us(slices, kv_dt)
    plan.upload()
    torch.cuda.synchronize()
    slots = plan.dev_array("slots")
    ws = kernels.new_workspace(plan.workspace_size(), dev)
    stream = torch.cuda.current_stream()
    if graph or step_graph:
        stream = torch.cuda.Stream()  # capture needs a stream other than the legacy default
        stream.wait_stream(torch.cuda.current_stream())

    def attn(l, st=None):
        kernels.ragged_paged_attention(qs[l], kc[l], vc[l], plan, case.scale, out=outs[l],
                                       workspace=ws, stream=st or stream)

    def eager_step():
        plan.upload(stream)
        for l in range(L):
            if separate_scatter:
                kernels.store_kv(knew[l], vnew[l], slots, kc[l], vc[l], stream=stream)
                attn(l)
            else:  # le_ragged_paged_attention_store: the scatter folded into the attention launch
                kernels.ragged_paged_attention(qs[l], kc[l], vc[l], plan, case.scale, out=outs[l],
                                               workspace=ws, stream=stream, k_new=knew[l], v_new=vnew[l])

    step = eager_step
    if graph or step_graph:
        # The whole step (upload + L x (scatter, attention)) as one HIP graph,
        # replayed per step. Nothing in it allocates or clears memory: the
        # workspace counters reset themselves.
        with torch.cuda.stream(stream):
            eager_step()
            hg = torch.cuda.CUDAGraph()
            with torch.cuda.graph(hg, stream=stream):
                eager_step()
        step = hg.replay

    with torch.cuda.stream(stream):
        for _ in range(warmup):
            step()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    with torch.cuda.stream(stream):
        e0.record(stream)
        for _ in range(steps):
            step()
        e1.record(stream)
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps

    kv_size = 2 if kv_dt == torch.bfloat16 else 4
    attn_b, write_b = algorithmic_bytes(ctx, q_len, kv_size, 4)
    step_bytes = L * (attn_b + write_b)
    value = step_bytes / (ms * 1e-3) / 1e9

    # Dominant kernel alone: the attention call per layer, back to back, timed
    # with events on the stream it is launched on.
    reps = max(4, steps // 2)
    attn_loop = lambda: [attn(l) for l in range(L)]
    if graph:
        with torch.cuda.stream(stream):
            agraph = torch.cuda.CUDAGraph()
            with torch.cuda.graph(agraph, stream=stream):
                attn_loop()
        attn_loop = agraph.replay
    a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    with torch.cuda.stream(stream):
        attn_loop()
        a0.record(stream)
        for _ in range(reps):
            attn_loop()
        a1.record(stream)
    torch.cuda.synchronize()
    attn_us = a0.elapsed_time(a1) * 1e3 / (reps * L)
    achieved = attn_b / (attn_us * 1e-6) / 1e9
    P = plan.plan
    roofline = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                "traffic": measured_traffic(workload, kv) if partition == 0 and chunk_partition == 0 else None,
                "kernel": "le_ragged_paged_attention ("
                          + ("ragged_kernel: chunk and decode workgroups in one launch"
                             if P.n_chunk_items and P.n_decode_items else
                             "chunk_kernel" if P.n_chunk_items else "decode mfma_kernel") + ")",
                "bytes_per_launch": attn_b, "us_per_launch": round(attn_us, 3)}
    if workload == "config3":
        fl = chunk_flops(ctx, q_len)
        tflops = fl / (attn_us * 1e-6) / 1e12
        roofline["chunk_flops_per_launch"] = fl
        roofline["chunk_tflops"] = round(tflops, 1)
        roofline["mfma_bf16_util"] = round(tflops / MFMA_BF16_PEAK_TFLOPS, 4)
    res = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": kv, "data": "synthetic",
        "config": {"workload": f"{workload}: {len(ctx)} seqs, {n} rows, ctx "
                               f"{'log-uniform [64,4096]' if workload == 'config2' else 'see bench.py'}"
                               f", Qwen2.5-0.5B GQA 14/2 x 64, block 16, pool {pool} blocks,"
                               f" {L} layers per step (own KV pool each)",
                   "kv_dtype": kv, "act_dtype": "f32", "layers": L,
                   "parallelism": "none (1 GPU)"},
        "pct_of_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_rows_per_s": round(n / (ms * 1e-3), 1),
        "plan": {"rows": P.n_tokens, "decode_items": P.n_decode_items, "chunk_items": P.n_chunk_items,
                 "parts": P.n_parts, "bytes": int(P.bytes), "pack_us": round(pack_us, 1)},
        "roofline": roofline,
    }
    del kc, vc, qs, knew, vnew, outs, ws, plan, step
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return res


def phase_summary(mixed):
    """Per-phase stamps of the last attention launch, from a measurement build
    (python llm-engine_amd/build.py -D LE_TIMING --out <dir>/libllm_engine_amd.so,
    loaded with LE_LIB_PATH): microseconds from the first workgroup's start,
    median and max over workgroups, per phase (le_common.h, slots 0-4), per
    workgroup kind (decode, chunk), with the number of distinct CUs the
    workgroups ran on. `mixed` reads the fused mixed-step kernel's stamps,
    which live in its own translation unit."""
    import ctypes
    from llm_engine_amd import _lib
    lib = _lib.load()
    fn = "le_timing_read_ragged" if mixed else "le_timing_read"
    if not hasattr(lib, fn):
        raise SystemExit("bench.py --phases needs a LE_TIMING build (LE_LIB_PATH)")
    buf = np.zeros(65536 * 16, dtype=np.uint64)
    rc = getattr(lib, fn)(ctypes.c_void_p(buf.ctypes.data), ctypes.c_int64(buf.nbytes))
    if rc != 0:
        raise SystemExit(f"{fn}: {rc}")
    t = buf.reshape(65536, 16).astype(np.int64)
    t = t[(t[:, 0] > 0) & (t[:, 7] > 0)]
    if not len(t):
        raise SystemExit("bench.py --phases: no stamps")
    t = t[t[:, 0] >= t[:, 0].max() - 100000]  # the last launch (stamps of launches 1 ms before stay)
    t0 = t[:, 0].min()
    # a CU: XCC_ID with HW_ID's cu/sh/se fields (bits 8-15; the low bits name the wave and SIMD)
    cus = set(zip((t[:, 5] >> 32).tolist(), ((t[:, 5] >> 8) & 0xff).tolist()))
    out = {"workgroups": int(len(t)), "distinct_cus": int(len(cus))}

    def stat(x):
        return {"median": round(float(np.median(x)), 2), "max": round(float(x.max()), 2)}

    for kinds, kname in (((1, 3), "decode"), ((2,), "chunk")):
        k = t[np.isin(t[:, 7], kinds)]
        if not len(k):
            continue
        rt = (k[:, 7] == 3).any()  # round-trip probe build (LE_TIMING_RT): slots 8 and 9 are its stamps
        us = (k[:, :5] - t0) / 100.0  # realtime counter: 100 MHz
        split = (k[:, 6] & 0xffffffff) > 0
        o = {"workgroups": int(len(k))}
        for i, name in enumerate(("start", "staged", "tiles_done", "written", "end")):
            o[name] = stat(us[:, i])
        if rt:
            o["ids_back"] = stat((k[:, 8] - t0) / 100.0)
            o["first_tile_back"] = stat((k[:, 9] - t0) / 100.0)
        elif (k[:, 8] > 0).any():  # every wave's tiles done (slots 8-15; 0 for waves that never stamp)
            w = k[:, 8:16]
            done = np.where(w > 0, w, 0).max(axis=1)
            o["tiles_done_all_waves"] = stat((done - t0) / 100.0)
        if split.any():
            o["end_split"] = stat(us[split, 4])
        if (~split).any():
            o["end_unsplit"] = stat(us[~split, 4])
        out[kname] = o
    return out


def e2e_run(arch, prompts, out_lens, pool_blocks, max_seqs=64, budget=512, arrivals_s=None,
            prefix_caching=False, seed=4, layers=None, decode_graph=False):
    """One end-to-end run of the engine: scheduler, packing, device model,
    device greedy. Random-init weights N(0, 0.02) held as bf16 on the device,
    bf16 K/V cache, block 16, chunked prefill budget `budget` tokens/step."""
    from llm_engine_amd.engine import Model, sched_config, synthetic_weights
    t0 = time.perf_counter()
    w = synthetic_weights(arch, seed, layers=layers)
    L = w.arch["layers"]
    w_arch = dict(w.arch)
    m = Model(w, pool_blocks, 16, dtype="bf16", kv_dtype="bf16", decode_graph=decode_graph)
    del w
    setup_s = time.perf_counter() - t0
    cfg = sched_config(max_num_seqs=max_seqs, max_num_batched_tokens=budget, prefill_chunk_size=budget)
    m.run_greedy([p[:64] for p in prompts[:4]], [4] * 4, cfg)  # warm-up: code objects, rocBLAS
    toks, st = m.run_greedy(prompts, out_lens, cfg, prefix_caching=prefix_caching, arrival_s=arrivals_s)
    replays = m.graph_replays
    m.close()
    gen_total = sum(len(t) for t in toks)
    if gen_total != sum(out_lens):
        raise SystemExit("bench.py: not every request finished")
    # Decode-step roofline: every step streams all weights (bf16; the LM head
    # too) and each row's K/V history once (bf16, per layer).
    a = w_arch
    kv_dim = a["kv_heads"] * a["head_dim"]
    per_layer = a["hidden"] * (a["q_heads"] * a["head_dim"] + 2 * kv_dim) + a["q_heads"] * a["head_dim"] * a["hidden"] \
        + 3 * a["hidden"] * a["inter"]
    weight_bytes = 2 * (L * per_layer + a["vocab"] * a["hidden"])
    roof = None
    if st.decode_steps:
        kv_bytes = st.decode_context_tokens / st.decode_steps * L * kv_dim * 2 * 2
        step_s = st.decode_seconds / st.decode_steps
        achieved = (weight_bytes + kv_bytes) / step_s / 1e9
        roof = {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "bytes_per_step": int(weight_bytes + kv_bytes),
                "weight_bytes": int(weight_bytes), "kv_bytes_per_step": int(kv_bytes),
                "what": "bf16 weights + K/V history per decode step / wall time per decode step"}
    return {"model": f"{arch}, {L} layers, random-init bf16 weights, bf16 KV",
            "requests": len(prompts), "pool_blocks": pool_blocks, "max_running": max_seqs,
            "prefix_caching": prefix_caching, "prompt_tokens_computed": int(st.prompt_tokens),
            "generated_tokens": gen_total, "steps": int(st.steps), "seconds": round(st.seconds, 3),
            "tok_per_s": round(gen_total / st.seconds, 1), "decode_steps": int(st.decode_steps),
            "decode_tok_per_s": round(st.decode_step_tokens / st.decode_seconds, 1) if st.decode_seconds else None,
            "decode_ms_per_step": round(1e3 * st.decode_seconds / st.decode_steps, 3) if st.decode_steps else None,
            "ttft_mean_s": round(st.ttft_mean_s, 4), "latency_mean_s": round(st.latency_mean_s, 3),
            "preemptions": int(st.preemptions), "setup_s": round(setup_s, 1),
            "plan_us_per_step": round(1e6 * st.plan_seconds / st.steps, 1) if st.steps else None,
            "decode_graph": decode_graph, "graph_replays": replays, "decode_roofline": roof}


def e2e_leg(which, layers=None):
    """The end-to-end workloads (TinyLlama-1.1B for decode64/config4, Qwen2.5-0.5B
    for config5):
      decode64  closed loop: 64 requests at t=0, prompts U[128, 1024], 256 greedy
                tokens each, at most 64 running; decode tok/s = tokens sampled in
                steps with no prefill / their wall time (host scheduling, packing,
                upload, all layers, greedy read-back); run eagerly, then again
                with decode steps replayed from HIP graphs ("with_decode_graph")
      config4   256 requests, Poisson arrivals at 8/s, prompts U[128, 1024],
                outputs U[64, 256], at most 64 running, budget 512
      config5   128 requests sharing a 512-token prefix (prefix caching on) plus
                unique suffixes U[64, 7680], 256 tokens each (contexts up to
                8192), 16384-block pool: preemption and recompute under pressure."""
    rng = np.random.default_rng(4)
    if which in ("decode64", "config4"):
        n = 64 if which == "decode64" else 256
        V = 32000
        prompts = [rng.integers(0, V, int(x)).astype(np.int32) for x in rng.integers(128, 1025, size=n)]
        if which == "decode64":
            eager = e2e_run("tinyllama-1.1b", prompts, [256] * n, 5120, layers=layers)
            graph = e2e_run("tinyllama-1.1b", prompts, [256] * n, 5120, layers=layers, decode_graph=True)
            return eager | {"with_decode_graph": {k: graph[k] for k in (
                "decode_tok_per_s", "decode_ms_per_step", "tok_per_s", "graph_replays", "plan_us_per_step",
                "decode_roofline")}}
        outs = rng.integers(64, 257, size=n).tolist()
        arr = np.cumsum(rng.exponential(1.0 / 8.0, size=n)).tolist()
        return e2e_run("tinyllama-1.1b", prompts, outs, 5120, arrivals_s=arr, layers=layers) | \
            {"arrivals_per_s": 8.0}
    V = 151936
    prefix = rng.integers(0, V, 512)
    prompts = [np.concatenate([prefix, rng.integers(0, V, int(x))]).astype(np.int32)
               for x in rng.integers(64, 7681, size=128)]
    return e2e_run("qwen2.5-0.5b", prompts, [256] * 128, 16384, max_seqs=128, prefix_caching=True,
                   layers=layers)


def copy_floor():
    """A plain copy of the same traffic as each attention workload's launch
    (algorithmic bytes, half read and half written), 24 rotating buffer pairs
    as the 24 layers' pools rotate, HIP events over 20 rounds."""
    import torch
    sizes = {"config2": 30345840, "config3": 26332552, "target": 134742784}
    out = {"calibration": "device copy (torch copy_, bf16) with the traffic of one attention launch, "
                          "24 rotating buffer pairs, HIP events over 20 x 24 launches", "sizes": {}}
    for name, nbytes in sizes.items():
        n = nbytes // 4  # bf16 elements read (and written): nbytes of traffic in all
        xs = [torch.empty(n, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(24)]
        ys = [torch.empty_like(x) for x in xs]
        for _ in range(3):
            for x, y in zip(xs, ys):
                y.copy_(x)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for _ in range(20):
            for x, y in zip(xs, ys):
                y.copy_(x)
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / (20 * 24)
        out["sizes"][name] = {"traffic_bytes": 4 * n, "us_per_launch": round(us, 3),
                              "gbs": round(4 * n / us / 1e3, 1),
                              "frac_of_8tbs": round(4 * n / us / 1e3 / HBM_PEAK_GBS, 4)}
        del xs, ys
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--kv", choices=["bf16", "f32"], default="bf16")
    ap.add_argument("--workload", choices=["config2", "target", "config3"], default="config2")
    ap.add_argument("--layers", type=int, default=LAYERS)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="replay the attention-only loop behind `roofline` from a captured HIP graph too")
    ap.add_argument("--eager-step", action="store_true",
                    help="launch the step's kernels eagerly instead of replaying it from a captured HIP graph")
    ap.add_argument("--separate-scatter", action="store_true",
                    help="scatter with le_kv_cache_write, then attend (instead of the fused entry point)")
    ap.add_argument("--e2e", choices=["decode64", "config4", "config5", "default", "all", "none"], default="default",
                    help="end-to-end leg after the attention measurement (see e2e_leg)")
    ap.add_argument("--e2e-layers", type=int, default=None, help="model layers (default: all)")
    ap.add_argument("--cpu-budget", type=float, default=10.0)
    ap.add_argument("--no-extra-workloads", action="store_true",
                    help="skip the target, target_f32 and config3 sub-measurements of a config2 run")
    ap.add_argument("--partition", type=int, default=0, help="decode partition tokens (0 = planner's choice)")
    ap.add_argument("--flags", type=int, default=4,
                    help="le_plan_config.flags (2 = LE_PLAN_TWO_LAUNCHES, 4 = LE_PLAN_XCD_LOCAL, the default: "
                         "the bench launches on torch's default stream, no CU mask)")
    ap.add_argument("--chunk-partition", type=int, default=0,
                    help="chunk-row key partition tokens (0 = planner's choice)")
    ap.add_argument("--phases", action="store_true",
                    help="add per-phase workgroup stamps of the last decode launch (needs a LE_TIMING "
                         "build of the library, selected with LE_LIB_PATH)")
    ap.add_argument("--calibrate-stream", action="store_true",
                    help="only measure the read rate of a library reduction (torch sum) over 134 MB "
                         "buffers that no recent launch touched: the practical HBM read ceiling")
    ap.add_argument("--calibrate-floor", action="store_true",
                    help="only time a plain device copy (torch copy_) whose traffic equals each "
                         "workload's algorithmic bytes per launch (half read, half written), over 24 "
                         "rotating buffer pairs: what a launch of that size reaches with no gather, "
                         "no compute and no merge")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a plain 256 MiB device copy (the reference kernel for scaling "
                         "rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes)")
    args = ap.parse_args()
    if args.calibrate_stream:
        import torch
        # 8 buffers of the target point's K/V size (134 MB), read round robin so
        # that the 256 MB MALL never holds the next one
        nbuf, nbytes = 8, 134217728
        bufs = [torch.empty(nbytes // 2, dtype=torch.bfloat16, device="cuda").normal_() for _ in range(nbuf)]
        outs = torch.empty(nbuf, dtype=torch.float32, device="cuda")
        for i in range(2 * nbuf):
            torch.sum(bufs[i % nbuf], 0, dtype=torch.float32, out=outs[i % nbuf])
        reps = 10 * nbuf
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0.record()
        for i in range(reps):
            torch.sum(bufs[i % nbuf], 0, dtype=torch.float32, out=outs[i % nbuf])
        t1.record()
        torch.cuda.synchronize()
        us = t0.elapsed_time(t1) * 1e3 / reps
        print(json.dumps({"calibration": "read-only reduction (torch.sum, bf16 -> fp32) over 8 rotating "
                                         "134217728-byte buffers, HIP events over 80 launches",
                          "bytes_per_launch": nbytes, "us_per_launch": round(us, 3),
                          "gbs": round(nbytes / us / 1e3, 1), "frac_of_8tbs": round(nbytes / us / 1e3 / HBM_PEAK_GBS, 4)}))
        return
    if args.calibrate_floor:
        print(json.dumps(copy_floor()))
        return
    if args.calibrate_copy:
        import torch
        x = torch.empty(256 << 20, dtype=torch.uint8, device="cuda")
        x.fill_(1)
        y = torch.empty_like(x)
        for _ in range(3):
            y.copy_(x)
        # two kernels that do one thing each, to check the copy's factors:
        # a reduction reads the 256 MiB and writes 8 bytes, a fill writes
        # them and reads nothing
        for _ in range(3):
            x.sum(dtype=torch.int64)
        for _ in range(3):
            y.fill_(2)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "copy, read-only sum, write-only fill", "bytes_read": x.numel(),
                          "bytes_written": y.numel()}))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build runs on one GPU only (the decode path shards by "
              "sequence with no exchange; multi-GPU runs are not part of it).", file=sys.stderr)
        sys.exit(2)

    # The north star's target point and the mixed step are measured the same
    # way (fewer steps), each with its own roofline, after the main workload.
    extras = []
    if args.workload == "config2" and not args.no_extra_workloads:
        extras = [("target", "target", "bf16"), ("target_f32", "target", "f32"), ("config3", "config3", "bf16")]
    # the K/V arena at the size of the largest leg, before the first
    import torch
    need = max(2 * args.layers * workload_shape(w)[2] * BS * KV_HEADS * HEAD_DIM * (2 if k == "bf16" else 4)
               for w, k in [(args.workload, args.kv)] + [(e[1], e[2]) for e in extras])
    kv_arena(need, torch.device("cuda:0"))
    res = attention_leg(args.workload, args.kv, args.layers, args.steps, args.warmup, args.partition,
                        args.chunk_partition, args.graph, args.separate_scatter, args.flags,
                        step_graph=not args.eager_step)
    if args.phases:
        res["phases"] = phase_summary(res["plan"].get("chunk_items", 0) > 0)
    if extras:
        for key, extra, kv in extras:
            sub = attention_leg(extra, kv, args.layers, max(10, args.steps // 2), args.warmup, flags=args.flags,
                                step_graph=not args.eager_step)
            res[key] = {k: sub[k] for k in ("value", "unit", "ms_per_step", "pct_of_peak", "config", "plan",
                                             "roofline")}
    ctx, q_len, _ = workload_shape(args.workload)
    if not args.no_cpu_baseline:
        res["cpu_baseline"] = cpu_baseline(ctx, q_len, args.kv == "bf16", args.cpu_budget)
    else:
        res["cpu_baseline"] = None
    legs = {"all": ["decode64", "config4", "config5"], "default": ["decode64", "config4"]}.get(args.e2e, [args.e2e])
    for leg in legs:
        if leg != "none":
            res["e2e_" + leg] = e2e_leg(leg, layers=args.e2e_layers)
            if leg == "decode64" and not args.no_cpu_baseline:
                res["e2e_decode64"]["cpu_baseline"] = cpu_e2e_decode_baseline()
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
