"""Writes the golden fixtures under tests/golden/ from the reference engine's
own CPU code, compiled from /root/reference by oracle/Makefile into
oracle/_ref/libref.so (ops.h, tensor.h, kv_cache.h, block_allocator.cpp,
scheduler.cpp, sampler.cpp). Run in the build container:

    make -C oracle ref && python tests/golden/make_golden.py

Fixtures are data only: seeded inputs and the reference's outputs.
  attention_ref.npz   paged attention (ops.h:87-111 via the cpu_model.cpp
                      (token, head) loop) on fragmented tables; K/V values are
                      bf16-representable fp32 so they can be stored as 16 bits
  ops_ref.npz         rmsnorm, rope tables + rotation, silu_mul, bf16/fp16
                      conversions, argmax ties
  schedule_ref.npz    step-by-step traces of the reference Scheduler +
                      KVCacheManager driving a deterministic fake model
"""
from __future__ import annotations

import ctypes
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
sys.path.insert(0, str(ROOT / "oracle"))
import oracle  # noqa: E402


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def bf16_exact(rng, shape):
    """N(0,1) rounded to bf16: exact fp32 values storable as 16 bits."""
    x = rng.standard_normal(shape, dtype=np.float32)
    return oracle.bf16_to_f32(oracle.f32_to_bf16(x))


def attention_case(seed, ctx, q_len, q_heads, kv_heads, head_dim, bs, spare_blocks=8):
    rng = np.random.default_rng(seed)
    ctx = np.asarray(ctx)
    q_len = np.asarray(q_len)
    nblk = (ctx + bs - 1) // bs
    num_blocks = int(nblk.sum()) + spare_blocks
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = perm[:int(nblk.sum())]
    table_offset = np.concatenate([[0], np.cumsum(nblk)[:-1]]).astype(np.int32)
    kv_dim = kv_heads * head_dim
    k = bf16_exact(rng, (num_blocks * bs, kv_dim))
    v = bf16_exact(rng, (num_blocks * bs, kv_dim))
    n = int(q_len.sum())
    q = rng.standard_normal((n, q_heads * head_dim), dtype=np.float32)
    token_seq = np.repeat(np.arange(len(ctx), dtype=np.int32), q_len)
    token_pos = np.concatenate([np.arange(c - ql, c) for c, ql in zip(ctx, q_len)]).astype(np.int32)
    out = np.zeros_like(q)
    scale = np.float32(1.0) / np.sqrt(np.float32(head_dim))
    R = oracle.ref()
    R.ref_paged_attention(ptr(q), q.shape[1], ptr(k), ptr(v), ptr(tables), ptr(table_offset),
                          ptr(nblk.astype(np.int32)), ptr(token_seq), ptr(token_pos), n, q_heads,
                          kv_heads, head_dim, bs, float(scale), ptr(out), q.shape[1])
    return dict(q=q, k_bf16=oracle.f32_to_bf16(k), v_bf16=oracle.f32_to_bf16(v), tables=tables,
                table_offset=table_offset, table_len=nblk.astype(np.int32), token_seq=token_seq,
                token_pos=token_pos, out=out,
                shape=np.array([q_heads, kv_heads, head_dim, bs, num_blocks], dtype=np.int32))


def write_attention():
    cases = {
        # Qwen2.5-0.5B GQA shape, decode rows, fragmented
        "qwen_decode": attention_case(1, [1, 17, 150, 300], [1, 1, 1, 1], 14, 2, 64, 16),
        # prefill chunks over a cached prefix beside decode rows
        "qwen_chunks": attention_case(2, [48, 120, 200], [48, 1, 33], 14, 2, 64, 16),
        # TinyLlama GQA group 8
        "tinyllama_decode": attention_case(3, [5, 64, 190], [1, 1, 1], 32, 4, 64, 16),
        # head_dim 128, block 8
        "hd128_bs8": attention_case(4, [9, 100], [3, 1], 8, 2, 128, 8),
    }
    flat = {f"{c}.{k}": v for c, d in cases.items() for k, v in d.items()}
    np.savez_compressed(HERE / "attention_ref.npz", **flat)


def write_ops():
    R = oracle.ref()
    rng = np.random.default_rng(7)
    out = {}
    x = rng.standard_normal((5, 896), dtype=np.float32) * 3
    w = (1 + 0.1 * rng.standard_normal(896)).astype(np.float32)
    y = np.empty_like(x)
    R.ref_rmsnorm(ptr(x), ptr(w), ptr(y), 5, 896, 1e-6)
    out.update({"rmsnorm.x": x, "rmsnorm.w": w, "rmsnorm.y": y})
    # RoPE tables (HF rotate_half) for Qwen (theta 1e6) and TinyLlama (theta 1e4):
    # a sample of rows of the 32768-position table
    rows = np.array(list(range(17)) + [255, 1000, 1024, 4095, 8191, 32767], dtype=np.int32)
    for name, theta in (("qwen", 1e6), ("llama", 1e4)):
        c = np.empty((32768, 32), dtype=np.float32)
        s = np.empty_like(c)
        R.ref_rope_tables(64, 32768, theta, ptr(c), ptr(s))
        out[f"rope_{name}.rows"] = rows
        out[f"rope_{name}.cos"] = c[rows]
        out[f"rope_{name}.sin"] = s[rows]
    xr = rng.standard_normal((3, 14 * 64), dtype=np.float32)
    pos = np.array([0, 1, 4095], dtype=np.int32)
    yr = xr.copy()
    for t in range(3):
        R.ref_rope_inplace(ptr(yr[t]), 14, 64, int(pos[t]), 4096, 1e6)
    out.update({"rope_apply.x": xr, "rope_apply.pos": pos, "rope_apply.y": yr})
    g = (rng.standard_normal(1000, dtype=np.float32) * 4)
    g[:6] = [-4.0, -0.5, 0.0, 0.5, 1.0, 7.0]  # the reference test's points (test_golden_ops.cpp:151)
    u = rng.standard_normal(1000, dtype=np.float32)
    gy = g.copy()
    R.ref_silu_mul(ptr(gy), ptr(u), 1000)
    out.update({"silu.gate": g, "silu.up": u, "silu.y": gy})
    # bf16 / fp16 conversions: random, specials, ties, subnormals
    f = np.concatenate([
        rng.standard_normal(4000).astype(np.float32) * 10.0 ** rng.integers(-40, 38, 4000),
        np.array([0.0, -0.0, 1.0, -1.0, 3.140625, 65504.0, 1e5, 1e-8, 5.960464477539063e-08,
                  np.inf, -np.inf, np.nan, 3.4028235e38, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8,
                  1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11], dtype=np.float32)]).astype(np.float32)
    out["conv.f32"] = f
    out["conv.bf16"] = np.array([R.ref_f32_to_bf16(float(v)) for v in f], dtype=np.uint16)
    R.ref_f32_to_f16.restype = ctypes.c_uint16
    R.ref_f32_to_f16.argtypes = [ctypes.c_float]
    out["conv.f16"] = np.array([R.ref_f32_to_f16(float(v)) for v in f], dtype=np.uint16)
    # argmax: first maximum wins (sampler.cpp:9-13)
    am = [np.array([-1.0, 5.0, 2.0, 5.0], dtype=np.float32), np.array([3.0], dtype=np.float32),
          np.array([-9.0, -8.0, -100.0], dtype=np.float32),
          rng.standard_normal(20000).astype(np.float32)]
    am[3][[10, 19999]] = am[3].max() + 1.0
    for i, a in enumerate(am):
        out[f"argmax.{i}.x"] = a
        out[f"argmax.{i}.y"] = np.array(R.ref_argmax(ptr(a), a.size), dtype=np.int32)
    np.savez_compressed(HERE / "ops_ref.npz", **out)


TRACE_CONFIGS = {
    # name: (num_blocks, bs, prefix, max_seqs, max_batched, chunk, watermark, fragment, n_seqs,
    #        prompt length range, max_tokens (or a range), continuous, lookahead, starvation)
    "fragmented": (256, 16, 0, 32, 4096, 512, -1, 40, 6, (20, 300), 8, 1, 1, 64),
    "chunked16": (256, 16, 0, 32, 4096, 16, -1, 0, 4, (40, 200), 6, 1, 1, 64),
    "preempt": (48, 16, 0, 8, 4096, 512, -1, 0, 8, (30, 120), 24, 1, 1, 64),
    "budget512": (1024, 16, 0, 64, 512, 512, -1, 0, 20, (128, 1024), 16, 1, 1, 64),
    "prefix": (256, 16, 1, 32, 4096, 512, -1, 0, 4, (20, 100), 8, 1, 1, 64),
    # static batching: members finish at different lengths and keep their
    # blocks until the batch drains; a small pool closes the batch early and
    # makes decode release finished members
    "static": (256, 16, 0, 4, 4096, 512, -1, 0, 10, (20, 200), (4, 30), 0, 1, 64),
    "static_mem": (40, 16, 0, 6, 4096, 128, 0, 0, 9, (40, 160), (10, 60), 0, 1, 64),
    # admission lookahead past a head that does not fit, bounded by starvation
    "lookahead": (40, 16, 0, 16, 4096, 256, -1, 0, 12, (16, 500), (8, 40), 1, 4, 3),
    # prefix cache under pressure: cached blocks are evicted and reused
    "prefix_evict": (72, 16, 1, 8, 4096, 512, -1, 0, 16, (10, 90), (4, 20), 1, 1, 64),
    # no admission headroom: decode growth preempts repeatedly
    "watermark0": (40, 16, 0, 8, 4096, 512, 0, 0, 10, (30, 120), (20, 60), 1, 1, 64),
    # the config-4 shape at trace size: budget 512, up to 64 running
    "config4": (2048, 16, 0, 64, 512, 512, -1, 0, 48, (128, 1024), (16, 64), 1, 1, 64),
}


def trace_inputs(name, n, lo, hi, mt, prefix):
    """Seeded prompts and max_tokens of one trace scenario."""
    rng = np.random.default_rng(len(name))
    lens = rng.integers(lo, hi + 1, size=n).astype(np.int32)
    if name == "prefix":  # a shared 96-token prefix (test_cuda_invariance.cpp:235-242)
        prompts = [np.concatenate([np.full(96, 1234), rng.integers(0, 32000, l)]).astype(np.int32) for l in lens]
    elif name == "prefix_evict":  # three shared prefixes of 2-4 blocks, taken in turn
        heads = [rng.integers(0, 32000, 16 * k).astype(np.int32) for k in (2, 3, 4)]
        prompts = [np.concatenate([heads[i % 3], rng.integers(0, 32000, l)]).astype(np.int32)
                   for i, l in enumerate(lens)]
    else:
        prompts = [rng.integers(0, 32000, l).astype(np.int32) for l in lens]
    lens = np.array([len(p) for p in prompts], dtype=np.int32)
    if isinstance(mt, tuple):
        maxt = rng.integers(mt[0], mt[1] + 1, size=n).astype(np.int32)
    else:
        maxt = np.full(n, mt, dtype=np.int32)
    return lens, np.concatenate(prompts).astype(np.int32), maxt


def write_schedules():
    R = oracle.ref()
    out = {}
    for name, c in TRACE_CONFIGS.items():
        nb, bs, prefix, ms, mbt, chunk, wm, frag, n, (lo, hi), mt, cont, look, starve = c
        lens, flat, maxt = trace_inputs(name, n, lo, hi, mt, prefix)
        buf = np.zeros(1 << 23, dtype=np.int32)
        got = R.ref_schedule_trace_ex(nb, bs, prefix, ms, mbt, chunk, wm, frag, cont, look, starve, n,
                                      ptr(lens), ptr(flat), ptr(maxt), 100000, ptr(buf), buf.size)
        assert got > 0, name
        out[f"{name}.config"] = np.array([nb, bs, prefix, ms, mbt, chunk, wm, frag, n, cont, look, starve],
                                         dtype=np.int32)
        out[f"{name}.prompt_lens"] = lens
        out[f"{name}.prompts"] = flat
        out[f"{name}.max_tokens"] = maxt
        out[f"{name}.trace"] = buf[:got].copy()
    np.savez_compressed(HERE / "schedule_ref.npz", **out)


if __name__ == "__main__":
    if not oracle.ref_available():
        oracle.build(ref=True)
    write_attention()
    write_ops()
    write_schedules()
    for f in sorted(HERE.glob("*.npz")):
        print(f.name, f.stat().st_size)
