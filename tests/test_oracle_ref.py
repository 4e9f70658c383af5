"""The C oracle (oracle/oracle.c) against the reference engine's own code.

Two sources pin it:
  * tests/golden/*.npz, written from the reference compiled from its sources
    (oracle/_ref/libref.so, tests/golden/make_golden.py): checked everywhere;
  * the reference library itself, when it has been built (this container):
    randomised cross-checks on fresh inputs.
Every comparison is bit-exact: the oracle keeps the reference's summation
order (float dot products, double softmax denominator, double RMSNorm sum of
squares, double-built RoPE tables)."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import oracle

GOLD = Path(__file__).resolve().parent / "golden"


def bits_equal(a, b):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    return a.shape == b.shape and np.array_equal(a.view(np.uint32), b.view(np.uint32))


def _cases():
    z = np.load(GOLD / "attention_ref.npz")
    names = sorted({k.split(".")[0] for k in z.files})
    return z, names


@pytest.mark.parametrize("name", _cases()[1])
def test_attention_matches_reference_fixture(name):
    """ops.h:87-111 through the cpu_model.cpp (token, head) loop, fragmented
    tables: the oracle reproduces the reference's output bit for bit."""
    z, _ = _cases()
    g = lambda k: z[f"{name}.{k}"]
    qh, kvh, hd, bs, nb = (int(v) for v in g("shape"))
    k = oracle.bf16_to_f32(g("k_bf16"))
    v = oracle.bf16_to_f32(g("v_bf16"))
    scale = float(np.float32(1.0) / np.sqrt(np.float32(hd)))
    out = oracle.paged_attention(g("q"), k, v, g("tables"), g("table_offset"), g("token_seq"),
                                 g("token_pos"), qh, kvh, hd, bs, scale, threads=4)
    assert bits_equal(out, g("out"))
    # the table really is fragmented (no two consecutive logical blocks adjacent everywhere)
    t = g("tables")
    assert np.any(np.diff(t) != 1)


def test_ops_match_reference_fixture():
    z = np.load(GOLD / "ops_ref.npz")
    assert bits_equal(oracle.rmsnorm(z["rmsnorm.x"], z["rmsnorm.w"], 1e-6), z["rmsnorm.y"])
    for name, theta in (("qwen", 1e6), ("llama", 1e4)):
        c, s = oracle.rope_tables(64, 32768, theta)
        rows = z[f"rope_{name}.rows"]
        assert bits_equal(c[rows], z[f"rope_{name}.cos"])
        assert bits_equal(s[rows], z[f"rope_{name}.sin"])
    c, s = oracle.rope_tables(64, 4096, 1e6)
    x = z["rope_apply.x"].copy()
    L = oracle.lib()
    for t, p in enumerate(z["rope_apply.pos"]):
        row = np.ascontiguousarray(x[t])
        L.orc_rope_inplace(oracle.ptr(row), 14, 64, int(p), oracle.ptr(c), oracle.ptr(s))
        x[t] = row
    assert bits_equal(x, z["rope_apply.y"])
    g = z["silu.gate"].copy()
    L.orc_silu_mul(oracle.ptr(g), oracle.ptr(np.ascontiguousarray(z["silu.up"])), g.size)
    assert bits_equal(g, z["silu.y"])
    assert np.array_equal(oracle.f32_to_bf16(z["conv.f32"]), z["conv.bf16"])
    assert np.array_equal(oracle.f32_to_f16(z["conv.f32"]).view(np.uint16), z["conv.f16"])
    i = 0
    while f"argmax.{i}.x" in z.files:
        assert oracle.argmax(z[f"argmax.{i}.x"]) == int(z[f"argmax.{i}.y"])
        i += 1


def test_f16_known_answers():
    """test_tensor.cpp:13-27: bit patterns, overflow, subnormals, ties to even."""
    h = lambda f: int(oracle.f32_to_f16(np.array([f], np.float32)).view(np.uint16)[0])
    assert h(1.0) == 0x3C00 and h(-2.0) == 0xC000 and h(65504.0) == 0x7BFF and h(1e5) == 0x7C00
    assert np.float32(np.array([1], np.uint16).view(np.float16)[0]) == np.float32(5.960464477539063e-08)
    assert h(1.0 + 2 ** -11) == 0x3C00 and h(1.0 + 3 * 2 ** -11) == 0x3C02
    for f in (0.0, 1.0, -1.0, 3.140625, 1024.0, -0.375, 2 ** -24, 65504.0):
        assert np.float32(oracle.f32_to_f16(np.array([f], np.float32))[0]) == np.float32(f)


def test_bf16_known_answers():
    """test_tensor.cpp:29-33: 1.0 -> 0x3F80, 0x4049 -> 3.140625, round trips."""
    assert oracle.f32_to_bf16(np.array([1.0], np.float32))[0] == 0x3F80
    assert oracle.bf16_to_f32(np.array([0x4049], np.uint16))[0] == np.float32(3.140625)
    for f in (0.0, 1.0, -1.0, 3.125, 1024.0, -0.375):
        assert oracle.bf16_to_f32(oracle.f32_to_bf16(np.array([f], np.float32)))[0] == np.float32(f)
    # ties to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7 -> 1.0
    assert oracle.f32_to_bf16(np.array([1 + 2 ** -8], np.float32))[0] == 0x3F80
    assert oracle.f32_to_bf16(np.array([1 + 3 * 2 ** -8], np.float32))[0] == 0x3F82


needs_ref = pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built")


def ptr(a):
    return a.ctypes.data_as(ctypes.c_void_p)


@needs_ref
@pytest.mark.parametrize("seed", range(6))
def test_attention_random_vs_reference(seed):
    rng = np.random.default_rng(100 + seed)
    qh, kvh = [(14, 2), (32, 4), (8, 8), (4, 1)][seed % 4]
    hd = 64 if seed % 3 else 128
    bs = [16, 8, 32][seed % 3]
    S = int(rng.integers(1, 6))
    ctx = rng.integers(1, 400, size=S)
    qlen = np.minimum(ctx, rng.integers(1, 5, size=S))
    nblk = (ctx + bs - 1) // bs
    num_blocks = int(nblk.sum()) + 5
    tables = rng.permutation(num_blocks)[:int(nblk.sum())].astype(np.int32)
    toff = np.concatenate([[0], np.cumsum(nblk)[:-1]]).astype(np.int32)
    kv = rng.standard_normal((num_blocks * bs, kvh * hd), dtype=np.float32)
    vv = rng.standard_normal((num_blocks * bs, kvh * hd), dtype=np.float32)
    n = int(qlen.sum())
    q = rng.standard_normal((n, qh * hd), dtype=np.float32) * 2
    tseq = np.repeat(np.arange(S, dtype=np.int32), qlen)
    tpos = np.concatenate([np.arange(c - l, c) for c, l in zip(ctx, qlen)]).astype(np.int32)
    scale = float(np.float32(1) / np.sqrt(np.float32(hd)))
    want = np.zeros_like(q)
    oracle.ref().ref_paged_attention(ptr(q), q.shape[1], ptr(kv), ptr(vv), ptr(tables), ptr(toff),
                                     ptr(nblk.astype(np.int32)), ptr(tseq), ptr(tpos), n, qh, kvh,
                                     hd, bs, scale, ptr(want), q.shape[1])
    got = oracle.paged_attention(q, kv, vv, tables, toff, tseq, tpos, qh, kvh, hd, bs, scale, threads=3)
    assert bits_equal(got, want)


@needs_ref
def test_scalar_ops_random_vs_reference():
    rng = np.random.default_rng(9)
    R = oracle.ref()
    f = (rng.standard_normal(20000) * 10.0 ** rng.integers(-45, 39, 20000)).astype(np.float32)
    ref_b = np.array([R.ref_f32_to_bf16(float(v)) for v in f], dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_bf16(f), ref_b)
    # fp16 over its whole range: normals, subnormals, underflow, overflow, ties
    g = np.concatenate([(rng.standard_normal(20000) * 2.0 ** rng.integers(-30, 18, 20000)).astype(np.float32),
                        (np.arange(-4096, 4096) * 2.0 ** -24 + 2.0 ** -26).astype(np.float32),
                        np.array([65504, 65519.996, 65520, -65520, 2 ** -25, 3 * 2 ** -26, np.inf, -np.inf, 0.0,
                                  -0.0], np.float32)])
    ref_h = np.array([R.ref_f32_to_f16(float(v)) for v in g], dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_f16(g).view(np.uint16), ref_h)
    assert np.array_equal(g.astype(np.float16).view(np.uint16), ref_h)  # and IEEE (numpy) agrees
    nans = np.array([0x7fc00000, 0xffc00000, 0x7f800001, 0xff812345, 0x7fffffff], np.uint32).view(np.float32)
    ref_n = np.array([R.ref_f32_to_f16(float(v)) for v in nans], dtype=np.uint16)
    assert np.array_equal(oracle.f32_to_f16(nans).view(np.uint16), ref_n)
    hb = rng.integers(0, 1 << 16, 5000).astype(np.uint16)
    hb = hb[(hb & 0x7c00) != 0x7c00]  # finite patterns
    ref_w = np.array([R.ref_f16_to_f32(int(h)) for h in hb], dtype=np.float32)
    assert bits_equal(oracle.f16_to_f32(hb), ref_w)
    assert bits_equal(hb.view(np.float16).astype(np.float32), ref_w)
    x = rng.standard_normal((7, 2048), dtype=np.float32)
    w = rng.standard_normal(2048).astype(np.float32)
    y = np.empty_like(x)
    R.ref_rmsnorm(ptr(x), ptr(w), ptr(y), 7, 2048, 1e-5)
    assert bits_equal(oracle.rmsnorm(x, w, 1e-5), y)
    blocks = rng.permutation(500).astype(np.int32)
    for pos in rng.integers(0, 500 * 16, 200):
        assert oracle.lib().orc_slot(ptr(blocks), int(pos), 16) == R.ref_slot(ptr(blocks), 500, int(pos), 16)
