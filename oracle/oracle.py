"""ctypes front end of the CPU oracle (liboracle.so): TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, as the checker or as the timed CPU baseline. See oracle.h for
the reference file:line each function restates.

Also loads oracle/_ref/libref.so (the reference's own CPU sources, compiled
by oracle/Makefile) when it has been built, via `ref()`.
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"
REF_LIB = HERE / "_ref" / "libref.so"

_P = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float


def build(ref: bool = False) -> None:
    targets = ["all"] + (["ref"] if ref else [])
    subprocess.run(["make", "-s", "-C", str(HERE), *targets], check=True)


_lib = None
_ref = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        L = ctypes.CDLL(str(LIB))
        L.orc_f32_to_bf16.restype = ctypes.c_uint16
        L.orc_f32_to_bf16.argtypes = [_f]
        L.orc_bf16_to_f32.restype = _f
        L.orc_bf16_to_f32.argtypes = [ctypes.c_uint16]
        L.orc_f32_to_bf16_n.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_bf16_to_f32_n.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_f32_to_f16_n.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_f16_to_f32_n.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_slot.restype = ctypes.c_int64
        L.orc_slot.argtypes = [_P, _i, _i]
        L.orc_pack_step.argtypes = [_P, _i, _i] + [_P] * 8
        L.orc_store_kv.argtypes = [_P, _P, _P, _P, _P, _i, _i]
        L.orc_store_kv_bf16.argtypes = [_P, _P, _P, _P, _P, _i, _i]
        L.orc_paged_attention_head.argtypes = [_P, _P, _P, _P, _i, _i, _i, _i, _i, _f, _P, _P]
        L.orc_paged_attention.argtypes = [_P, _i, _P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i, _f,
                                          _P, _i, _i]
        L.orc_paged_attention_bf16kv.argtypes = L.orc_paged_attention.argtypes
        L.orc_rmsnorm.argtypes = [_P, _P, _P, _i, _i, _f]
        L.orc_rope_tables.argtypes = [_i, _i, _f, _P, _P]
        L.orc_rope_inplace.argtypes = [_P, _i, _i, _i, _P, _P]
        L.orc_silu_mul.argtypes = [_P, _P, ctypes.c_size_t]
        L.orc_linear.argtypes = [_P, _i, _i, _P, _i, _P, _P, _i]
        L.orc_argmax.restype = ctypes.c_int32
        L.orc_argmax.argtypes = [_P, _i]
        L.orc_forward.argtypes = [_P, _P, _P, _P, _P, _i, _P, _P, _P, _P, _P, _P, _i, _P, _i, _i,
                                  _P, _i]
        L.orc_forward_trace.argtypes = L.orc_forward.argtypes + [_P]
        _lib = L
    return _lib


def ref_available() -> bool:
    return REF_LIB.exists()


def ref() -> ctypes.CDLL:
    """The reference's own CPU code (block allocator, scheduler, sampler, ops.h)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(str(REF_LIB))
        R.ref_f32_to_bf16.restype = ctypes.c_uint16
        R.ref_f32_to_bf16.argtypes = [_f]
        R.ref_f32_to_f16.restype = ctypes.c_uint16
        R.ref_f32_to_f16.argtypes = [_f]
        R.ref_f16_to_f32.restype = _f
        R.ref_f16_to_f32.argtypes = [ctypes.c_uint16]
        R.ref_bf16_to_f32.restype = _f
        R.ref_bf16_to_f32.argtypes = [ctypes.c_uint16]
        R.ref_slot.restype = ctypes.c_int64
        R.ref_slot.argtypes = [_P, _i, _i, _i]
        R.ref_rmsnorm.argtypes = [_P, _P, _P, _i, _i, _f]
        R.ref_rope_tables.argtypes = [_i, _i, _f, _P, _P]
        R.ref_rope_inplace.argtypes = [_P, _i, _i, _i, _i, _f]
        R.ref_silu_mul.argtypes = [_P, _P, ctypes.c_size_t]
        R.ref_argmax.restype = ctypes.c_int32
        R.ref_argmax.argtypes = [_P, _i]
        R.ref_paged_attention.argtypes = [_P, _i, _P, _P, _P, _P, _P, _P, _P, _i, _i, _i, _i, _i,
                                          _f, _P, _i]
        R.ref_schedule_trace.restype = ctypes.c_int64
        R.ref_schedule_trace.argtypes = [_i] * 9 + [_P, _P, _P, _i, _P, ctypes.c_int64]
        R.ref_schedule_trace_ex.restype = ctypes.c_int64
        R.ref_schedule_trace_ex.argtypes = [_i] * 12 + [_P, _P, _P, _i, _P, ctypes.c_int64]
        _ref = R
    return _ref


def ptr(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def threads_default() -> int:
    return int(os.environ.get("LE_ORACLE_THREADS", str(min(16, os.cpu_count() or 1))))


# ---------------------------------------------------------------- wrappers
def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().orc_f32_to_bf16_n(ptr(x), ptr(out), x.size)
    return out


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    h = np.ascontiguousarray(h, dtype=np.uint16)
    out = np.empty(h.shape, dtype=np.float32)
    lib().orc_bf16_to_f32_n(ptr(h), ptr(out), h.size)
    return out


class Packed:
    """Arrays of one packed step, as the reference's upload_step_indices builds them."""

    def __init__(self, token_ids, positions, slots, token_seq, tables, table_offset, logit_rows):
        self.token_ids = token_ids
        self.positions = positions
        self.slots = slots
        self.token_seq = token_seq
        self.tables = tables
        self.table_offset = table_offset
        self.logit_rows = logit_rows


class OrcSlice(ctypes.Structure):
    _fields_ = [("seq_key", ctypes.c_int64), ("start", ctypes.c_int32), ("len", ctypes.c_int32),
                ("needs_logits", ctypes.c_int32), ("num_blocks", ctypes.c_int32),
                ("blocks", ctypes.c_void_p), ("tokens", ctypes.c_void_p)]


def pack_step(slices, block_size: int) -> Packed:
    """slices: list of (seq_key, start, len, needs_logits, blocks ndarray, tokens ndarray)."""
    keep = []
    arr = (OrcSlice * max(1, len(slices)))()
    for i, (key, start, ln, nl, blocks, tokens) in enumerate(slices):
        b = np.ascontiguousarray(blocks, dtype=np.int32)
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        keep += [b, t]
        arr[i] = OrcSlice(key, start, ln, int(nl), b.size, b.ctypes.data, t.ctypes.data)
    counts = np.zeros(4, dtype=np.int32)
    L = lib()
    L.orc_pack_step(arr, len(slices), block_size, None, None, None, None, None, None, None,
                    ptr(counts))
    n, s, t, r = (int(c) for c in counts)
    a = [np.zeros(max(x, 1), dtype=np.int32) for x in (n, n, n, n, t, s, r)]
    L.orc_pack_step(arr, len(slices), block_size, *[ptr(x) for x in a], ptr(counts))
    sizes = (n, n, n, n, t, s, r)
    return Packed(*[x[:k] for x, k in zip(a, sizes)])


def f32_to_f16(x) -> np.ndarray:
    """fp32 -> fp16 (orc_f32_to_f16: tensor.h:38-56, round to nearest even),
    returned as a float16 array."""
    a = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().orc_f32_to_f16_n(ptr(a), ptr(out), a.size)
    return out.view(np.float16)


def f16_to_f32(h) -> np.ndarray:
    """fp16 (float16 array or uint16 bits) -> fp32 (orc_f16_to_f32, exact)."""
    a = np.ascontiguousarray(h).view(np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().orc_f16_to_f32_n(ptr(a), ptr(out), a.size)
    return out


def paged_attention(q, k_cache, v_cache, tables, table_offset, token_seq, token_pos, q_heads,
                    kv_heads, head_dim, block_size, scale, threads=None):
    """q: [N, q_heads*head_dim] f32; caches [slots, kv_heads*head_dim] as f32,
    uint16 (bf16 bits) or float16. Returns out [N, q_heads*head_dim] f32.
    fp16 caches are widened to fp32 first (exact), as the reference's fp16
    kernels widen each element in registers (attention_decode.cu:94-103)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    n = q.shape[0]
    out = np.zeros((n, q_heads * head_dim), dtype=np.float32)
    args = [np.ascontiguousarray(x, dtype=np.int32) for x in (tables, table_offset, token_seq, token_pos)]
    if k_cache.dtype == np.float16:
        k_cache = f16_to_f32(k_cache)
        v_cache = f16_to_f32(v_cache)
    kc = np.ascontiguousarray(k_cache)
    vc = np.ascontiguousarray(v_cache)
    fn = lib().orc_paged_attention_bf16kv if kc.dtype == np.uint16 else lib().orc_paged_attention
    fn(ptr(q), q_heads * head_dim, ptr(kc), ptr(vc), *[ptr(x) for x in args], n, q_heads,
       kv_heads, head_dim, block_size, float(scale), ptr(out), q_heads * head_dim,
       threads or threads_default())
    return out


def store_kv(k, v, slots, k_cache, v_cache):
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    s = np.ascontiguousarray(slots, dtype=np.int32)
    kv_dim = k.shape[1]
    if k_cache.dtype == np.float16:  # store_kv.cu:20-36 into an fp16 cache
        ok = (s >= 0) & (s < k_cache.shape[0])
        k_cache[s[ok]] = f32_to_f16(k[ok])
        v_cache[s[ok]] = f32_to_f16(v[ok])
        return
    fn = lib().orc_store_kv_bf16 if k_cache.dtype == np.uint16 else lib().orc_store_kv
    fn(ptr(k), ptr(v), ptr(s), ptr(k_cache), ptr(v_cache), k.shape[0], kv_dim)


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty_like(x)
    lib().orc_rmsnorm(ptr(x), ptr(np.ascontiguousarray(w, dtype=np.float32)), ptr(out),
                      x.shape[0], x.shape[1], float(eps))
    return out


def rope_tables(head_dim, max_pos, theta):
    c = np.empty((max_pos, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables(head_dim, max_pos, float(theta), ptr(c), ptr(s))
    return c, s


def rope(x, positions, cos_t, sin_t, heads, head_dim):
    """RoPE (rotate_half) in place on the first heads*head_dim columns of each
    row of x (fp32 [N, cols]) at positions[t]."""
    assert x.dtype == np.float32 and x.flags.c_contiguous
    L = lib()
    row_bytes = x.strides[0]
    base = x.ctypes.data
    for t, p in enumerate(np.asarray(positions, dtype=np.int64)):
        L.orc_rope_inplace(ctypes.c_void_p(base + t * row_bytes), heads, head_dim, int(p), ptr(cos_t),
                           ptr(sin_t))
    return x


def linear(a, b, bias=None, threads=None):
    a = np.ascontiguousarray(a, dtype=np.float32)
    b = np.ascontiguousarray(b, dtype=np.float32)
    out = np.empty((a.shape[0], b.shape[0]), dtype=np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().orc_linear(ptr(a), a.shape[0], a.shape[1], ptr(b), b.shape[0],
                     None if bb is None else ptr(bb), ptr(out), threads or threads_default())
    return out


def argmax(logits: np.ndarray) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return int(lib().orc_argmax(ptr(x), x.size))
