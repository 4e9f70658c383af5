"""Python face of the C ABI for torch device tensors.

The names mirror the reference launchers (include/engine/cuda_kernels.h:43-64:
launch_store_kv, launch_attention_decode[_gqa]) plus the ragged step API.
Every call goes through libllm_engine_amd.so; there is no CPU path. Shapes
are checked on the host before anything is launched, and a non-zero status
raises LeError, as the reference launchers throw std::runtime_error.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from ._lib import LE_BF16, LE_F16, LE_F32, PlanConfig, StepPlan, StepSlice, check


_DTYPES = {torch.float32: LE_F32, torch.bfloat16: LE_BF16, torch.float16: LE_F16}


def _dt(t: torch.Tensor | torch.dtype) -> int:
    d = t if isinstance(t, torch.dtype) else t.dtype
    if d not in _DTYPES:
        raise TypeError(f"unsupported dtype {d}: expected float32, bfloat16 or float16")
    return _DTYPES[d]


def _stream(stream) -> ctypes.c_void_p:
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def _p(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def _req(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _dev_i32(t: torch.Tensor, name: str, n: int | None = None) -> None:
    _req(t.is_cuda and t.dtype == torch.int32 and t.is_contiguous(), f"{name}: contiguous int32 cuda tensor")
    if n is not None:
        _req(t.numel() >= n, f"{name}: needs {n} entries, has {t.numel()}")


def store_kv(k: torch.Tensor, v: torch.Tensor, slots: torch.Tensor, k_cache: torch.Tensor,
             v_cache: torch.Tensor, stream=None) -> None:
    """k_cache[slots[t]] = k[t], v likewise (store_kv.cu:20-36). k, v: [N, kv_dim];
    caches: [num_slots, kv_dim] or [num_slots, kv_heads, head_dim]."""
    _req(k.shape == v.shape and k.dim() == 2, "k, v: [N, kv_dim]")
    n, kv_dim = k.shape
    _req(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype, "k/v caches must match")
    num_slots = k_cache.shape[0]
    _req(k_cache.numel() == num_slots * kv_dim, "cache row size must equal kv_dim")
    _req(k.is_contiguous() and v.is_contiguous() and k_cache.is_contiguous() and v_cache.is_contiguous(),
         "contiguous tensors")
    _dev_i32(slots, "slots", n)
    check("le_kv_cache_write", _lib.load().le_kv_cache_write(
        _p(k), _p(v), _dt(k), _p(slots), _p(k_cache), _p(v_cache), _dt(k_cache), n, kv_dim,
        num_slots, _stream(stream)))


def rope_store_kv(qkv: torch.Tensor, positions: torch.Tensor, slots: torch.Tensor, cos_t: torch.Tensor,
                  sin_t: torch.Tensor, q_heads: int, kv_heads: int, head_dim: int, k_cache: torch.Tensor,
                  v_cache: torch.Tensor, bias: torch.Tensor | None = None, q_out: torch.Tensor | None = None,
                  stream=None) -> torch.Tensor:
    """Bias + RoPE + cache-write scatter over fused QKV rows
    (cuda_model.cu:358-368 as one launch). qkv: [N, >= (q_heads + 2*kv_heads)*head_dim]
    laid out [q | k | v]; cos_t/sin_t: fp32 [max_pos, head_dim/2]. Returns q: [N, q_heads*head_dim]."""
    _req(qkv.dim() == 2 and qkv.stride(1) == 1, "qkv: [N, row] with unit column stride")
    n = qkv.shape[0]
    _req(qkv.shape[1] >= (q_heads + 2 * kv_heads) * head_dim, "qkv rows too short")
    _req(cos_t.dtype == torch.float32 and cos_t.shape == sin_t.shape and cos_t.is_contiguous()
         and sin_t.is_contiguous() and cos_t.shape[1] == head_dim // 2, "cos/sin: fp32 [max_pos, head_dim/2]")
    kv_dim = kv_heads * head_dim
    _req(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype and k_cache.is_contiguous()
         and v_cache.is_contiguous(), "k/v caches must match and be contiguous")
    num_slots = k_cache.shape[0]
    _req(k_cache.numel() == num_slots * kv_dim, "cache row size must equal kv_dim")
    _dev_i32(positions, "positions", n)
    _dev_i32(slots, "slots", n)
    if bias is not None:
        _req(bias.dtype == torch.float32 and bias.is_contiguous()
             and bias.numel() == (q_heads + 2 * kv_heads) * head_dim, "bias: fp32 [q_dim + 2*kv_dim]")
    if q_out is None:
        q_out = torch.empty(n, q_heads * head_dim, dtype=qkv.dtype, device=qkv.device)
    check("le_rope_kv_cache_write", _lib.load().le_rope_kv_cache_write(
        _p(qkv), _dt(qkv), qkv.stride(0), None if bias is None else _p(bias), _p(positions), _p(slots),
        _p(cos_t), _p(sin_t), cos_t.shape[0], n, q_heads, kv_heads, head_dim, _p(q_out), _p(k_cache),
        _p(v_cache), _dt(k_cache), num_slots, _stream(stream)))
    return q_out


def argmax_rows(logits: torch.Tensor, stream=None) -> torch.Tensor:
    """First-maximum index of each row of fp32 logits [rows, vocab] (sampler.cpp:9-13)."""
    _req(logits.dtype == torch.float32 and logits.dim() == 2 and logits.is_contiguous() and logits.is_cuda,
         "logits: contiguous fp32 cuda [rows, vocab]")
    out = torch.empty(logits.shape[0], dtype=torch.int32, device=logits.device)
    check("le_argmax_rows", _lib.load().le_argmax_rows(_p(logits), logits.shape[0], logits.shape[1], _p(out),
                                                       _stream(stream)))
    return out


def new_workspace(nbytes: int, device="cuda") -> torch.Tensor:
    """A workspace for the attention calls: zero-filled once, as the ABI requires
    (the kernels leave its arrival counters at zero after every launch)."""
    return torch.zeros(max(int(nbytes), 1), dtype=torch.uint8, device=device)


def attention_decode_workspace_size(n_tokens: int, q_heads: int, kv_heads: int, head_dim: int) -> int:
    return int(_lib.load().le_attention_decode_workspace_size(n_tokens, q_heads, kv_heads, head_dim))


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     block_tables: torch.Tensor, table_offset: torch.Tensor,
                     token_seq: torch.Tensor, token_pos: torch.Tensor, q_heads: int, kv_heads: int,
                     head_dim: int, block_size: int, scale: float, out: torch.Tensor | None = None,
                     workspace: torch.Tensor | None = None, stream=None) -> torch.Tensor:
    """Paged attention with the reference launcher's arguments
    (launch_attention_decode_gqa, cuda_kernels.h:60-64). q: [N, q_heads*head_dim]."""
    n = q.shape[0]
    _req(q.is_contiguous() and q.numel() == n * q_heads * head_dim, "q: [N, q_heads*head_dim]")
    _req(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype, "k/v caches must match")
    kv_dim = kv_heads * head_dim
    _req(k_cache.numel() % (block_size * kv_dim) == 0, "cache must hold whole blocks")
    num_blocks = k_cache.numel() // (block_size * kv_dim)
    for name, t in (("block_tables", block_tables), ("table_offset", table_offset),
                    ("token_seq", token_seq), ("token_pos", token_pos)):
        _dev_i32(t, name)
    _req(token_seq.numel() >= n and token_pos.numel() >= n, "token_seq/token_pos: N entries")
    if out is None:
        out = torch.empty_like(q)
    _req(out.dtype == q.dtype and out.shape == q.shape and out.is_contiguous(), "out like q")
    need = attention_decode_workspace_size(n, q_heads, kv_heads, head_dim)
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=q.device)
    check("le_attention_decode", _lib.load().le_attention_decode(
        _p(q), _dt(q), _p(k_cache), _p(v_cache), _dt(k_cache), _p(block_tables), _p(table_offset),
        _p(token_seq), _p(token_pos), _p(out), n, q_heads, kv_heads, head_dim, block_size,
        float(scale), num_blocks, _p(workspace), workspace.numel() * workspace.element_size(),
        _stream(stream)))
    return out


@dataclass
class Slice:
    """One scheduler slice (sequence.h:74-80): tokens [start, start+len) of a sequence."""
    seq_key: int
    start: int
    len: int
    needs_logits: bool
    blocks: np.ndarray   # int32 block table of the sequence
    tokens: np.ndarray   # int32 token ids of the sequence


class Plan:
    """A packed step (le_plan_step), its pinned host buffer and its device copy."""

    FIELDS = ("token_ids", "positions", "slots", "token_seq", "tables", "table_offset",
              "cu_seqlens_q", "seq_lens_k", "logit_rows")

    def __init__(self, slices: list[Slice], q_heads: int, kv_heads: int, head_dim: int,
                 block_size: int, kv_dtype: torch.dtype, partition_tokens: int = 0,
                 chunk_partition_tokens: int = 0, device="cuda", pin: bool = True, chunk_q_tile: int = 0,
                 flags: int = 0, table_capacity: int = 0):
        self.cfg = PlanConfig(q_heads, kv_heads, head_dim, block_size, _dt(kv_dtype),
                              partition_tokens, chunk_q_tile, chunk_partition_tokens, flags, table_capacity)
        keep = []
        arr = (StepSlice * max(1, len(slices)))()
        for i, s in enumerate(slices):
            b = np.ascontiguousarray(s.blocks, dtype=np.int32)
            t = np.ascontiguousarray(s.tokens, dtype=np.int32)
            keep += [b, t]
            arr[i] = StepSlice(s.seq_key, s.start, s.len, int(s.needs_logits), b.size,
                               b.ctypes.data, t.ctypes.data)
        self.plan = StepPlan()
        L = _lib.load()
        st = L.le_plan_step(arr, len(slices), ctypes.byref(self.cfg), None, 0, ctypes.byref(self.plan))
        _req(st == _lib.LE_ENOSPACE, f"le_plan_step sizing returned {st}")
        nbytes = int(self.plan.bytes)
        self.host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pin and torch.cuda.is_available())
        check("le_plan_step", L.le_plan_step(arr, len(slices), ctypes.byref(self.cfg),
                                             ctypes.c_void_p(self.host.data_ptr()), nbytes,
                                             ctypes.byref(self.plan)))
        self.device_buf = None
        self.device = device

    # host views of the packed arrays (numpy int32)
    def host_array(self, name: str) -> np.ndarray:
        n = {"token_ids": self.plan.n_tokens, "positions": self.plan.n_tokens,
             "slots": self.plan.n_tokens, "token_seq": self.plan.n_tokens,
             "tables": self.plan.n_table, "table_offset": self.plan.n_seqs,
             "cu_seqlens_q": self.plan.n_slices + 1, "seq_lens_k": self.plan.n_slices,
             "logit_rows": self.plan.n_logits}[name]
        off = getattr(self.plan, "off_" + name)
        return self.host.numpy()[off:off + 4 * n].view(np.int32).copy()

    def upload(self, stream=None) -> "Plan":
        nbytes = int(self.plan.bytes)
        if self.device_buf is None or self.device_buf.numel() < nbytes:
            self.device_buf = torch.empty(nbytes, dtype=torch.uint8, device=self.device)
        check("le_plan_upload", _lib.load().le_plan_upload(
            ctypes.byref(self.plan), ctypes.c_void_p(self.host.data_ptr()),
            ctypes.c_void_p(self.device_buf.data_ptr()), _stream(stream)))
        return self

    def dev_array(self, name: str) -> torch.Tensor:
        n = len(self.host_array(name))
        off = getattr(self.plan, "off_" + name)
        return self.device_buf[off:off + 4 * n].view(torch.int32)

    def workspace_size(self) -> int:
        return int(_lib.load().le_ragged_workspace_size(ctypes.byref(self.plan)))


def ragged_paged_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                           plan: Plan, scale: float, out: torch.Tensor | None = None,
                           workspace: torch.Tensor | None = None, stream=None,
                           k_new: torch.Tensor | None = None, v_new: torch.Tensor | None = None) -> torch.Tensor:
    """Ragged paged attention over a packed step. With k_new/v_new ([N, kv_dim],
    the step's new rows), the rows are first stored at the plan's slots
    (le_ragged_paged_attention_store: inside the attention launch on a decode
    step)."""
    P = plan.plan
    cfg = P.cfg
    n = P.n_tokens
    _req(plan.device_buf is not None, "plan not uploaded")
    _req(q.is_contiguous() and q.numel() == n * cfg.q_heads * cfg.head_dim, "q: [N, q_heads*head_dim]")
    kv_dim = cfg.kv_heads * cfg.head_dim
    _req(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype, "k/v caches must match")
    num_blocks = k_cache.numel() // (cfg.block_size * kv_dim)
    if out is None:
        out = torch.empty_like(q)
    need = plan.workspace_size()
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=q.device)
    if k_new is not None:
        _req(v_new is not None and k_new.shape == v_new.shape == (n, kv_dim) and k_new.dtype == v_new.dtype
             and k_new.is_contiguous() and v_new.is_contiguous(), "k_new, v_new: [N, kv_dim], same dtype")
        check("le_ragged_paged_attention_store", _lib.load().le_ragged_paged_attention_store(
            _p(q), _dt(q), _p(k_new), _p(v_new), _dt(k_new), _p(k_cache), _p(v_cache), _dt(k_cache), num_blocks,
            ctypes.byref(P), float(scale), _p(out), _p(workspace), workspace.numel() * workspace.element_size(),
            _stream(stream)))
        return out
    check("le_ragged_paged_attention", _lib.load().le_ragged_paged_attention(
        _p(q), _dt(q), _p(k_cache), _p(v_cache), _dt(k_cache), num_blocks, ctypes.byref(P),
        float(scale), _p(out), _p(workspace), workspace.numel() * workspace.element_size(),
        _stream(stream)))
    return out


def ragged_paged_attention_qkv(qkv: torch.Tensor, bias: torch.Tensor | None, cos_t: torch.Tensor,
                               sin_t: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                               plan: Plan, scale: float, out: torch.Tensor | None = None,
                               workspace: torch.Tensor | None = None, q_scratch: torch.Tensor | None = None,
                               stream=None, rms_x: torch.Tensor | None = None, rms_eps: float = 1e-6) -> torch.Tensor:
    """A layer's attention from its stacked QKV rows (cuda_model.cu:358-377:
    bias, RoPE, the K/V store and attention). Equals rope_kv_cache_write on the
    plan's positions and slots followed by ragged_paged_attention, bit for bit;
    on a decode-only step all of it runs in the attention launch
    (le_ragged_paged_attention_qkv). qkv: [N, >= (q_heads + 2*kv_heads)*head_dim]
    laid out [q | k | v]; cos_t/sin_t: fp32 [max_pos, head_dim/2]. With rms_x
    ([N, hidden] in qkv's dtype, the residual stream the rows were projected
    from through norm-weighted columns), the pre-attention RMSNorm is folded
    in: each row is scaled by 1/sqrt(mean(x^2) + rms_eps) before its bias
    (le_ragged_paged_attention_qkv_rms)."""
    P = plan.plan
    cfg = P.cfg
    n = P.n_tokens
    _req(plan.device_buf is not None, "plan not uploaded")
    hd, qd, kv_dim = cfg.head_dim, cfg.q_heads * cfg.head_dim, cfg.kv_heads * cfg.head_dim
    _req(qkv.dim() == 2 and qkv.stride(1) == 1 and qkv.shape[0] == n and qkv.shape[1] >= qd + 2 * kv_dim,
         "qkv: [N, >= q_dim + 2*kv_dim] with unit column stride")
    _req(cos_t.dtype == torch.float32 and cos_t.shape == sin_t.shape and cos_t.is_contiguous()
         and sin_t.is_contiguous() and cos_t.shape[1] == hd // 2, "cos/sin: fp32 [max_pos, head_dim/2]")
    if bias is not None:
        _req(bias.dtype == torch.float32 and bias.is_contiguous() and bias.numel() == qd + 2 * kv_dim,
             "bias: fp32 [q_dim + 2*kv_dim]")
    _req(k_cache.shape == v_cache.shape and k_cache.dtype == v_cache.dtype, "k/v caches must match")
    num_blocks = k_cache.numel() // (cfg.block_size * kv_dim)
    if out is None:
        out = torch.empty(n, qd, dtype=qkv.dtype, device=qkv.device)
    if q_scratch is None:
        q_scratch = torch.empty(n, qd, dtype=qkv.dtype, device=qkv.device)
    _req(q_scratch.is_contiguous() and q_scratch.numel() >= n * qd and q_scratch.dtype == qkv.dtype,
         "q_scratch: [N, q_dim] in the activation dtype")
    need = plan.workspace_size()
    if workspace is None or workspace.numel() * workspace.element_size() < need:
        workspace = torch.zeros(max(need, 1), dtype=torch.uint8, device=qkv.device)
    if rms_x is not None:
        _req(rms_x.dtype == qkv.dtype and rms_x.dim() == 2 and rms_x.shape[0] == n and rms_x.is_contiguous(),
             "rms_x: [N, hidden] contiguous, qkv's dtype")
        check("le_ragged_paged_attention_qkv_rms", _lib.load().le_ragged_paged_attention_qkv_rms(
            _p(qkv), _dt(qkv), qkv.stride(0), None if bias is None else _p(bias), _p(rms_x), rms_x.shape[1],
            float(rms_eps), _p(cos_t), _p(sin_t), cos_t.shape[0], _p(k_cache), _p(v_cache), _dt(k_cache),
            num_blocks, ctypes.byref(P), float(scale), _p(out), _p(q_scratch), _p(workspace),
            workspace.numel() * workspace.element_size(), _stream(stream)))
        return out
    check("le_ragged_paged_attention_qkv", _lib.load().le_ragged_paged_attention_qkv(
        _p(qkv), _dt(qkv), qkv.stride(0), None if bias is None else _p(bias), _p(cos_t), _p(sin_t),
        cos_t.shape[0], _p(k_cache), _p(v_cache), _dt(k_cache), num_blocks, ctypes.byref(P), float(scale),
        _p(out), _p(q_scratch), _p(workspace), workspace.numel() * workspace.element_size(),
        _stream(stream)))
    return out
