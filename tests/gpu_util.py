"""Helpers for GPU parity tests: move a seeded case to the device, run the
oracle on exactly the inputs the device sees."""
from __future__ import annotations

import numpy as np
import torch

import oracle
from cases import AttnCase


def to_dev_cache(c: np.ndarray, dev) -> torch.Tensor:
    """uint16 arrays hold bf16 bits; float16 and float32 map to themselves."""
    if c.dtype == np.uint16:
        return torch.from_numpy(c.view(np.int16)).to(dev).view(torch.bfloat16)
    return torch.from_numpy(c).to(dev)


def from_dev_cache(c: torch.Tensor) -> np.ndarray:
    if c.dtype == torch.bfloat16:
        return c.view(torch.int16).cpu().numpy().view(np.uint16)
    return c.cpu().numpy()


def i32(a, dev) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).to(dev)


def device_q(case: AttnCase, act: torch.dtype, dev) -> tuple[torch.Tensor, np.ndarray]:
    """The device q in `act`, and the fp32 values the device actually holds."""
    if act == torch.bfloat16:
        qh = oracle.bf16_to_f32(oracle.f32_to_bf16(case.q))
        return torch.from_numpy(qh).to(dev).to(torch.bfloat16), qh
    if act == torch.float16:
        qh = oracle.f32_to_f16(case.q).astype(np.float32)
        return torch.from_numpy(qh).to(dev).to(torch.float16), qh
    return torch.from_numpy(case.q).to(dev), case.q


def oracle_out(case: AttnCase, q_f32: np.ndarray) -> np.ndarray:
    return oracle.paged_attention(q_f32, case.k_cache, case.v_cache, case.tables,
                                  case.table_offset, case.token_seq, case.token_pos, case.q_heads,
                                  case.kv_heads, case.head_dim, case.block_size, case.scale)


def max_abs(a, b) -> float:
    return float(np.max(np.abs(np.asarray(a, dtype=np.float64) - np.asarray(b, dtype=np.float64))))


def slices_of(case: AttnCase):
    """Scheduler-style slices for a case (one per sequence, prefill chunks and
    decode rows in case order); token ids are irrelevant to attention."""
    from llm_engine_amd.kernels import Slice
    out = []
    for s in range(len(case.table_len)):
        start = int(case.seq_start[s])
        ln = int(case.seq_qlen[s])
        out.append(Slice(s, start, ln, True, case.blocks_of(s),
                         np.zeros(start + ln, dtype=np.int32)))
    return out


# Element types by name, as the parity tests parametrize them.
TORCH_DT = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}


def round_to(a: np.ndarray, dt: str) -> np.ndarray:
    """fp32 values as a `dt` tensor holds them (host RNE rules of tensor.h)."""
    a = np.asarray(a, dtype=np.float32)
    if dt == "bf16":
        return oracle.bf16_to_f32(oracle.f32_to_bf16(a))
    if dt == "f16":
        return oracle.f32_to_f16(a).astype(np.float32)
    return a


def random_cache(rng: np.random.Generator, shape, dt: str) -> np.ndarray:
    """A host cache in the layout to_dev_cache takes; 16-bit caches hold
    arbitrary bit patterns (a scatter must leave untouched slots as they are)."""
    if dt == "f32":
        return rng.standard_normal(shape, dtype=np.float32)
    bits = rng.integers(0, 2 ** 16, size=shape).astype(np.uint16)
    return bits if dt == "bf16" else bits.view(np.float16)


def emulated_bar(case: AttnCase, q_f32: np.ndarray, want: np.ndarray | None = None, factor: float = 2.0) -> float:
    """The tolerance a 16-bit-cache case is held to: `factor` times the error
    the host emulation of the kernels' roundings (tests/precision.py) makes on
    this very case against the fp32 oracle. Rows of prefill chunks (a
    sequence with more than one row) are emulated as chunk-tile rows."""
    from precision import emulate
    dt = "bf16" if case.k_cache.dtype == np.uint16 else "f16"
    if want is None:
        want = oracle_out(case, q_f32)
    chunk = np.array([case.seq_qlen[s] > 1 for s in case.token_seq])
    bar = factor * float(np.abs(emulate(case, q_f32, dt, chunk) - want).max())
    if dt == "bf16" and chunk.any():
        # split chunk tiles of a bf16 cache carry normalised partials as fp16:
        # each is a convex combination of V rows, rounded with relative error
        # <= 2^-11, and the merge is a convex combination of them
        # (max over live rows: tests may poison unused rows with NaN)
        bar += 2.0 ** -11 * float(np.nanmax(np.abs(_widen_cache(case.v_cache))))
    return bar


def _widen_cache(c: np.ndarray) -> np.ndarray:
    return oracle.bf16_to_f32(c) if c.dtype == np.uint16 else c.astype(np.float32)


def poison_unused(case: AttnCase) -> None:
    """NaN in every cache row that no sequence's live positions map to (the
    rest of each last block, and every block outside the tables): a kernel
    that reads one of them into a live result turns that row's output NaN."""
    bs = case.block_size
    used = np.zeros(case.num_blocks * bs, dtype=bool)
    ctx = case.seq_start + case.seq_qlen
    for s in range(len(ctx)):
        pos = np.arange(int(ctx[s]))
        blocks = case.tables[case.table_offset[s] + pos // bs].astype(np.int64)
        used[blocks * bs + pos % bs] = True
    for c in (case.k_cache, case.v_cache):
        if c.dtype == np.uint16:
            c[~used] = 0x7FC0  # bf16 quiet NaN
        else:
            c[~used] = np.nan
