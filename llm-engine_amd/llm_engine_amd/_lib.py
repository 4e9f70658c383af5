"""Loads libllm_engine_amd.so (the gfx950 C ABI) with ctypes and declares its
entry points. There is no fallback: if the library is missing, importing the
kernels raises, so nothing silently runs on the CPU instead."""
from __future__ import annotations

import ctypes
from pathlib import Path

import os

# LE_LIB_PATH selects another build of the same library (e.g. a variant under
# test); by default the in-tree build is loaded.
LIB_PATH = Path(os.environ.get("LE_LIB_PATH") or
                Path(__file__).resolve().parent.parent / "lib" / "libllm_engine_amd.so")

LE_OK = 0
LE_EINVAL = -1
LE_EUNSUPPORTED = -2
LE_ENOSPACE = -3
LE_EDEVICE = -4
LE_ETOOLARGE = -5
LE_F32 = 0
LE_BF16 = 1
LE_F16 = 2
LE_PLAN_TWO_LAUNCHES = 2
LE_PLAN_XCD_LOCAL = 4

c_i32p = ctypes.POINTER(ctypes.c_int32)


class StepSlice(ctypes.Structure):
    _fields_ = [
        ("seq_key", ctypes.c_int64),
        ("start", ctypes.c_int32),
        ("len", ctypes.c_int32),
        ("needs_logits", ctypes.c_int32),
        ("num_blocks", ctypes.c_int32),
        ("blocks", ctypes.c_void_p),
        ("tokens", ctypes.c_void_p),
    ]


class PlanConfig(ctypes.Structure):
    _fields_ = [
        ("q_heads", ctypes.c_int32),
        ("kv_heads", ctypes.c_int32),
        ("head_dim", ctypes.c_int32),
        ("block_size", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("partition_tokens", ctypes.c_int32),
        ("chunk_q_tile", ctypes.c_int32),
        ("chunk_partition_tokens", ctypes.c_int32),
        ("flags", ctypes.c_int32),
        ("table_capacity", ctypes.c_int32),
    ]


class StepPlan(ctypes.Structure):
    _fields_ = [
        ("cfg", PlanConfig),
        ("n_tokens", ctypes.c_int32),
        ("n_seqs", ctypes.c_int32),
        ("n_table", ctypes.c_int32),
        ("n_logits", ctypes.c_int32),
        ("n_decode_items", ctypes.c_int32),
        ("n_chunk_items", ctypes.c_int32),
        ("n_combine_items", ctypes.c_int32),
        ("n_parts", ctypes.c_int32),
        ("max_pos", ctypes.c_int32),
        ("n_slices", ctypes.c_int32),
        ("off_token_ids", ctypes.c_int64),
        ("off_positions", ctypes.c_int64),
        ("off_slots", ctypes.c_int64),
        ("off_token_seq", ctypes.c_int64),
        ("off_tables", ctypes.c_int64),
        ("off_table_offset", ctypes.c_int64),
        ("off_cu_seqlens_q", ctypes.c_int64),
        ("off_seq_lens_k", ctypes.c_int64),
        ("off_logit_rows", ctypes.c_int64),
        ("off_decode_items", ctypes.c_int64),
        ("off_chunk_items", ctypes.c_int64),
        ("off_combine_items", ctypes.c_int64),
        ("off_decode_ids", ctypes.c_int64),
        ("decode_ids_stride", ctypes.c_int32),
        ("xcd_local", ctypes.c_int32),
        ("bytes", ctypes.c_int64),
        ("dev", ctypes.c_void_p),
    ]


class SchedConfig(ctypes.Structure):
    _fields_ = [
        ("continuous", ctypes.c_int32),
        ("max_num_seqs", ctypes.c_int32),
        ("max_num_batched_tokens", ctypes.c_int32),
        ("prefill_chunk_size", ctypes.c_int32),
        ("admission_lookahead", ctypes.c_int32),
        ("starvation_wait_steps", ctypes.c_int32),
        ("watermark_blocks", ctypes.c_int32),
        ("reserved_", ctypes.c_int32),
        ("max_queue_wait_seconds", ctypes.c_double),
    ]


_fpp = ctypes.POINTER(ctypes.c_void_p)


class ModelDesc(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int32) for n in ("hidden", "inter", "layers", "q_heads", "kv_heads",
                                              "head_dim", "vocab", "max_pos")] + [
        ("eps", ctypes.c_float), ("theta", ctypes.c_float),
        ("tie_word_embeddings", ctypes.c_int32), ("dtype", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32), ("attention", ctypes.c_int32),
        ("embed", ctypes.c_void_p), ("final_norm", ctypes.c_void_p), ("lm_head", ctypes.c_void_p),
    ] + [(n, _fpp) for n in ("in_norm", "post_norm", "wq", "wk", "wv", "wo", "bq", "bk", "bv",
                              "wgate", "wup", "wdown")] + [("unfused_norms", ctypes.c_int32)]


class RunStats(ctypes.Structure):
    _fields_ = [("steps", ctypes.c_int64), ("prompt_tokens", ctypes.c_int64),
                ("decode_tokens", ctypes.c_int64), ("preemptions", ctypes.c_int64),
                ("seconds", ctypes.c_double), ("decode_seconds", ctypes.c_double),
                ("decode_steps", ctypes.c_int64), ("decode_step_tokens", ctypes.c_int64),
                ("ttft_mean_s", ctypes.c_double), ("latency_mean_s", ctypes.c_double),
                ("plan_seconds", ctypes.c_double), ("decode_context_tokens", ctypes.c_int64)]


# name -> (restype, argtypes). Exactly the symbols include/*.h declare.
SIGNATURES = {
    "le_version": (ctypes.c_char_p, []),
    "le_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "le_embedding": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
                                     ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "le_rmsnorm": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
                                   ctypes.c_int, ctypes.c_float, ctypes.c_void_p]),
    "le_silu_mul": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p]),
    "le_rope": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p]),
    "le_add_inplace": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t,
                                       ctypes.c_void_p]),
    "le_add_bias": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int,
                                    ctypes.c_void_p]),
    "le_kv_cache_write": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int64,
        ctypes.c_void_p]),
    "le_rope_kv_cache_write": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_int, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_int64, ctypes.c_void_p]),
    "le_attention_decode_workspace_size": (ctypes.c_size_t, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]),
    "le_attention_decode": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
        ctypes.c_int64, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "le_plan_step": (ctypes.c_int, [
        ctypes.POINTER(StepSlice), ctypes.c_int, ctypes.POINTER(PlanConfig), ctypes.c_void_p,
        ctypes.c_int64, ctypes.POINTER(StepPlan)]),
    "le_plan_upload": (ctypes.c_int, [
        ctypes.POINTER(StepPlan), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "le_ragged_workspace_size": (ctypes.c_size_t, [ctypes.POINTER(StepPlan)]),
    "le_sched_trace": (ctypes.c_int64, [
        ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.POINTER(SchedConfig), ctypes.c_int,
        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_void_p, ctypes.c_int64]),
    "le_sched_create": (ctypes.c_void_p, [ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(SchedConfig), ctypes.c_int]),
    "le_sched_destroy": (None, [ctypes.c_void_p]),
    "le_sched_add": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int,
                                    ctypes.c_int]),
    "le_sched_has_work": (ctypes.c_int, [ctypes.c_void_p]),
    "le_sched_step": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(StepSlice), ctypes.c_int,
                                     ctypes.POINTER(ctypes.c_int)]),
    "le_sched_done": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]),
    "le_sched_generated": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p,
                                          ctypes.c_int]),
    "le_model_create": (ctypes.c_void_p, [ctypes.POINTER(ModelDesc), ctypes.c_int, ctypes.c_int,
                                          ctypes.POINTER(ctypes.c_int)]),
    "le_model_destroy": (None, [ctypes.c_void_p]),
    "le_model_set_decode_graph": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
    "le_model_graph_replays": (ctypes.c_int64, [ctypes.c_void_p]),
    "le_model_set_plan_flags": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    "le_model_eager_fallbacks": (ctypes.c_int64, [ctypes.c_void_p]),
    "le_model_forward": (ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(StepSlice), ctypes.c_int,
                                        ctypes.c_void_p, ctypes.c_void_p]),
    "le_run_greedy": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.POINTER(SchedConfig), ctypes.c_int, ctypes.c_int, ctypes.c_int,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.POINTER(RunStats)]),
    "le_argmax_rows": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                      ctypes.c_void_p]),
    "le_ragged_paged_attention": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_int64, ctypes.POINTER(StepPlan), ctypes.c_float, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "le_noalloc_scratch_bytes": (ctypes.c_size_t, []),
    "le_ragged_paged_attention_noalloc": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int,
        ctypes.c_int64, ctypes.POINTER(StepPlan), ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p]),
    "le_ragged_paged_attention_store": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p,
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.POINTER(StepPlan), ctypes.c_float,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "le_ragged_paged_attention_qkv": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
        ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.POINTER(StepPlan),
        ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]),
    "le_ragged_paged_attention_qkv_rms": (ctypes.c_int, [
        ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_float,
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_int64,
        ctypes.POINTER(StepPlan), ctypes.c_float, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t,
        ctypes.c_void_p]),
}

_lib = None


def load() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python llm-engine_amd/build.py` "
                "(there is no CPU fallback for these kernels)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class LeError(RuntimeError):
    def __init__(self, fn: str, status: int):
        msg = load().le_status_string(status).decode()
        super().__init__(f"{fn} failed: status {status} ({msg})")
        self.status = status


def check(fn: str, status: int) -> None:
    if status != LE_OK:
        raise LeError(fn, status)
