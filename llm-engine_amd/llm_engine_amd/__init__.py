"""llm-engine on MI355X: the ragged continuous-batching hot path as gfx950 HIP
kernels behind a C ABI (include/llm_engine_amd.h).

    from llm_engine_amd import kernels
    kernels.store_kv(k, v, slots, k_cache, v_cache)
    kernels.attention_decode(q, k_cache, v_cache, tables, table_offset, token_seq, token_pos, ...)
    plan = kernels.Plan(slices, q_heads, kv_heads, head_dim, block_size, kv_dtype).upload()
    kernels.ragged_paged_attention(q, k_cache, v_cache, plan, scale)
"""
from ._lib import LIB_PATH, LeError, load  # noqa: F401

__all__ = ["LIB_PATH", "LeError", "load"]
