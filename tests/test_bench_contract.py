"""bench.py's contract on the CPU: one GPU only, and the roofline's
algorithmic bytes and flops equal their closed forms for the benchmark
workloads (the figures roofline.achieved divides by the measured time)."""
import subprocess
import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
sys.path.insert(0, str(ROOT))

import bench  # noqa: E402


def test_more_than_one_gpu_exits_with_a_message():
    r = subprocess.run([sys.executable, str(ROOT / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       timeout=120)
    assert r.returncode != 0
    assert "one GPU" in r.stderr


def test_target_bytes_closed_form():
    """64 x 4096 bf16: K and V once per kv head, 64*4096*2*64*2*2 bytes, plus
    q and the output (fp32) and the block tables and per-row metadata."""
    ctx, q_len, _ = bench.workload_shape("target")
    attn, write = bench.algorithmic_bytes(ctx, q_len, 2, 4)
    kv = 64 * 4096 * 2 * 64 * 2 * 2
    assert kv == 134_217_728
    qo = 64 * 14 * 64 * 4 * 2
    tables = 64 * (4096 // 16) * 4
    meta = 64 * 4 * 2 + 64 * 4
    assert attn == kv + qo + tables + meta
    # the scatter: each new row read (fp32) and written (bf16), K and V, plus its slot
    assert write == 64 * 2 * 64 * 2 * (4 + 2) + 64 * 4


def test_config3_chunk_flops_closed_form():
    """Config 3's chunk rows: 4 * q_heads * head_dim * sum over rows of the
    keys attended; the chunk at 0 attends 1..512 keys, the one at 1024
    attends 1025..1536: 786,944 row-keys, 2.82 GFLOP per layer."""
    ctx, q_len, _ = bench.workload_shape("config3")
    assert list(ctx[:2]) == [512, 1536] and list(q_len[:2]) == [512, 512] and int(q_len.sum()) == 1056
    row_keys = sum(range(1, 513)) + sum(range(1025, 1537))
    assert row_keys == 786_944
    assert bench.chunk_flops(ctx, q_len) == 4 * 14 * 64 * row_keys


def test_config2_shape():
    """Config 2: 64 rows, contexts log-uniform in [64, 4096], a 32768-block pool."""
    ctx, q_len, pool = bench.workload_shape("config2")
    assert len(ctx) == 64 and np.all(q_len == 1) and pool == 32768
    assert ctx.min() >= 64 and ctx.max() <= 4096
