"""The drop-in boundary through the reference's own launcher signatures:
runs the compiled tests/bridge/bridge_test (fp16 buffers through
launch_store_kv / launch_attention_decode[_gqa], checked against the CPU
oracle inside the program) as a child process."""
import subprocess
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

EXE = Path(__file__).resolve().parent / "bridge" / "bridge_test"


@pytest.mark.parametrize("n_seqs,seed", [(64, 1), (7, 2), (200, 3)])
def test_reference_signatures_fp16(n_seqs, seed):
    assert EXE.exists(), "build it first: make -C tests/bridge (done by __graft_entry__.build())"
    r = subprocess.run([str(EXE), str(n_seqs), str(seed)], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "bridge ok" in r.stdout
