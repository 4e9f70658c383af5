"""The XCD placement guard of split rows (le_xcd_misplacements).

Split rows of a plan launch exchange partials through one XCD's L2, placed
on the assumption that workgroups whose ids are equal modulo 8 share an XCD.
Each partition reports its XCD when it arrives, and a merge whose partitions
were spread over XCDs writes NaN instead of a wrong value. The
LE_PLAN_SIMULATE_MISPLACEMENT flag forces the condition from the host (the
kernels make every workgroup whose bits 3 and 4 of the linear id differ report another XCD),
so the guard's paths run while every kernel still exits normally."""
import numpy as np
import pytest
import torch

from cases import make_case
from gpu_util import device_q, slices_of, to_dev_cache
from llm_engine_amd._lib import LE_PLAN_SIMULATE_MISPLACEMENT, LE_PLAN_WRITE_THROUGH

pytestmark = pytest.mark.gpu


def _setup(gpu):
    from llm_engine_amd import kernels
    # split decode rows (long contexts, 256-token partitions) and split chunk tiles
    ctx = [3000, 2600, 2100, 1800, 900, 1500] + [1200] * 24
    q_len = [200, 1, 1, 1, 130, 1] + [1] * 24
    case = make_case(ctx, q_len=q_len, num_blocks=4096, seed=71, kv_bf16=True)
    q, _ = device_q(case, torch.float32, gpu)
    kc, vc = to_dev_cache(case.k_cache, gpu), to_dev_cache(case.v_cache, gpu)

    def run(flags):
        plan = kernels.Plan(slices_of(case), case.q_heads, case.kv_heads, case.head_dim, case.block_size,
                            kc.dtype, partition_tokens=256, flags=flags).upload()
        assert plan.plan.n_parts > 0 and plan.plan.n_chunk_items > 0
        ws = kernels.new_workspace(plan.workspace_size(), gpu)
        out = kernels.ragged_paged_attention(q, kc, vc, plan, case.scale, workspace=ws)
        torch.cuda.synchronize()
        assert int(ws[:512 * 1024].count_nonzero().item()) == 0  # counters left at zero
        return out.float().cpu().numpy()

    return case, run


def test_misplaced_partials_are_correct_or_nan(gpu):
    from llm_engine_amd import kernels
    case, run = _setup(gpu)
    kernels.xcd_placement_recheck()
    ref = run(LE_PLAN_WRITE_THROUGH)          # placement plays no part
    l2 = run(0)
    if kernels.xcd_misplacements() != 0:
        pytest.skip("this device does not hold the XCD placement; the guard's L2 path is off")
    assert np.array_equal(l2, ref)            # same partials, same merge order

    sim = run(LE_PLAN_SIMULATE_MISPLACEMENT)
    misses = kernels.xcd_misplacements()      # reads, clears, switches to write-through
    groups = sim.reshape(sim.shape[0], case.kv_heads, -1)
    nan = np.isnan(groups).all(axis=2)
    ok = (groups == ref.reshape(groups.shape)).all(axis=2)
    print(f"split groups found spread over XCDs {misses}; (row, kv head) groups poisoned {int(nan.sum())} "
          f"of {nan.size}, exact {int(ok.sum())}")
    # a split group whose partitions all report the same XCD is exact, one
    # whose partitions report two XCDs is NaN
    assert misses > 0 and nan.sum() > 0
    assert np.all(nan | ok)                   # every group is right or all NaN, never wrong

    # after a nonzero count the device stores write-through: the simulation is inert
    assert np.array_equal(run(LE_PLAN_SIMULATE_MISPLACEMENT), ref)
    assert kernels.xcd_misplacements() == 0

    # a recheck probes again and restores the L2 exchange
    kernels.xcd_placement_recheck()
    assert np.array_equal(run(0), ref)
    assert kernels.xcd_misplacements() == 0


@pytest.mark.parametrize("graph", [False, True])
def test_engine_reruns_a_poisoned_step(gpu, graph):
    """The device model copies the misplacement counter back with every step;
    a step whose merges were poisoned runs again (on write-through partials)
    before its tokens are used. With the fault injection on from the first
    step, config 1 must still give the fixture's tokens, after at least one
    re-run."""
    import json
    import sys
    from pathlib import Path
    from llm_engine_amd import kernels
    from llm_engine_amd.engine import Model, sched_config, synthetic_weights
    gold = Path(__file__).resolve().parent / "golden"
    sys.path.insert(0, str(gold))
    from make_config1 import weight_digest
    fx = json.loads((gold / "config1_tokens.json").read_text())
    w = synthetic_weights(fx["arch"], fx["weight_seed"])
    assert weight_digest(w) == fx["weight_digest"]
    kernels.xcd_placement_recheck()
    kernels.xcd_misplacements()
    m = Model(w, fx["num_blocks"], 16, dtype="f32", decode_graph=graph)
    m.set_plan_flags(LE_PLAN_SIMULATE_MISPLACEMENT)
    toks, _ = m.run_greedy(fx["prompts"], [fx["gen"]] * len(fx["prompts"]),
                           sched_config(max_num_batched_tokens=fx["max_num_batched_tokens"]),
                           fragment_blocks=fx["fragment_blocks"])
    reruns = m.placement_reruns
    m.close()
    kernels.xcd_placement_recheck()  # the re-run switched the device to write-through
    print(f"graph {graph}: {reruns} re-run step(s)")
    if reruns == 0:
        pytest.skip("no split row in this run took the L2 exchange (device not on the L2 path)")
    assert reruns >= 1
    assert toks == fx["tokens"]
