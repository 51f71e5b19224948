"""End-to-end parity at full model depth on the GPU.

The bench workload (c3: 32-layer 8B-shaped Llama, 8192-token cache, 64 rows in
16 intervals) and c4 (36-layer Qwen3-8B shape, 32768-token cache, 1383 rows in
32 intervals) run three ways on the same seeded inputs: this build's stage, the
reference path restated by the oracle (bf16), and the same restatement in fp32
(model and stale cache upcast exactly) as the control. Per layer and per K/V,
the refreshed rows must meet the reference's own precision-floor gate
(tests/test_packed_cache.py:291-315): this build's max-abs and RMSE error
against fp32 at most twice the reference path's, with an fp32-epsilon floor;
its angular error (1 - cosine) per row at most twice the reference's largest;
and every row the refresh does not select must be bit-identical to the
reference's (rotated K within 0 ulp, copied V and prefix exact).
"""

from __future__ import annotations

import json

import pytest
import torch

import bench
from oracle import reference_path as ref

pytestmark = pytest.mark.gpu


def _stage_three_ways(device, workload):
    from kv_cache_repair_amd.cache import OperatorShim, cache_from_tensors

    model = bench.make_model(device, workload)
    old, old_ids, new_ids = bench.make_request(device, workload)
    intervals = workload.intervals()
    ours = bench.hip_stage(OperatorShim(model), old, old_ids, new_ids, intervals)
    theirs = ref.reference_refresh_stage(model, old, old_ids, new_ids, intervals)
    control_model = model.float()  # in place: the bf16 weights upcast exactly; the bf16 runs are done
    control_old = cache_from_tensors([(l.keys.float(), l.values.float()) for l in old.layers])
    control = ref.reference_refresh_stage(control_model, control_old, old_ids, new_ids, intervals)
    del control_model, control_old, old, model
    return ours, theirs, control


@pytest.mark.parametrize("name", ["c3", "c4"])
def test_full_depth_refresh_within_the_reference_precision_floor(gpu_device, name):
    workload = bench.WORKLOADS[name]
    print(f"full-depth parity: {workload.description}", flush=True)
    ours, theirs, control = _stage_three_ways(gpu_device, workload)
    result = bench.depth_parity(ours, theirs, control, workload.positions())
    summary = {k: v for k, v in result.items() if k != "layers"}
    print(json.dumps({"workload": name, **summary}), flush=True)
    for row in result["layers"]:
        print(f"  layer {row['layer']:2d} {row['part']}: ours-fp32 max {row['ours_vs_fp32']['max_abs']:.4f} "
              f"rmse {row['ours_vs_fp32']['rmse']:.5f} cos {row['ours_vs_fp32']['min_cos']:.6f} | ref-fp32 max "
              f"{row['reference_vs_fp32']['max_abs']:.4f} rmse {row['reference_vs_fp32']['rmse']:.5f} cos "
              f"{row['reference_vs_fp32']['min_cos']:.6f}", flush=True)
    assert len(result["layers"]) == 2 * workload.layers
    assert result["unselected_rows_bit_exact_vs_reference"]
    for row in result["layers"]:
        where = f"{name} layer {row['layer']} {row['part']}"
        assert row["gate"], (where, row)
        ours_angle = 1.0 - row["ours_vs_fp32"]["min_cos"]
        ref_angle = 1.0 - row["reference_vs_fp32"]["min_cos"]
        assert ours_angle <= 2.0 * max(ref_angle, 1e-7), (where, row)
    del ours, theirs, control
    torch.cuda.empty_cache()
