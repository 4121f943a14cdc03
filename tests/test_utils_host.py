"""Host-side schedule helpers of utils (no GPU): update_mask_penalty_lr (legacy/utils.py:142-180)."""
import math

import pytest
import torch


def _model(n=3):
    from sparseforge_amd.sparse_modeling import SparseLinear

    # SparseLinear instances without running their constructor: the schedule only sets an attribute
    m = torch.nn.Module()
    for i in range(n):
        layer = SparseLinear.__new__(SparseLinear)
        torch.nn.Module.__init__(layer)
        layer.mask_penalty_lr = -1.0
        m.add_module(f"l{i}", layer)
    return m


@pytest.mark.parametrize("schedule", ["linear", "cosine", "constant", "unknown"])
def test_penalty_lr_schedules(schedule):
    from sparseforge_amd.utils import update_mask_penalty_lr

    model = _model()
    lo, hi, total = 0.01, 0.3, 1000
    start = update_mask_penalty_lr(model, 0, total, lo, hi, schedule)
    mid = update_mask_penalty_lr(model, total // 2, total, lo, hi, schedule)
    end = update_mask_penalty_lr(model, 5 * total, total, lo, hi, schedule)  # progress clamps at 1
    assert all(layer.mask_penalty_lr == end for layer in model.children())
    if schedule in ("linear", "cosine"):
        assert start == lo and math.isclose(mid, (lo + hi) / 2) and math.isclose(end, hi)
        quarter = update_mask_penalty_lr(model, total // 4, total, lo, hi, schedule)
        # the cosine ramp starts slower than the linear one
        assert math.isclose(quarter, lo + (hi - lo) * (0.25 if schedule == "linear" else
                                                        0.5 * (1 - math.cos(math.pi / 4))))
    else:
        assert start == mid == end == hi
