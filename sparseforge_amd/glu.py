"""GLU gate/up joint mask update (legacy/utils.py:363-479) on the HIP kernels."""
from __future__ import annotations


def glu_joint_update(gate_module, up_module, step, lambda_mid, sample_idx=None):
    raise NotImplementedError("GLU joint mask update: not built on the MI355X path yet")
