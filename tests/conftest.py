"""pytest configuration: the `gpu` marker and shared fixtures."""
import os
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

GOLDEN = os.path.join(REPO, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, f"ref_{name}.npz"), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


BF16_ULP = 2.0 ** -7  # one bf16 ulp, relative to the value, at most


def gemm_err(got, ref, dtype, extra=None) -> float:
    """Largest ratio of |got - ref| to the elementwise bar of a product accumulated in float32 and stored
    in `dtype`, against a float64 product of the same (already rounded) operands; <= 1 passes.

    bf16: 2^-7 |ref| + 2^-12 max|ref|.  Rounding the float32 sum to bf16 moves it by at most half an ulp
    (2^-8 relative); the float32 accumulation itself by about K 2^-24 of the terms' scale, far below the
    absolute term.  A dropped or doubled 8-wide k chunk at K = 256 moves an element by about 4e-2 of the
    output scale: 180 times the absolute term.  float32: 1e-5 max|ref|.
    `extra`: elementwise slack for a bf16 intermediate that two float32 sums may round to neighbouring
    values (one ulp of each of its terms), or for a result rounded twice: the products add a bias (or
    accumulate into C) after rounding the product to bf16, as the reference's `out + bias` does, which
    is one more half ulp of the product against the exact value (bias_slack)."""
    import torch

    got = torch.as_tensor(got).detach().double().cpu()
    ref = torch.as_tensor(ref).detach().double().cpu()
    assert got.shape == ref.shape, (tuple(got.shape), tuple(ref.shape))
    scale = float(ref.abs().max())
    if dtype == torch.bfloat16:
        bound = ref.abs() * BF16_ULP + scale * 2.0 ** -12
    else:
        bound = torch.full_like(ref, scale * 1e-5)
    if extra is not None:
        bound = bound + torch.as_tensor(extra).detach().double().cpu()
    return float(((got - ref).abs() / bound.clamp_min(1e-300)).max())


@pytest.fixture(scope="session")
def cuda_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    return torch.device("cuda", 0)


def bias_slack(prod, dtype, ulps: float = 0.5):
    """`ulps` bf16 ulps of |prod| (the product rounded before a bias or C is added), 0 for float32."""
    import torch

    if dtype != torch.bfloat16:
        return None
    return torch.as_tensor(prod).detach().double().cpu().abs() * (BF16_ULP * ulps)
