"""GPU soft_max_ext (mask NULL, max_bias 0) against the oracle's
ggml_compute_forward_soft_max restatement; rows sum to 1."""
import numpy as np
import pytest
import torch

from gpu_helpers import dev

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("shape", [(3, 5, 17), (2, 4, 576), (1, 16, 5184)])
def test_soft_max(mi, ctx, orc, shape):
    x = orc.normal(int(np.prod(shape)), 0, 3).reshape(shape) * np.float32(4.0)
    xd = dev(x)
    out = torch.empty_like(xd)
    ne = list(shape[::-1])
    ctx.soft_max_ext(mi.from_torch(xd, mi.F32, ne), mi.from_torch(out, mi.F32, ne), 0.125)
    ctx.synchronize()
    got = out.cpu().numpy()
    ref = orc.soft_max_ext(x, 0.125)
    assert np.abs(got - ref).max() <= 1e-6
    assert np.abs(got.sum(-1) - 1).max() <= 1e-5
