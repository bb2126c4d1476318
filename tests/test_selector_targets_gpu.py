"""load_teacher on the GPU (selector/targets.py:62-123 in the reference):
targets, row mass and the deferred (unnormalised) mass from the HIP kernels
against oracle/reference_cpu.py's restatement of the reference's torch ops.
Bar: 1e-6 absolute on targets (float32 sums of 7 heads), 1e-5 relative on
row mass, one bfloat16 ulp on the deferred mass (stored in the features' dtype)."""
import numpy as np
import pytest
import torch

import oracle.reference_cpu as rc
from selector.targets import load_teacher

pytestmark = pytest.mark.gpu


def _write(path, L=3, G=4, H=28, QB=37, P=8, D=32, dtype=torch.bfloat16, seed=0):
    g = torch.Generator().manual_seed(seed)
    pooled = torch.rand(1, L, H, QB, QB, generator=g) * 64
    pooled[..., 5, :] = 0.0                             # an all-zero row: eps keeps it finite
    torch.save({"pooled": pooled,
                "pooledQ": torch.randn(1, L, G, QB, P, D, generator=g).to(dtype),
                "pooledK": torch.randn(1, L, G, QB, P, D, generator=g).to(dtype),
                "seq_len": QB * 64 - 10, "block_size": 64, "proto": P}, path)
    return pooled[0], G


@pytest.mark.parametrize("device", ["cpu", "cuda"])
def test_load_teacher_targets_match_reference_ops(tmp_path, device):
    path = tmp_path / "teacher.pt"
    pooled, G = _write(path)
    out = load_teacher(path, device=device)
    et, er, _ = rc.teacher_targets(pooled, G, eps=1e-9, k=1)
    assert out["target"].device.type == device and out["q_feat"].dtype == torch.float32
    assert np.abs(out["target"].cpu().numpy() - et.numpy()).max() <= 1e-6
    np.testing.assert_allclose(out["row_mass"].cpu().numpy(), er.numpy(), rtol=1e-5, atol=1e-6)
    assert torch.equal(out["cmask"].cpu(), torch.tril(torch.ones(37, 37, dtype=torch.bool)))
    assert (out["target"][..., 5, :] == 0).all()
    assert out["meta"]["num_layers"] == 3 and out["meta"]["qb"] == 37 and out["meta"]["proto"] == 8


def test_load_teacher_deferred_mass(tmp_path):
    path = tmp_path / "teacher.pt"
    pooled, G = _write(path, seed=3)
    out = load_teacher(path, device="cuda", eps=1e-7, defer_normalization=True)
    assert out["mass"].dtype == torch.bfloat16 and out["q_feat"].dtype == torch.bfloat16
    assert out["normalization_eps"] == 1e-7
    # Both sides round a float32 mass to bfloat16: equal, or one bf16 ulp
    # apart (relative 2^-7) where the float32 values straddle a rounding point.
    exp = rc.group_mass(pooled, G).to(torch.bfloat16).float().numpy()
    got = out["mass"].float().cpu().numpy()
    assert np.all(np.abs(got - exp) <= 2.0 ** -7 * np.abs(exp))
    assert (got == exp).mean() > 0.99
