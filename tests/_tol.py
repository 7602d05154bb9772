"""Tolerances of the parity tests (the bar BASELINE.json's north_star sets):
  * fp32 results: within 1e-4 relative, measured normwise as
    max|got - ref| / max|ref|;
  * bf16 / fp16 results: within 2e-2 max-abs, with the error measured against
    max(1, max|ref|) so that sums over many rows (weight gradients) are held
    to the same relative bar as O(1) activations.
The reference value is always the fp64 oracle evaluated on the same
(already rounded) inputs the GPU saw."""
import torch

FP32_RTOL = 1e-4
LOWP_ATOL = 2e-2


def err(got: torch.Tensor, ref: torch.Tensor) -> tuple[float, float]:
    g = got.detach().double().cpu()
    r = ref.detach().double().cpu()
    assert g.shape == r.shape, (g.shape, r.shape)
    assert torch.isfinite(g).all(), "non-finite values in GPU result"
    diff = (g - r).abs().max().item() if g.numel() else 0.0
    scale = r.abs().max().item() if r.numel() else 0.0
    return diff, scale


def assert_close(got, ref, dtype, what=""):
    diff, scale = err(got, ref)
    if dtype == torch.float32:
        bound = FP32_RTOL * max(scale, 1e-30)
    else:
        bound = LOWP_ATOL * max(1.0, scale)
    assert diff <= bound, f"{what}: max|diff| {diff:.3e} > {bound:.3e} (max|ref| {scale:.3e})"
