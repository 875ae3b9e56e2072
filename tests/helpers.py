"""Comparison helpers shared by the parity tests."""
import torch

# tolerances stated by the north star: fp32 paths rtol 1e-4, bf16 paths
# rtol 2e-2 / atol 2e-2 on outputs, gradients and final states.
FP32_RTOL = 1e-4
BF16_RTOL = 2e-2
BF16_ATOL = 2e-2


def assert_parity(actual, expected, dtype, name="", fp32_atol_rel=1e-5):
    """Check `actual` (device or CPU) against the fp64 oracle `expected`.

    fp32: |a-e| <= 1e-4*|e| + fp32_atol_rel*max|e| elementwise.
    bf16: the stated rtol 2e-2 / atol 2e-2, plus a scale-aware bound
          max|a-e| <= 2e-2 * max|e| so that tiny outputs cannot pass
          trivially under the absolute term.
    """
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    scale = e.abs().max().item() if e.numel() else 0.0
    err = (a - e).abs()
    if dtype == torch.float32:
        bound = FP32_RTOL * e.abs() + fp32_atol_rel * max(scale, 1e-30)
        bad = err > bound
        assert not bad.any(), (
            f"{name}: {int(bad.sum())} elements beyond fp32 tolerance; "
            f"max err {err.max().item():.3e}, scale {scale:.3e}")
    else:
        bad = err > BF16_ATOL + BF16_RTOL * e.abs()
        if bad.any():
            idx = torch.nonzero(bad)[:5].tolist()
            show = [(i, a[tuple(i)].item(), e[tuple(i)].item()) for i in idx]
            raise AssertionError(
                f"{name}: {int(bad.sum())}/{e.numel()} elements beyond rtol 2e-2/atol 2e-2; "
                f"max err {err.max().item():.3e}, scale {scale:.3e}; first (index, got, expected): {show}")
        mx = err.max().item() if e.numel() else 0.0
        assert mx <= BF16_RTOL * max(scale, 1e-30), (
            f"{name}: max err {mx:.3e} > 2e-2 * scale {scale:.3e}")


def assert_scaled(actual, expected, name="", frac=BF16_RTOL):
    """Finite, and max|a-e| <= frac * max|e| (the scale-aware half of the bf16
    bound) -- for inputs whose dynamic range puts single bf16 roundings of
    the largest terms above the elementwise atol."""
    a = actual.detach().to("cpu", torch.float64)
    e = expected.detach().to("cpu", torch.float64)
    assert a.shape == e.shape, f"{name}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    assert torch.isfinite(a).all(), f"{name}: non-finite values"
    scale = e.abs().max().item() if e.numel() else 0.0
    mx = (a - e).abs().max().item() if e.numel() else 0.0
    assert mx <= frac * max(scale, 1e-30), f"{name}: max err {mx:.3e} > {frac} * scale {scale:.3e}"
