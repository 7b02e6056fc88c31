"""Conversions between torch tensors and the oracle's numpy representations."""
import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor -> uint16 bit patterns (host copy)."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, device=None) -> torch.Tensor:
    """uint16 bit patterns -> bf16 tensor."""
    t = torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16)
    return t if device is None else t.to(device)


def f64(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def assert_attention_close(actual, expected, max_abs=2e-2, mean_abs=2e-3):
    """The attention tolerance: max-abs <= 2e-2 and mean-abs <= 2e-3 (bf16 I/O, fp32 acc)."""
    actual = np.asarray(actual, dtype=np.float64)
    err = np.abs(actual - expected)
    assert np.isfinite(actual).all(), "non-finite attention output"
    assert err.max() <= max_abs and err.mean() <= mean_abs, (
        f"max-abs {err.max():.3e} (<= {max_abs}), mean-abs {err.mean():.3e} (<= {mean_abs})")
    return err
