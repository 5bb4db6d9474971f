"""Shared test helpers (importable as ``helpers`` from every test module)."""
import torch


def rel_err(a: torch.Tensor, b: torch.Tensor) -> float:
    """max|a-b| / max|b|: the parity metric."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = b.abs().max().item()
    return (a - b).abs().max().item() / (den if den > 0 else 1.0)


def equivariance_err(out1: torch.Tensor, out2: torch.Tensor) -> float:
    """max|a-b| / (max|a| + 1e-8), the reference's metric (tests/helpers.py:54-69)."""
    return ((out1 - out2).abs().max() / (out1.abs().max() + 1e-8)).item()
