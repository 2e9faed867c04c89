"""Error metrics shared by the parity tests. A non-finite value on either side scores inf, so that NaN (which every
comparison, and Python's max, would otherwise pass over) can never satisfy a tolerance."""
import math

import torch


def rel_err_floor(x, y, floor=1e-3):
    """max_i |x_i - y_i| / max(|y_i|, floor * max|y|): per-element relative error with a floor for elements near
    zero (the off-diagonal entries of Q sit near 0)."""
    x = x.detach().double().cpu()
    y = y.detach().double().cpu()
    if not (bool(torch.isfinite(x).all()) and bool(torch.isfinite(y).all())):
        return math.inf
    den = torch.clamp(y.abs(), min=floor * float(y.abs().max()) if y.numel() else 1.0)
    den = torch.where(den > 0, den, torch.ones_like(den))
    return float(((x - y).abs() / den).max()) if y.numel() else 0.0


def rel_err_norm(x, y):
    """||x - y||_F / ||y||_F."""
    x = x.detach().double().cpu()
    y = y.detach().double().cpu()
    if not (bool(torch.isfinite(x).all()) and bool(torch.isfinite(y).all())):
        return math.inf
    return float((x - y).norm() / max(float(y.norm()), 1e-300))
