"""Shared helpers of the test suite (bit views, NaN-aware equality, synthetic data)."""
import numpy as np
import torch

TDT = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
NAME = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float32: "f32"}


def to_torch(bits, dt):
    """numpy bit patterns (uint16) or float32 -> torch tensor of dtype dt."""
    if dt == "f32":
        return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.float32))
    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).view(TDT[dt])


def to_bits(t):
    """torch tensor -> numpy bit patterns (uint16 for 16-bit types, float32 otherwise)."""
    t = t.detach().cpu().contiguous()
    if t.dtype == torch.float32:
        return t.numpy()
    return t.view(torch.int16).numpy().view(np.uint16)


def as_float(bits, dt):
    return to_torch(bits, dt).float().numpy()


def mismatches(a, b, dt):
    """Count of positions whose bit patterns differ, treating any two NaNs as equal."""
    a = np.asarray(a)
    b = np.asarray(b)
    fa, fb = as_float(a, dt), as_float(b, dt)
    same = (a.view(np.uint32) == b.view(np.uint32)) if dt == "f32" else (a == b)
    same |= np.isnan(fa) & np.isnan(fb)
    return int((~same).sum())


def synth(rows, cols, seed, dt, std=1.0, outliers=8, laplace_frac=0.005, laplace_scale=20.0):
    """Seeded N(0, std^2) tensor with outlier channels x50 and a Laplace tail (CPU, dtype dt)."""
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(rows, cols, generator=g) * std
    if outliers:
        oc = torch.randperm(cols, generator=g)[:outliers]
        x[:, oc] *= 50.0
    n = rows * cols
    k = int(n * laplace_frac)
    if k:
        idx = torch.randperm(n, generator=g)[:k]
        u = torch.rand(k, generator=g) - 0.5
        x.view(-1)[idx] = -laplace_scale * std * torch.sign(u) * torch.log1p(-2.0 * u.abs())
    return x.to(TDT[dt])
