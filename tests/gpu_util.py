"""Helpers shared by the GPU parity tests (host side only)."""

from __future__ import annotations

import numpy as np
import torch


def to_np(t: torch.Tensor) -> np.ndarray:
    """Device tensor -> numpy (bf16 widened exactly to fp32, e4m3 / uint8 as uint8 codes)."""
    t = t.detach().cpu()
    if t.dtype == torch.bfloat16:
        return t.float().numpy()
    if t.dtype == torch.float8_e4m3fn:
        return t.view(torch.uint8).numpy()
    return t.numpy()


def seeded(shape, seed: int, dtype=torch.float32, device="cuda", scale: float = 1.0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(*shape, generator=g) * scale
    return x.to(dtype).to(device)


def rel_errors(out: np.ndarray, ref: np.ndarray):
    """(max |d| / max |ref|, mean |d| / mean |ref|)."""
    d = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    r = np.abs(ref.astype(np.float64))
    return float(d.max() / max(r.max(), 1e-30)), float(d.mean() / max(r.mean(), 1e-30))


def vtile_permute(codes: np.ndarray) -> np.ndarray:
    """(B, H, T, D) codes -> the FLW_LAYOUT_VTILE byte layout, restated independently of the
    kernel from the layout's definition in include/flower_amd.h."""
    B, H, T, D = codes.shape
    nt = (T + 63) // 64
    padded = np.zeros((B, H, nt * 64, D), np.uint8)
    padded[:, :, :T] = codes
    out = np.zeros((B, H, nt, 64 * D), np.uint8)
    kk = np.arange(64)[:, None]
    d = np.arange(D)[None, :]
    r = kk % 32
    h = (r // 4) % 2
    b = 4 * (r // 8) + r % 4
    off = (d // 32) * 2048 + (kk // 32) * 1024 + ((d % 32) + 32 * h) * 16 + b
    tiles = padded.reshape(B, H, nt, 64, D)
    out[:, :, :, off.reshape(-1)] = tiles.reshape(B, H, nt, 64 * D)
    return out.reshape(-1)
