"""Shared test helpers: device upload/download and the reference's
tolerance rules."""
from __future__ import annotations

import numpy as np
import torch

import oracle


def up(x, dtype=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dtype=dtype, device="cuda")


def up_f16(x):
    """f32 values to an f16 device tensor (RNE, bit-identical to the oracle's)."""
    return torch.from_numpy(oracle.f32_to_f16(x).view(np.float16)).to("cuda")


def down(t):
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()


def full_scale_err(want, got):
    """Worst |want - got| as a fraction of max |want|
    (crates/llmtie-cuda/tests/kernels.rs:53-69, assert_close_to)."""
    want = np.asarray(want, np.float64)
    got = np.asarray(got, np.float64)
    scale = max(np.abs(want).max(), 1e-6)
    return float(np.abs(want - got).max() / scale)


def per_head_cos(want, got, rows, heads, hd):
    w = np.asarray(want, np.float64).reshape(rows, heads, hd).transpose(1, 0, 2).reshape(heads, -1)
    g = np.asarray(got, np.float64).reshape(rows, heads, hd).transpose(1, 0, 2).reshape(heads, -1)
    num = (w * g).sum(1)
    den = np.sqrt((w * w).sum(1) * (g * g).sum(1))
    return num / np.maximum(den, 1e-300)
