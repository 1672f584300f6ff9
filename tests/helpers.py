"""Shared helpers of the test suite (tolerances, tensor <-> numpy bit views)."""
from __future__ import annotations

import numpy as np


def bits16(t) -> np.ndarray:
    """bf16 torch tensor -> uint16 numpy bit patterns (host copy)."""
    import torch
    return t.detach().contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def bits8(t) -> np.ndarray:
    import torch
    return t.detach().contiguous().view(torch.uint8).cpu().numpy()


def np_(t) -> np.ndarray:
    return t.detach().contiguous().cpu().numpy()


def bf16_f32(h: np.ndarray) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_bf16_close(got_bits, ref_bits, rtol=1e-2, what=""):
    """bf16 outputs within the stated relative error, measured per row as ||got - ref||_2 / ||ref||_2.

    Returns (worst row error, worst elementwise error |g - r| / (|r| + rms(r)), exact fraction) so a
    test can report how close the two are beyond the bar.  The norm form is the bar because e4m3
    re-quantization of an intermediate turns a last-bit difference upstream (the fp8 MFMA does not
    round its block sums exactly, unlike the CPU) into a step of one e4m3 code on single elements."""
    g = bf16_f32(got_bits).astype(np.float64)
    r = bf16_f32(ref_bits).astype(np.float64)
    g2 = g.reshape(g.shape[0], -1) if g.ndim > 1 else g[None]
    r2 = r.reshape(r.shape[0], -1) if r.ndim > 1 else r[None]
    assert np.all(np.isfinite(g2)), f"{what}: non-finite output"
    nrm = np.sqrt(np.sum(r2 * r2, axis=1)) + 1e-30
    row = np.sqrt(np.sum((g2 - r2) ** 2, axis=1)) / nrm
    rms = np.sqrt(np.mean(r2 * r2, axis=1, keepdims=True)) + 1e-30
    elem = np.abs(g2 - r2) / (np.abs(r2) + rms)
    worst = float(row.max()) if row.size else 0.0
    exact = float(np.mean(g2 == r2)) if g2.size else 1.0
    print(f"{what}: row error {worst:.3e} (bar {rtol:g}), worst elementwise |g-r|/|r| "
          f"{elementwise_rel(g2, r2):.3e}, exact {exact:.4f}", flush=True)
    assert worst <= rtol, f"{what}: worst row relative error {worst:.3e} > {rtol}"
    return worst, float(elem.max()) if elem.size else 0.0, exact


def elementwise_rel(g2: np.ndarray, r2: np.ndarray) -> float:
    """Worst |g - r| / |r| over the elements whose |r| is at least one bf16 ulp of their row's largest
    |r| (2^(e - 7) for a row maximum in [2^e, 2^(e+1))): smaller references are rounding noise of the
    row's scale, where a relative error says nothing."""
    if not g2.size:
        return 0.0
    rmax = np.max(np.abs(r2), axis=1, keepdims=True)
    ulp = np.where(rmax > 0, np.exp2(np.floor(np.log2(np.where(rmax > 0, rmax, 1.0))) - 7), np.inf)
    keep = np.abs(r2) >= ulp
    if not keep.any():
        return 0.0
    return float(np.max(np.abs(g2 - r2)[keep] / np.abs(r2)[keep]))


def assert_f32_close(got, ref, rtol=1e-4, what=""):
    """fp32 values within rtol relative to the magnitude of the reference (per leading row)."""
    g = np.asarray(got, dtype=np.float64)
    r = np.asarray(ref, dtype=np.float64)
    g2 = g.reshape(g.shape[0], -1)
    r2 = r.reshape(r.shape[0], -1)
    scale = np.max(np.abs(r2), axis=1, keepdims=True) + 1e-30
    worst = float((np.abs(g2 - r2) / scale).max())
    assert np.all(np.isfinite(g2)), f"{what}: non-finite output"
    assert worst <= rtol, f"{what}: worst relative error {worst:.3e} > {rtol}"
    return worst
