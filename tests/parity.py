"""Helpers for GPU parity tests: device buffers through torch (plumbing only),
tolerance checks against the oracle.

Tolerances (BASELINE: rel-err <= 1e-5 fp32, <= 1e-2 bf16; masks bit-exact):
  * normwise:    max|got - ref| <= tol * max|ref|            (tol 1e-5 / 1e-2)
  * elementwise: |got - ref| <= 2 * gamma_K * (|A| |B|)_ij + out_round * |ref|_ij
    where gamma_K = 1.01 * K * 2^-24.  Both the sequential oracle and any
    other summation order are within gamma_K (|A||B|) of the exact product,
    so this bound holds for every order; it is the per-element criterion.
  * ReLU masks: identical wherever |pre-activation| exceeds that bound; any
    flip inside the band is counted and reported.
"""
from __future__ import annotations

import numpy as np
import torch

U = 2.0 ** -24

# Every buffer made by dev()/dev_bf16()/empty() stays referenced until the
# test ends (release_buffers(), called by an autouse fixture), so a pointer
# taken from a temporary, e.g. ptr(dev(x)) inline in a call, stays valid
# while the asynchronous kernel runs.
_KEEP: list = []


def release_buffers() -> None:
    _KEEP.clear()


def _keep(t: torch.Tensor) -> torch.Tensor:
    _KEEP.append(t)
    return t


def dev(a: np.ndarray, device="cuda:0") -> torch.Tensor:
    return _keep(torch.from_numpy(np.ascontiguousarray(a)).to(device))


def dev_bf16(a: np.ndarray, device="cuda:0") -> torch.Tensor:
    """Upload fp32 values as bf16 storage (RNE, the same rounding the oracle applies)."""
    from oracle import oracle as O

    bits = O.pack_bf16(a).view(np.int16)
    return _keep(torch.from_numpy(bits.copy()).to(device).view(torch.bfloat16))


def host(t: torch.Tensor) -> np.ndarray:
    torch.cuda.synchronize()
    if t.dtype == torch.bfloat16:
        bits = t.view(torch.int16).cpu().numpy().view(np.uint16)
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return t.cpu().numpy()


def empty(shape, dtype=torch.float32, fill=np.nan, device="cuda:0") -> torch.Tensor:
    """Output buffer pre-filled with NaN so an unwritten element is caught."""
    t = torch.empty(shape, dtype=dtype, device=device)
    t.fill_(float(fill))
    return _keep(t)


def ptr(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def gemm_bound(A: np.ndarray, B: np.ndarray, K: int) -> np.ndarray:
    """2 * gamma_K * (|A| |B|) in float64."""
    return 2.0 * 1.01 * K * U * (np.abs(A.astype(np.float64)) @ np.abs(B.astype(np.float64)))


def assert_close_gemm(got, ref, bound, tol, out_round=0.0, what=""):
    got = got.astype(np.float64)
    ref = ref.astype(np.float64)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    assert np.all(np.isfinite(got)), f"{what}: non-finite output"
    err = np.abs(got - ref)
    scale = max(np.max(np.abs(ref)), 1e-30)
    rel = float(np.max(err) / scale) if err.size else 0.0
    assert rel <= tol, f"{what}: normwise rel err {rel:.3e} > {tol}"
    allowed = bound + out_round * np.abs(ref) + 1e-38
    bad = err > allowed
    assert not bad.any(), f"{what}: {int(bad.sum())} elements outside the per-element bound; worst " \
                          f"{float(np.max(err - allowed)):.3e}"
    return rel


def mask_flips(y_got, z_ref, band):
    """Count ReLU mask differences; assert every one lies inside the rounding band."""
    m_got = y_got > 0
    m_ref = z_ref > 0
    diff = m_got != m_ref
    outside = diff & (np.abs(z_ref) > band)
    assert not outside.any(), f"{int(outside.sum())} mask flips outside the rounding band"
    return int(diff.sum())


def ce_bounds(logits, lbl, d_ref):
    """Per-element bounds of a softmax-CE against the oracle: exp/log within a
    few ulp on either side and a reordered row sum give, with C classes,
      loss_i:  2 (C + 8) u + 4 u (|max_i| + |lse_i| + |x_{i,y}|)
      dlogit:  (2 (C + 8) u p_ij + 2 u) / M        (p = softmax)."""
    M, C = logits.shape
    L = logits.astype(np.float64)
    mx = L.max(1)
    lse = mx + np.log(np.exp(L - mx[:, None]).sum(1))
    xy = L[np.arange(M), lbl]
    loss_b = 2 * (C + 8) * U + 4 * U * (np.abs(mx) + np.abs(lse) + np.abs(xy))
    t = np.zeros_like(L)
    t[np.arange(M), lbl] = 1.0
    p = d_ref.astype(np.float64) * M + t
    d_b = (2 * (C + 8) * U * np.abs(p) + 2 * U) / M
    return loss_b, d_b


def check_ce(got_rows, got_d, logits, lbl, rows_ref, d_ref, d_round=0.0):
    """CE outputs within ce_bounds (plus d_round relative for a rounded
    gradient) and normwise rel-err 1e-5 (or d_round)."""
    loss_b, d_b = ce_bounds(logits, lbl, d_ref)
    if got_rows is not None:
        err = np.abs(got_rows.astype(np.float64) - rows_ref)
        assert np.all(err <= loss_b), f"loss rows: max excess {np.max(err - loss_b):.3e}"
        assert np.max(err) <= 1e-5 * max(np.max(np.abs(rows_ref)), 1e-30)
    err = np.abs(got_d.astype(np.float64) - d_ref)
    bound = d_b + d_round * np.abs(d_ref)
    assert np.all(err <= bound), f"dlogits: max excess {np.max(err - bound):.3e}"
    assert np.max(err) <= max(1e-5, d_round) * np.max(np.abs(d_ref))
