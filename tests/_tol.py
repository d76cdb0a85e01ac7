"""Tolerances of the hot-path parity bar: bf16 outputs within max abs err 2e-2 and
mean relative err 1e-3 (normwise: mean|a-b| / mean|b|); salient sets bit-exact except
rows whose fp32 cosine lies within 1e-6 of tau."""
import numpy as np
import torch

MAX_ABS = 2e-2
MEAN_REL = 1e-3
TAU_BAND = 1e-6


def assert_bf16_close(got, want, max_abs=MAX_ABS, mean_rel=MEAN_REL, what="output"):
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape, (what, g.shape, w.shape)
    assert torch.isfinite(g).all(), f"{what}: non-finite values"
    d = (g - w).abs()
    mx = d.max().item() if d.numel() else 0.0
    rel = (d.mean() / w.abs().mean().clamp_min(1e-30)).item() if d.numel() else 0.0
    assert mx <= max_abs, f"{what}: max abs err {mx:.3e} > {max_abs}"
    assert rel <= mean_rel, f"{what}: mean rel err {rel:.3e} > {mean_rel}"
    return mx, rel


def assert_mask_equal(got_mask, want_mask, cos_ref, tau, band=TAU_BAND, what="salient set"):
    g = np.asarray(got_mask).astype(bool)
    w = np.asarray(want_mask).astype(bool)
    c = np.asarray(cos_ref, dtype=np.float64)
    keep = np.abs(c - tau) > band
    bad = np.nonzero((g != w) & keep)[0]
    assert bad.size == 0, f"{what}: {bad.size} rows differ outside the tau band, e.g. {bad[:8]} cos={c[bad[:8]]}"
    return int((~keep).sum())


def assert_routing_weights(got, want, what="routing weights"):
    """Router weights are bf16 roundings of one fp32 softmax probability: the device's fp32
    (dot-product order, exp) may differ from torch's by a few fp32 ulps, which can move the bf16
    rounding by at most one bf16 ulp of the value. Bar: every weight within one bf16 ulp, and the
    normwise mean relative error within MEAN_REL (1e-3)."""
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape
    ulp = torch.exp2(torch.floor(torch.log2(w.abs().clamp_min(1e-30))) - 7)
    bad = ((g - w).abs() > ulp).nonzero()
    assert bad.numel() == 0, f"{what}: {bad.shape[0]} weights differ by more than one bf16 ulp"
    rel = ((g - w).abs().mean() / w.abs().mean()).item()
    assert rel <= MEAN_REL, f"{what}: mean rel err {rel:.3e} > {MEAN_REL}"
