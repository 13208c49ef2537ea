"""Seeded inputs and the tolerance check shared by the parity tests.

With PTB_REPORT_ERRORS=1 in the environment the checks also print, for checks that pass, the
largest absolute error and the largest relative error over outputs at least the absolute floor in
size (run pytest with -s to see them)."""
import os

import torch


def _report(what, g, w, atol):
    if not os.environ.get("PTB_REPORT_ERRORS"):
        return
    diff = (g.double() - w.double()).abs().nan_to_num(0.0)
    big = w.double().abs() >= atol
    rel = float((diff[big] / w.double().abs()[big]).max()) if bool(big.any()) else 0.0
    print(f"[errors] {what}: max_abs_err={float(diff.max()):.3g} max_rel_err={rel:.3g} "
          f"(relative over |want| >= {atol:.3g}; {diff.numel()} outputs)", flush=True)


def randn(shape, seed, dtype=torch.bfloat16, std=1.0, mean=0.0):
    """torch.Generator().manual_seed(seed) + randn, as the reference's make_inputs draw inputs
    (validation/pytorchsim/*/..._spec.py:28-36), scaled and cast."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(shape, generator=g) * std + mean).to(dtype)


def rms(t) -> float:
    """Root mean square of a tensor's values (fp64): the output scale absolute tolerances are
    scaled by where outputs are not O(1)."""
    return float(t.detach().double().cpu().pow(2).mean().sqrt())


def assert_close(got, want, rtol, atol, what=""):
    """allclose(got, want, rtol, atol, equal_nan) with the reference verify's report
    (tests/runtime/verify.py:28-69) in the failure message."""
    g = got.detach().float().cpu()
    w = want.detach().float().cpu()
    assert g.shape == w.shape, f"{what}: shape {tuple(g.shape)} != {tuple(w.shape)}"
    ok = torch.allclose(g, w, rtol=rtol, atol=atol, equal_nan=True)
    if ok:
        _report(what, g, w, atol)
    if not ok:
        diff = (g - w).abs().nan_to_num(0.0)
        rel = diff / w.abs().clamp_min(1e-12)
        idx = int(diff.reshape(-1).argmax())
        bad = int((diff > atol + rtol * w.abs()).sum())
        raise AssertionError(
            f"{what}: max_abs_err={float(diff.max()):.6g} max_rel_err={float(rel.max()):.6g} "
            f"worst at {idx}: got={float(g.reshape(-1)[idx])!r} want={float(w.reshape(-1)[idx])!r}; "
            f"{bad}/{diff.numel()} outside (rtol={rtol}, atol={atol})")


def rows_close(got, want, rtol, atol_frac):
    """Per-row bound for outputs whose scale varies by row (late attention rows average more keys,
    so their outputs shrink): |got - want| <= atol_frac * RMS(want row) + rtol * |want|, rows being
    the last dimension.  Returns (ok, report)."""
    g = got.detach().double().cpu()
    w = want.detach().double().cpu()
    d = w.shape[-1]
    g2, w2 = g.reshape(-1, d), w.reshape(-1, d)
    scale = w2.pow(2).mean(dim=1, keepdim=True).sqrt()
    diff = (g2 - w2).abs().nan_to_num(float("inf"))
    bound = atol_frac * scale + rtol * w2.abs()
    bad = diff > bound
    if not bool(bad.any()):
        _report("per-row check", g2, w2, float(atol_frac * scale.mean()))
        return True, ""
    ratio = (diff / bound.clamp_min(1e-30)).reshape(-1)
    idx = int(ratio.argmax())
    return False, (f"{int(bad.sum())}/{bad.numel()} outside the per-row bound; worst at flat {idx}: "
                   f"got={float(g2.reshape(-1)[idx])!r} want={float(w2.reshape(-1)[idx])!r} "
                   f"(row {idx // d}, row RMS {float(scale[idx // d]):.3g})")


def assert_close_rows(got, want, rtol, atol_frac, what=""):
    ok, report = rows_close(got, want, rtol, atol_frac)
    assert ok, f"{what}: {report}"


def bits_equal(got, want):
    """Exact equality of the stored bits (any dtype: floats compared as their bit patterns, so NaN
    payloads and the sign of zero count)."""
    a, b = got.detach().cpu().contiguous(), want.detach().cpu().contiguous()
    if a.dtype != b.dtype or a.shape != b.shape:
        return False
    if a.element_size() == 2:
        return torch.equal(a.view(torch.int16), b.view(torch.int16))
    if a.element_size() == 1:
        return torch.equal(a.view(torch.uint8), b.view(torch.uint8))
    if a.element_size() == 4:
        return torch.equal(a.view(torch.int32), b.view(torch.int32))
    if a.element_size() == 8:
        return torch.equal(a.view(torch.int64), b.view(torch.int64))
    return torch.equal(a, b)
