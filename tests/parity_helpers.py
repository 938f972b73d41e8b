"""Shared helpers of the GPU parity tests: identically dequantised host weights, the oracle call
and the stated bar (max|out - oracle| <= 1e-2 * RMS(oracle); a bf16 output also gets half a bf16
ulp of the oracle value)."""
import json
import os

import numpy as np

from oracle import bf16 as obf16
from oracle import bfp8 as obfp8
from oracle import mlp as omlp

TOL = 1e-2

# With QMLP_MARGINS=<path>, every check appends one JSON line {test, what, kind, ratio} (ratio =
# error / bar; a case passes at <= 1), so a run leaves the margin of every parity case behind.
MARGINS_ENV = "QMLP_MARGINS"


def record_margin(what, kind, ratio):
    path = os.environ.get(MARGINS_ENV)
    if not path:
        return
    test = os.environ.get("PYTEST_CURRENT_TEST", "").split(" (")[0]
    with open(path, "a") as f:
        f.write(json.dumps({"test": test, "what": what, "kind": kind, "ratio": round(float(ratio), 4)}) + "\n")


def bits(t):
    import torch

    return t.contiguous().view(torch.int16).cpu().numpy().view(np.uint16)


def host_matrix(pkg, w, mfmt):
    """fp32 host copy of one bf16 GPU matrix as the kernels see it in matrix format ``mfmt``."""
    if mfmt in ("bfp8", "bf4"):
        q, e8 = pkg.quantize_bf4(w) if mfmt == "bf4" else pkg.quantize_bfp8(w)
        return obfp8.dequantize(q.cpu().numpy(), e8.cpu().numpy())
    return obf16.bits_to_f32(bits(w))


def host_weights(pkg, sd, fmt):
    """fp32 host copies of the identically dequantised weights (keyed by HF name)."""
    gu_fmt, down_fmt = pkg.matrix_formats(fmt)
    return {name: host_matrix(pkg, sd[f"{name}.weight"], down_fmt if name == "down_proj" else gu_fmt)
            for name in ("gate_proj", "up_proj", "down_proj")}


def oracle(xf, hw, residual=True, h_bf16=False, dtype=np.float32):
    return omlp.swiglu(xf, hw["gate_proj"], hw["up_proj"], hw["down_proj"], residual=xf if residual else None,
                       h_bf16=h_bf16, dtype=dtype)


def check(y, ref, what):
    """The stated bar on an fp32 (unrounded) output; returns err / bound."""
    ok, err, bound = omlp.tolerance_ok(y, ref, TOL)
    print(f"{what}: max|err|={err:.4e} bound={bound:.4e} ({err / bound:.2f} of the bar)", flush=True)
    record_margin(what, "fp32", err / bound if bound > 0 else (0.0 if err == 0 else float("inf")))
    assert ok, f"{what}: {err} > {bound}"
    return err / bound


def check_bf16(y, ref, what):
    """A bf16 output cannot be closer to the fp32 oracle than its own rounding: elementwise
    |y - ref| <= 1e-2 * RMS(ref) + half a bf16 ulp of ref."""
    ok, worst, bound = omlp.tolerance_ok_bf16(y, ref, TOL)
    print(f"{what} (bf16 out): max(|err| - half ulp)={worst:.4e} bar={bound:.4e}", flush=True)
    record_margin(what, "bf16", max(worst, 0.0) / bound if bound > 0 else 0.0)
    assert ok, f"{what}: {worst} > {bound}"


def worst_row_ratio(y, ref):
    """max over token rows of max|y - ref| / (1e-2 * RMS of that row of ref): the bar applied row
    by row (a diagnostic for inputs whose rows differ by orders of magnitude)."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1))
    err = np.max(np.abs(y - ref), axis=1)
    return float(np.max(err / (TOL * np.maximum(rms, 1e-300))))


def check_rows(y, ref, what, bf16_out=False):
    """The stated bar applied to each token row on its own (every row of the MLP is an
    independent forward): max|y_m - ref_m| <= 1e-2 * RMS(ref_m) for every row m (plus half a bf16
    ulp of ref for a bf16 output).  Returns the worst row's ratio."""
    y = np.asarray(y, np.float64)
    ref = np.asarray(ref, np.float64)
    rms = np.sqrt(np.mean(ref * ref, axis=1))
    dev = np.abs(y - ref)
    if bf16_out:
        _, e = np.frexp(np.abs(ref))
        dev = dev - np.ldexp(1.0, e - 9)
    ratio = np.max(dev, axis=1) / (TOL * np.maximum(rms, 1e-300))
    worst = float(np.max(ratio))
    print(f"{what}: worst row at {worst:.2f} of the per-row bar (row {int(np.argmax(ratio))})", flush=True)
    record_margin(what, "row-bf16" if bf16_out else "row-fp32", worst)
    assert worst <= 1.0, f"{what}: row {int(np.argmax(ratio))} at {worst:.3f} of the bar"
    return worst



def fp16_h_reference(xf, hw):
    """The output with h rounded to fp16's significand, and the per-element allowance for the
    places where the kernels' fp32 h may legitimately round the other way.

    The kernels compute h in fp32 (products exact, fp32 sums, SiLU through the hardware exp2 and
    reciprocal) and round h * 2^th to fp16.  Where the exact h lies within that fp32 error of an
    fp16 rounding midpoint, the kernel may round to the other neighbour: one fp16 ulp.  The fp32
    error is taken as 2^-24 (16 + 2 sqrt(K) (sum|x w_g| / |g| + sum|x w_u| / |u|)) relative (sums
    of K products: about sqrt(K) ulp of the absolute sum, 2x that here; SiLU and the products a
    few ulp).  Values that scale into fp16's subnormal range (|h| 2^th < 2^-13, th from the
    Cauchy-Schwarz bound, one binade wide of the kernels' own) may be flushed or lose bits: their
    whole value is allowed.  Returns (y_fp16h [M, H] float64, allowance [M, H] float64)."""
    x = np.asarray(xf, np.float64)
    wg, wu, wd = (np.asarray(hw[n], np.float64) for n in ("gate_proj", "up_proj", "down_proj"))
    g, u = x @ wg.T, x @ wu.T
    ax = np.abs(x)
    cg, cu = ax @ np.abs(wg).T, ax @ np.abs(wu).T
    with np.errstate(divide="ignore", invalid="ignore", over="ignore"):
        h = g / (1.0 + np.exp(-g)) * u
        rel = 2.0 ** -24 * (16 + 2 * np.sqrt(x.shape[1]) * (cg / np.abs(g) + cu / np.abs(u)))
    rel = np.where(np.isfinite(rel), rel, np.inf)
    hr = omlp.round_fp16_significand(h)
    m, e = np.frexp(h)
    ulp = np.ldexp(1.0, e - 11)
    t = np.abs(np.ldexp(m, 11))
    mid_dist = np.abs(t - np.floor(t) - 0.5) * ulp  # distance to the nearest midpoint
    near_tie = mid_dist <= rel * np.abs(h)
    gn = np.sqrt((wg * wg).sum(1)).max()
    un = np.sqrt((wu * wu).sum(1)).max()
    bound = (x * x).sum(1) * gn * un * (1 + 1 / 64)
    th = np.where(bound > 0, 15 - np.frexp(bound)[1], 0)
    tiny = np.abs(h) < np.ldexp(1.0, -13 - th)[:, None]
    slack = np.where(tiny, np.abs(h) + ulp, np.where(near_tie, ulp, 0.0))
    return hr @ wd.T, slack @ np.abs(wd).T


def check_fp16_h(y, xf, hw, what, frac=0.02, per_row=False):
    """The kernels' bare MLP output (no residual) against the fp16-h formula (``fp16_h_reference``):
    every element within its rounding-tie allowance plus ``frac`` of the bar (1e-2 x RMS of the
    exact output, or of its token row with ``per_row``).  This separates the one specified rounding
    of h from everything else the kernels do."""
    y = np.asarray(y, np.float64)
    y16, allow = fp16_h_reference(xf, hw)
    exact = oracle(xf, hw, residual=False, dtype=np.float64).astype(np.float64)
    if per_row:
        bar = TOL * np.maximum(np.sqrt(np.mean(exact * exact, axis=1, keepdims=True)), 1e-300)
    else:
        bar = TOL * np.sqrt(np.mean(exact * exact))
    over = float(np.max((np.abs(y - y16) - allow) / bar))
    raw = float(np.max(np.abs(y - y16) / bar))
    print(f"{what} vs the fp16-h formula: {raw:.4f} of the bar, {over:.4f} beyond the tie allowance "
          f"(allowed {frac})", flush=True)
    record_margin(what, "fp16-h", max(over, 0.0) / frac)
    record_margin(what, "fp16-h-raw", raw)  # information only: the distance before the tie allowance
    assert over <= frac, f"{what}: {over:.4f} of the bar beyond the fp16-h formula's tie allowance"
    return over
