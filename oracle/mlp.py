"""fp32 SwiGLU MLP formula (oracle; test infrastructure only).

The reference's CPU path for the MLP is the fp32 torch expression
``(silu(a @ G.T) * (a @ U.T)) @ D.T`` (``scripts/ci/mlp-sweep.py:121-126``); its single-device
module applies the same order -- gate linear with SiLU, up linear, multiply, down linear
(``docker/qwen-c2-graft/graft/mlp.py:402-423``) -- and the decoder layer adds the residual stream
afterwards (``docker/qwen-c2-graft/graft/layer.py:352-357``).  This module restates that formula in
numpy float32 (BLAS sgemm accumulates in fp32), plus the same formula in torch for the CPU
baseline timing.
"""
import numpy as np


def silu(v):
    """SiLU in the dtype of ``v``: ``v / (1 + exp(-v))``."""
    v = np.asarray(v)
    one = v.dtype.type(1)
    return v / (one + np.exp(-v))


def epilogue_h_bf16(g, u):
    """The gate/up epilogue with a bf16 intermediate: ``h = bf16(silu(g) * u)`` from float32 g and
    u, rounded once to nearest-even and returned as float32.  The reference's fused gate/up hands
    the down projection a bf16 h (``scripts/ci/fused_1d.py:10-22,121``); its promoted register
    epilogue rounds the fp32 product once (``scripts/ci/mlp_register_epilogue.py:13-30``), the rule
    the bf16-weight kernels follow."""
    from . import bf16 as obf16

    g = np.asarray(g, dtype=np.float32)
    u = np.asarray(u, dtype=np.float32)
    return obf16.round_f32(silu(g) * u)


def round_fp16_significand(v):
    """Round values to fp16's 11 significant bits (nearest-even) with an unbounded exponent range,
    in float64.  Equal to fp16 rounding for every value in fp16's normal range and, as a power-of-two
    scale commutes with such rounding, to the block-float kernels' h = fp16(h * 2^th) * 2^-th for
    every h that their per-token th keeps normal."""
    v = np.asarray(v, dtype=np.float64)
    m, e = np.frexp(v)  # v = m * 2^e, 0.5 <= |m| < 1
    return np.ldexp(np.rint(np.ldexp(m, 11)), e - 11)


def swiglu(x, wg, wu, wd, residual=None, h_bf16=False, dtype=np.float32):
    """``residual + down(silu(gate(x)) * up(x))`` in float32 (or in ``dtype``).

    x: [M, H]; wg, wu: [I, H] (out, in); wd: [H, I]; residual: [M, H] or None.  With ``h_bf16`` the
    intermediate h is rounded to bf16 once (``epilogue_h_bf16``) before the down projection, as the
    bf16-weight path and the reference's fused gate/up keep it.  ``dtype=np.float64`` evaluates
    the same formula in double precision (the bf16 rounding of h then rounds the double product):
    on heavy-tailed data, where the float32 formula's own rounding is a sizeable part of a 1e-2
    bar, it stands in for exact arithmetic.  The result is returned as float32 either way.
    Follows ``scripts/ci/mlp-sweep.py:121-126`` and ``layer.py:357``.
    """
    x = np.asarray(x, dtype=dtype)
    g = x @ np.asarray(wg, dtype=dtype).T
    u = x @ np.asarray(wu, dtype=dtype).T
    if h_bf16:
        from . import bf16 as obf16

        h = obf16.round_f64(silu(g) * u) if dtype == np.float64 else epilogue_h_bf16(g, u)
    else:
        h = silu(g) * u
    y = h @ np.asarray(wd, dtype=dtype).T
    if residual is not None:
        y = y + np.asarray(residual, dtype=dtype)
    return y.astype(np.float32)


def swiglu_torch(x, wg, wu, wd, residual=None):
    """The same formula with torch CPU tensors (float32), exactly the reference's expression
    ``(torch.nn.functional.silu(a @ G.T) * (a @ U.T)) @ D.T`` (``scripts/ci/mlp-sweep.py:126``)."""
    import torch

    y = (torch.nn.functional.silu(x @ wg.T) * (x @ wu.T)) @ wd.T
    if residual is not None:
        y = y + residual
    return y


def rmsnorm(x, weight, eps=1e-6):
    """Zero-centred RMSNorm of each row in float32: ``x / sqrt(mean(x^2) + eps) * (1 + weight)``.

    The decoder's ``ffn_norm`` is the framework RMSNorm with ``add_unit_offset=True`` (the ``+1`` on
    the stored weight, ``docker/qwen-c2-graft/graft/layer.py:110-112,228-237``); the mean runs over
    the hidden dimension.  x: [M, H]; weight: [H].
    """
    x = np.asarray(x, dtype=np.float32)
    w = np.asarray(weight, dtype=np.float32)
    ms = np.mean(x.astype(np.float64) ** 2, axis=1, keepdims=True)
    rstd = (1.0 / np.sqrt(ms + eps)).astype(np.float32)
    return (x * rstd * (np.float32(1) + w)).astype(np.float32)


def norm_swiglu(h, norm_weight, wg, wu, wd, eps=1e-6):
    """The decoder's feed-forward half: ``h + down(silu(gate(n)) * up(n))`` with
    ``n = bf16(rmsnorm(h))`` -- the norm's output is a bf16 tensor that the MLP consumes
    (``layer.py:352-357``).  Returns float32 [M, H]."""
    from . import bf16 as obf16

    n = rmsnorm(h, norm_weight, eps)
    n = obf16.round_f32(n)
    return swiglu(n, wg, wu, wd, residual=h)


def tolerance_ok(actual, expected, rel=1e-2):
    """Parity bar: ``max|actual - expected| <= rel * RMS(expected)``.  Returns (ok, err, bound)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(expected * expected)))
    err = float(np.max(np.abs(actual - expected))) if expected.size else 0.0
    bound = rel * rms
    return err <= bound, err, bound


def tolerance_ok_bf16(actual, expected, rel=1e-2):
    """The same bar for an output rounded to bf16, which cannot be closer to the fp32 oracle than
    its own rounding: elementwise ``|actual - expected| - half a bf16 ulp of expected <=
    rel * RMS(expected)``.  Returns (ok, worst excess, bound)."""
    actual = np.asarray(actual, dtype=np.float64)
    expected = np.asarray(expected, dtype=np.float64)
    rms = float(np.sqrt(np.mean(expected * expected)))
    _, e = np.frexp(np.abs(expected))
    half_ulp = np.ldexp(1.0, e - 9)  # |expected| in [2^(e-1), 2^e): bf16 ulp 2^(e-8)
    worst = float((np.abs(actual - expected) - half_ulp).max()) if expected.size else 0.0
    bound = rel * rms
    return worst <= bound, worst, bound
