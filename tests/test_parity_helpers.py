"""CPU checks of the GPU tests' fp16-h decomposition (``parity_helpers.check_fp16_h``): a float32
emulation of the block-float kernels' arithmetic (fp32 sums, fp32 SiLU, h rounded to fp16 at a
per-token power-of-two scale) passes it, and planted mistakes in that emulation fail it."""
import numpy as np
import pytest

import parity_helpers as ph


def _case(seed, M=64, H=256, I=512):
    rng = np.random.RandomState(seed)
    x = rng.standard_normal((M, H)).astype(np.float32)
    x[:, rng.permutation(H)[:4]] *= 300.0  # outlier channels
    x = ph.obf16.round_f32(x)  # bf16 activations, as the kernels receive them
    w = {n: (rng.standard_normal(s) * 0.02 * np.exp2(rng.uniform(-4, 4, (s[0], 1)))).astype(np.float32)
         for n, s in (("gate_proj", (I, H)), ("up_proj", (I, H)), ("down_proj", (H, I)))}
    return x, w


def _kernel_like(x, w, h_round="fp16", drop_k=None):
    g = x @ w["gate_proj"].T  # float32 sums
    u = x @ w["up_proj"].T
    h = g * u / (np.float32(1) + np.exp(-g))
    gn = np.sqrt((w["gate_proj"].astype(np.float64) ** 2).sum(1)).max()
    un = np.sqrt((w["up_proj"].astype(np.float64) ** 2).sum(1)).max()
    bound = (x.astype(np.float64) ** 2).sum(1) * gn * un * (1 + 1 / 64)
    th = 15 - np.frexp(bound)[1]
    s = np.ldexp(1.0, th)[:, None]
    if h_round == "fp16":
        hk = (h * s).astype(np.float16).astype(np.float64) / s
    else:  # bf16
        hk = ph.obf16.round_f32((h * s).astype(np.float32)).astype(np.float64) / s
    wd = w["down_proj"].astype(np.float64).copy()
    if drop_k is not None:
        wd[:, drop_k] = 0.0
    return hk @ wd.T


def test_kernel_arithmetic_passes():
    for seed in range(3):
        x, w = _case(seed)
        ph.check_fp16_h(_kernel_like(x, w), x, w, f"emulated kernel seed {seed}")
        ph.check_fp16_h(_kernel_like(x, w), x, w, f"emulated kernel seed {seed} per row", per_row=True)


def test_allowance_is_small():
    # the tie allowance covers rare elements only: it is far below the bar almost everywhere
    x, w = _case(5)
    _, allow = ph.fp16_h_reference(x, w)
    exact = ph.oracle(x, w, residual=False, dtype=np.float64)
    bar = ph.TOL * np.sqrt(np.mean(exact.astype(np.float64) ** 2))
    assert np.median(allow) < 0.01 * bar and np.mean(allow > 0.02 * bar) < 0.05


@pytest.mark.parametrize("mistake", ["bf16 h", "dropped K column"])
def test_planted_mistakes_fail(mistake):
    x, w = _case(7)
    y = _kernel_like(x, w, h_round="bf16") if mistake == "bf16 h" else _kernel_like(x, w, drop_k=11)
    with pytest.raises(AssertionError):
        ph.check_fp16_h(y, x, w, mistake)
