"""Pins for the CPU oracle (no GPU).  Each check is chosen so that a plausible slip -- a wrong tie
rule, a dropped clamp, an off-by-one exponent, a transposed operand -- fails one of them."""
import math

import numpy as np
import pytest

from oracle import bf16, bfp8, c_oracle
from oracle import mlp as omlp


def _bf16_words(rng, shape, scale=1.0):
    return bf16.f32_to_bits((rng.standard_normal(shape) * scale).astype(np.float32))


# ---------------------------------------------------------------- bf16 rounding


def test_rne_and_ties_away_over_every_finite_bin():
    # Same enumeration as scripts/ci/test_mlp_rounding_policy.py:16-27.
    uppers = np.arange(65536, dtype=np.uint32)
    uppers = uppers[(uppers & 0x7F80) != 0x7F80]
    for tail in (0, 0x7FFF, 0x8000, 0x8001, 0xFFFF):
        words = (uppers << 16) | tail
        vals = words.astype(np.uint32).view(np.float32)
        nearest = bf16.f32_to_bits(vals).astype(np.int64)
        away = bf16.f32_to_bits(vals, ties_away=True).astype(np.int64)
        if tail == 0x8000:
            even = (uppers % 2) == 0
            assert np.array_equal(away[even], nearest[even] + 1)
            assert np.array_equal(away[~even], nearest[~even])
        else:
            assert np.array_equal(away, nearest)


def test_rne_matches_torch_cast():
    torch = pytest.importorskip("torch")
    rng = np.random.RandomState(11)
    words = rng.randint(0, 2**32, size=200000, dtype=np.uint64).astype(np.uint32)
    words = words[(words & 0x7F800000) != 0x7F800000]
    vals = words.view(np.float32)
    ours = bf16.f32_to_bits(vals)
    ref = torch.from_numpy(vals.copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, ref)
    # the C oracle's rounding agrees too
    for v in vals[:2000]:
        assert c_oracle.f32_to_bf16_rne(v) == int(bf16.f32_to_bits(np.float32(v))[0])


def test_double_rounding_known_answer():
    # scripts/ci/test_mlp_c1e_pack.py:533-540: one rounding of silu(g)*u gives 0xBEBF, rounding the
    # operands first gives 0xBEC0.
    g = np.array([0xBFB582D0], dtype=np.uint32).view(np.float32)
    u = np.array([0x3FAD03BC], dtype=np.uint32).view(np.float32)
    s = omlp.silu(g)
    assert int(bf16.f32_to_bits(s * u)[0]) == 0xBEBF
    assert int(bf16.f32_to_bits(bf16.round_f32(s) * bf16.round_f32(u))[0]) == 0xBEC0
    # the oracle's bf16 epilogue is the single rounding
    assert int(bf16.f32_to_bits(omlp.epilogue_h_bf16(g, u))[0]) == 0xBEBF


def test_swiglu_with_bf16_h_rounds_only_the_intermediate():
    # With every weight and activation a small power of two the products and sums are exact, so
    # the bf16 intermediate changes the result only through the rounding of h; an h that is
    # already a bf16 value is left alone, one that is not moves to its nearest-even neighbour.
    x = np.array([[0.5, 0.25]], dtype=np.float32)
    wg = np.array([[2.0, 0.0], [0.0, 0.0]], dtype=np.float32)  # g = [1, 0]
    wu = np.array([[1.0, 0.0], [0.0, 4.0]], dtype=np.float32)  # u = [0.5, 1]
    wd = np.array([[1.0, 1.0]], dtype=np.float32)
    h = omlp.silu(np.float32(1.0)) * np.float32(0.5)  # 0.36552..., not a bf16 value
    exact = omlp.swiglu(x, wg, wu, wd)
    rounded = omlp.swiglu(x, wg, wu, wd, h_bf16=True)
    assert exact[0, 0] == np.float32(h)
    assert rounded[0, 0] == bf16.round_f32(np.float32(h))[()]
    assert rounded[0, 0] != exact[0, 0]
    assert abs(float(rounded[0, 0]) - float(h)) <= 2.0 ** -9 * abs(float(h))
    # h already on the bf16 grid (g = 0 gives h = 0): unchanged
    x0 = np.zeros((1, 2), dtype=np.float32)
    assert np.array_equal(omlp.swiglu(x0, wg, wu, wd, h_bf16=True), omlp.swiglu(x0, wg, wu, wd))


def test_double_rounding_changes_a_large_share():
    # scripts/ci/test_mlp_c1e_pack.py:524-530 (same distribution, numpy generator).
    rng = np.random.RandomState(7)
    gate = (rng.standard_normal(200000) * 1.43).astype(np.float32)
    up = (rng.standard_normal(200000) * 1.43).astype(np.float32)
    s = omlp.silu(gate)
    fused = bf16.f32_to_bits(s * up)
    separate = bf16.f32_to_bits(bf16.round_f32(s) * bf16.round_f32(up))
    assert (fused != separate).mean() > 0.25


# ---------------------------------------------------------------- bfp8 quantiser


EDGE_WORDS = [
    [0x0000] * 16,                                    # all zero -> e8 0
    [0x8000] + [0x0000] * 15,                         # negative zero only
    [0x7F7F] + [0x0001] * 15,                         # bf16 max with denormals
    [0x0001, 0x8002, 0x0003] + [0x0000] * 13,         # denormals only (tiny group, e8 clamps to 1)
    [0x3F80, 0x3F81, 0xBF80, 0x3B80] + [0x3C00] * 12, # 1.0 neighbourhood
]


def test_quantise_edge_words_numpy_vs_c():
    words = np.array(EDGE_WORDS, dtype=np.uint16).reshape(len(EDGE_WORDS), 16)
    q, e8 = bfp8.quantize(words)
    qc, ec = c_oracle.quantize(words)
    assert np.array_equal(q, qc) and np.array_equal(e8, ec)
    assert e8[0, 0] == 0 and not q[0].any()
    assert e8[1, 0] == 0 and not q[1].any()
    # 0x7F7F = 255 * 2^120: frexp exponent 128 -> e8 248, 255/2 ties to 128 -> clamp 127
    assert e8[2, 0] == 248 and q[2, 0] == 127
    assert e8[3, 0] == 1  # denormal group: scale floor 2^-126


@pytest.mark.parametrize("scale", [0.02, 1.0, 3e-5, 7e4])
def test_quantise_numpy_matches_c(scale):
    rng = np.random.RandomState(int(scale * 1000) % 997)
    w = _bf16_words(rng, (48, 256), scale)
    q, e8 = bfp8.quantize(w)
    qc, ec = c_oracle.quantize(w)
    assert np.array_equal(q, qc)
    assert np.array_equal(e8, ec)
    assert np.array_equal(bfp8.dequantize(q, e8), c_oracle.dequantize(q, e8))


def test_dequantised_groups_are_block_float_exact():
    # The reference's representability invariant (scripts/ci/ordered_cache_hw_plan.py:243-260).
    rng = np.random.RandomState(3)
    for scale in (0.02, 1.0, 1e-3):
        w = _bf16_words(rng, (64, 512), scale)
        q, e8 = bfp8.quantize(w)
        assert bfp8.bf8_exact(bfp8.dequantize(q, e8))
        assert np.abs(q.astype(np.int32)).max() <= 127


def test_dequantise_float32_form_matches_float64_everywhere():
    """Every (mantissa, exponent) pair: the float32 dequantiser equals the float64 form bit for bit,
    and both equal the closed form q * 2^(e8 - 127) built with Python's exact ldexp."""
    import math

    qs = np.arange(-127, 128, dtype=np.int8)
    for e8 in range(256):
        q = np.tile(qs, 1)[None, :240]  # 240 = 15 groups of 16
        e = np.full((1, 15), e8, dtype=np.uint8)
        a, b = bfp8.dequantize(q, e), bfp8.dequantize_f64(q, e)
        if e8 <= 248:
            assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), e8
        exact = np.array([0.0 if e8 == 0 else math.ldexp(float(v), e8 - 127) for v in q[0]])
        with np.errstate(over="ignore"):
            assert np.array_equal(b[0], exact.astype(np.float32)), e8


def test_round_trip_exact_on_representable_groups():
    rng = np.random.RandomState(5)
    groups = 4096
    q = rng.randint(-127, 128, size=(groups, 16))
    q[:, 0] = np.where(rng.rand(groups) < 0.5, 1, -1) * rng.randint(64, 128, size=groups)  # max |q| in [64, 127]
    E = rng.randint(-40, 40, size=groups)
    v = (q * np.ldexp(1.0, (E - 7))[:, None]).astype(np.float32)
    words = bf16.f32_to_bits(v)
    assert np.array_equal(bf16.bits_to_f32(words), v)  # 7-bit integers times 2^k are exact in bf16
    assert bfp8.bf8_exact(v)
    qq, e8 = bfp8.quantize(words.reshape(groups // 4, 64))
    assert np.array_equal(qq.reshape(groups, 16), q)
    assert np.array_equal(e8.reshape(groups), (E + 120).astype(np.uint8))
    assert np.array_equal(bfp8.dequantize(qq, e8).reshape(groups, 16), v)


def test_brute_force_nearest_on_single_groups():
    rng = np.random.RandomState(9)
    for trial in range(300):
        scale = 10.0 ** rng.uniform(-6, 4)
        words = _bf16_words(rng, (1, 16), scale)
        vals = [float(x) for x in bf16.bits_to_f32(words)[0]]
        q, e8 = bfp8.quantize(words)
        shared = max(math.frexp(v)[1] for v in vals if v != 0)
        assert int(e8[0, 0]) == shared + 120
        s = 2.0 ** (shared - 7)
        for v, got in zip(vals, q[0]):
            best = min(range(-127, 128), key=lambda c: (abs(v - c * s), c % 2))
            assert int(got) == best, (trial, v, s, got, best)


def test_error_is_at_most_half_a_step():
    rng = np.random.RandomState(13)
    w = _bf16_words(rng, (128, 1024), 0.02)
    q, e8 = bfp8.quantize(w)
    v = bf16.bits_to_f32(w).astype(np.float64).reshape(128, 64, 16)
    d = bfp8.dequantize(q, e8).astype(np.float64).reshape(128, 64, 16)
    step = np.ldexp(1.0, e8.astype(np.int64) - 127)[..., None]
    clamped = np.abs(v) > 127.5 * step
    err = np.abs(v - d)
    assert (err[~clamped] <= step.repeat(16, axis=2)[~clamped] / 2).all()
    assert (err[clamped] <= step.repeat(16, axis=2)[clamped]).all()


def test_non_finite_weights_are_rejected():
    w = np.zeros((1, 16), np.uint16)
    w[0, 3] = 0x7F80
    with pytest.raises(ValueError):
        bfp8.quantize(w)
    with pytest.raises(ValueError):
        c_oracle.quantize(w)


# ---------------------------------------------------------------- device tile layout (restated)


def test_tiled_layout_is_a_bijection_and_lossless():
    rng = np.random.RandomState(21)
    rows, cols = 48, 768
    w = _bf16_words(rng, (rows, cols), 0.02)
    q, e8 = bfp8.quantize(w)
    tiles, rowexp, flushed = bfp8.pack_tiles(q, e8)
    assert flushed == 0
    assert tiles.size + rows * 4 + bfp8.TRAILER_BYTES == bfp8.packed_bytes(rows, cols, "bfp8")
    assert np.array_equal(bfp8.dequant_tiles(tiles, rowexp, rows, cols), bfp8.dequantize(q, e8))
    # every mantissa byte appears exactly once
    m = tiles.reshape(-1, bfp8.BLOCK_BYTES)[:, :4096].reshape(-1)
    assert np.array_equal(np.sort(m.astype(np.int64) - 128), np.sort(q.reshape(-1).astype(np.int64)))
    # bf16 tiles are a permutation of the words
    tb = bfp8.pack_tiles_bf16(w).view(np.uint16)
    assert np.array_equal(np.sort(tb), np.sort(w.reshape(-1)))


def test_tiled_layout_reports_groups_outside_the_window():
    rows, cols = 16, 256
    w = np.zeros((rows, cols), np.float32)
    w[:, :16] = 1.0
    w[:, 16:32] = 2.0 ** -19   # 19 binades below: kept
    w[:, 32:48] = 2.0 ** -20   # 20 binades below: outside the fp16 window
    q, e8 = bfp8.quantize(bf16.f32_to_bits(w))
    tiles, rowexp, flushed = bfp8.pack_tiles(q, e8)
    assert flushed == rows
    d = bfp8.dequant_tiles(tiles, rowexp, rows, cols)
    assert (d[:, 16:32] == 2.0 ** -19).all() and (d[:, 32:48] == 0).all()


# ---------------------------------------------------------------- SwiGLU formula


def _brute(x, wg, wu, wd, res):
    M, H = x.shape
    I = wg.shape[0]
    out = np.zeros((M, H))
    for m in range(M):
        h = []
        for n in range(I):
            g = sum(float(x[m, k]) * float(wg[n, k]) for k in range(H))
            u = sum(float(x[m, k]) * float(wu[n, k]) for k in range(H))
            h.append(g / (1.0 + math.exp(-g)) * u)
        for n in range(H):
            out[m, n] = float(res[m, n]) + sum(h[k] * float(wd[n, k]) for k in range(I))
    return out


def _small(seed, M=3, H=32, I=48):
    rng = np.random.RandomState(seed)
    x = rng.standard_normal((M, H)).astype(np.float32)
    wg = (rng.standard_normal((I, H)) * 0.3).astype(np.float32)
    wu = (rng.standard_normal((I, H)) * 0.3).astype(np.float32)
    wd = (rng.standard_normal((H, I)) * 0.3).astype(np.float32)
    res = rng.standard_normal((M, H)).astype(np.float32)
    return x, wg, wu, wd, res


def test_swiglu_matches_float64_brute_force():
    x, wg, wu, wd, res = _small(1)
    got = omlp.swiglu(x, wg, wu, wd, residual=res)
    ref = _brute(x, wg, wu, wd, res)
    assert np.allclose(got, ref, rtol=2e-5, atol=2e-5)


def test_swiglu_float64_matches_brute_force_to_double_precision():
    # the float64 evaluation is the same formula: against the Python-float brute force it agrees
    # to double rounding, and it moves away from the float32 evaluation by float32's error only
    x, wg, wu, wd, res = _small(11)
    ref = _brute(x, wg, wu, wd, res)
    got64 = omlp.swiglu(x, wg, wu, wd, residual=res, dtype=np.float64)
    assert got64.dtype == np.float32
    assert np.allclose(got64, ref, rtol=0, atol=4e-7 * np.abs(ref).max())  # float32 output rounding
    got32 = omlp.swiglu(x, wg, wu, wd, residual=res)
    assert not np.array_equal(got32, got64) and np.allclose(got32, got64, rtol=2e-5, atol=2e-5)


def _nearest_bf16(v):
    """Brute force: the bf16 neighbours of float64 v (exhaustive over the two candidates of its
    exponent), nearest, ties to the even word."""
    lo = int(bf16.f32_to_bits(np.array([v], np.float32))[0])  # some nearby word
    best = None
    for w in range(lo - 2, lo + 3):
        c = float(bf16.bits_to_f32(np.array([w & 0xFFFF], np.uint16))[0])
        key = (abs(c - v), w & 1)
        if best is None or key < best[0]:
            best = (key, c)
    return best[1]


def test_round_f64_rounds_once():
    # a value just above a bf16 tie rounds up; through float32 nearest-even it would land on the
    # tie and go to the even word (1.0)
    assert bf16.round_f64(np.array([1 + 2.0 ** -8 + 2.0 ** -30]))[0] == 1.0078125
    assert float(bf16.round_f32(np.float32(1 + 2.0 ** -8 + 2.0 ** -30))) == 1.0  # the double rounding
    assert bf16.round_f64(np.array([1 + 2.0 ** -8]))[0] == 1.0  # an exact tie: even
    assert bf16.round_f64(np.array([1 + 3 * 2.0 ** -8]))[0] == 1.015625
    rng = np.random.RandomState(3)
    v = rng.standard_normal(3000) * np.exp2(rng.randint(-20, 20, 3000))
    ties = bf16.bits_to_f32(bf16.f32_to_bits(v[:500].astype(np.float32))).astype(np.float64)
    v[:500] = ties * (1 + 2.0 ** -9 * np.sign(rng.standard_normal(500)))  # near the midpoints
    v[500:700] = ties[:200] * (1 + 2.0 ** -9) + rng.choice([-1, 1], 200) * np.abs(ties[:200]) * 2.0 ** -40
    got = bf16.round_f64(v)
    assert all(got[i] == _nearest_bf16(v[i]) for i in range(v.size))


def test_swiglu_float64_rounds_h_once_to_bf16():
    x, wg, wu, wd, _ = _small(12)
    x64, g64, u64, d64 = (a.astype(np.float64) for a in (x, wg, wu, wd))
    g, u = x64 @ g64.T, x64 @ u64.T
    h = np.vectorize(_nearest_bf16)(g / (1 + np.exp(-g)) * u)
    want = (h @ d64.T).astype(np.float32)
    assert np.array_equal(omlp.swiglu(x, wg, wu, wd, h_bf16=True, dtype=np.float64), want)


def test_round_fp16_significand_is_fp16_rounding_in_the_normal_range():
    # numpy's float16 conversion rounds to nearest-even: the two agree on every normal value, and
    # a power-of-two scale commutes with the significand rounding
    rng = np.random.RandomState(7)
    v = rng.standard_normal(20000) * np.exp2(rng.uniform(-13, 15, 20000))
    v = v[(np.abs(v) < 65504) & (np.abs(v) >= 2.0 ** -14)]  # the normal range
    assert np.array_equal(omlp.round_fp16_significand(v), v.astype(np.float16).astype(np.float64))
    ties = np.array([1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, -(1 + 2.0 ** -11)])  # halfway: even
    assert np.array_equal(omlp.round_fp16_significand(ties), [1.0, 1 + 2.0 ** -9, -1.0])
    assert np.array_equal(omlp.round_fp16_significand(v * 2.0 ** -40), omlp.round_fp16_significand(v) * 2.0 ** -40)


def test_swiglu_matches_c_oracle_and_torch_float64():
    torch = pytest.importorskip("torch")
    x, wg, wu, wd, res = _small(2, M=5, H=64, I=96)
    got = omlp.swiglu(x, wg, wu, wd, residual=res)
    assert np.allclose(c_oracle.swiglu(x, wg, wu, wd, residual=res), got, rtol=1e-5, atol=1e-5)
    t = [torch.from_numpy(a).double() for a in (x, wg, wu, wd, res)]
    ref = (torch.nn.functional.silu(t[0] @ t[1].T) * (t[0] @ t[2].T)) @ t[3].T + t[4]
    assert np.allclose(got, ref.numpy(), rtol=1e-5, atol=1e-5)
    # the torch-float32 restatement used for the CPU baseline is the same formula
    tt = [torch.from_numpy(a) for a in (x, wg, wu, wd, res)]
    assert np.allclose(omlp.swiglu_torch(*tt[:4], residual=tt[4]).numpy(), got, rtol=1e-5, atol=1e-5)


def test_swiglu_zero_input_returns_residual():
    x, wg, wu, wd, res = _small(3)
    assert np.array_equal(omlp.swiglu(np.zeros_like(x), wg, wu, wd, residual=res), res)


def test_swiglu_is_exactly_linear_in_the_down_weight():
    x, wg, wu, wd, _ = _small(4)
    a = omlp.swiglu(x, wg, wu, wd)
    b = omlp.swiglu(x, wg, wu, 2.0 * wd)
    assert np.array_equal(b, 2.0 * a)


def test_swiglu_gate_and_up_are_not_interchangeable():
    # a transposed/swapped operand must show: silu is applied to the gate only
    x, wg, wu, wd, _ = _small(5)
    assert not np.allclose(omlp.swiglu(x, wg, wu, wd), omlp.swiglu(x, wu, wg, wd), atol=1e-3)


def test_swiglu_is_invariant_under_intermediate_permutation():
    x, wg, wu, wd, res = _small(6)
    perm = np.random.RandomState(0).permutation(wg.shape[0])
    a = omlp.swiglu(x, wg, wu, wd, residual=res)
    b = omlp.swiglu(x, wg[perm], wu[perm], wd[:, perm], residual=res)
    assert np.allclose(a, b, rtol=1e-5, atol=1e-5)


def test_tolerance_helper():
    ok, err, bound = omlp.tolerance_ok(np.array([1.0, 2.0]), np.array([1.0, 2.01]))
    assert ok and abs(err - 0.01) < 1e-12 and abs(bound - 1e-2 * math.sqrt((1 + 2.01**2) / 2)) < 1e-12
    ok, _, _ = omlp.tolerance_ok(np.array([1.0, 2.1]), np.array([1.0, 2.0]))
    assert not ok


def test_tolerance_helper_bf16():
    """The bf16 bar allows exactly half a bf16 ulp of the expected value on top of the fp32 bar:
    at 5.0 (exponent range [4, 8), ulp 2^-5) a rounded output may sit 2^-6 away for free."""
    exp = np.zeros(1000)
    exp[0] = 5.0
    bar = 1e-2 * 5.0 / math.sqrt(1000)  # 1.58e-3, below the half ulp 2^-6
    err = np.zeros(1000)
    err[0] = 2.0**-6
    ok, worst, bound = omlp.tolerance_ok_bf16(exp + err, exp)
    assert ok and abs(worst) < 1e-15 and abs(bound - bar) < 1e-12
    err[0] = 2.0**-6 + bar * 1.01
    ok, worst, _ = omlp.tolerance_ok_bf16(exp + err, exp)
    assert not ok and abs(worst - bar * 1.01) < 1e-12
    # the unrounded bar alone rejects the first case
    err[0] = 2.0**-6
    assert not omlp.tolerance_ok(exp + err, exp)[0]


# ---------------------------------------------------------------- zero-centred RMSNorm prologue


def test_rmsnorm_matches_torch_float64():
    """Independent implementation: torch's rms_norm in float64 with weight 1 + w."""
    import torch

    rng = np.random.default_rng(11)
    x = (rng.standard_normal((6, 256)) * rng.uniform(0.01, 50, (6, 1))).astype(np.float32)
    w = (rng.standard_normal(256) * 0.3).astype(np.float32)
    for eps in (1e-6, 1e-2):
        got = omlp.rmsnorm(x, w, eps)
        ref = torch.nn.functional.rms_norm(torch.from_numpy(x).double(), (256,),
                                           weight=1 + torch.from_numpy(w).double(), eps=eps).numpy()
        assert np.max(np.abs(got - ref) / (np.abs(ref) + 1e-30)) < 2e-6


def test_rmsnorm_closed_forms():
    """With w = 0 every row's RMS is sqrt(ms / (ms + eps)); a constant row c maps to
    c / sqrt(c^2 + eps); the unit offset matters (w = -1 gives zeros)."""
    rng = np.random.default_rng(12)
    x = rng.standard_normal((5, 512)).astype(np.float32)
    eps = 1e-3
    y = omlp.rmsnorm(x, np.zeros(512, np.float32), eps).astype(np.float64)
    ms = np.mean(x.astype(np.float64) ** 2, axis=1)
    assert np.allclose(np.sqrt(np.mean(y * y, axis=1)), np.sqrt(ms / (ms + eps)), rtol=1e-6)
    c = np.full((1, 64), 0.25, np.float32)
    assert np.allclose(omlp.rmsnorm(c, np.zeros(64, np.float32), eps), 0.25 / np.sqrt(0.0625 + eps), rtol=1e-6)
    assert not np.any(omlp.rmsnorm(x, -np.ones(512, np.float32), eps))


def test_norm_swiglu_composition():
    """The fused feed-forward is the residual plus the MLP of the bf16-rounded norm output, and a
    missing unit offset or a missing rounding would be visible."""
    rng = np.random.default_rng(13)
    H, I, M = 64, 96, 3
    h = rng.standard_normal((M, H)).astype(np.float32) * 4
    nw = (rng.standard_normal(H) * 0.2).astype(np.float32)
    wg, wu, wd = (rng.standard_normal(s).astype(np.float32) * 0.1 for s in ((I, H), (I, H), (H, I)))
    got = omlp.norm_swiglu(h, nw, wg, wu, wd, 1e-6)
    from oracle import bf16 as obf16

    n = obf16.round_f32(omlp.rmsnorm(h, nw, 1e-6))
    assert np.array_equal(got, omlp.swiglu(n, wg, wu, wd, residual=h))
    assert not np.allclose(got, omlp.swiglu(obf16.round_f32(omlp.rmsnorm(h, nw - 1, 1e-6)), wg, wu, wd, residual=h))


# ---------------------------------------------------------------- bf4 (3 magnitude bits)


def test_bf4_round_trip_exact_on_representable_groups():
    """Groups that the reference's predicate with 3 mantissa bits accepts quantise exactly."""
    rng = np.random.RandomState(41)
    groups = 4096
    q = rng.randint(-7, 8, size=(groups, 16))
    q[:, 0] = np.where(rng.rand(groups) < 0.5, 1, -1) * rng.randint(4, 8, size=groups)  # max |q| in [4, 7]
    E = rng.randint(-40, 40, size=groups)
    v = (q * np.ldexp(1.0, (E - 3))[:, None]).astype(np.float32)
    words = bf16.f32_to_bits(v)
    assert bfp8.bf8_exact(v, mantissa_bits=3) and not bfp8.bf8_exact(v * 1.0625, mantissa_bits=3)
    qq, e8 = bfp8.quantize(words.reshape(groups // 4, 64), mantissa_bits=3)
    assert np.array_equal(qq.reshape(groups, 16), q)
    assert np.array_equal(e8.reshape(groups), (E + 124).astype(np.uint8))


def test_bf4_brute_force_nearest_and_c():
    rng = np.random.RandomState(43)
    for trial in range(300):
        scale = 10.0 ** rng.uniform(-6, 4)
        words = _bf16_words(rng, (1, 16), scale)
        vals = [float(x) for x in bf16.bits_to_f32(words)[0]]
        q, e8 = bfp8.quantize(words, mantissa_bits=3)
        shared = max(math.frexp(v)[1] for v in vals if v != 0)
        assert int(e8[0, 0]) == shared + 124
        s = 2.0 ** (shared - 3)
        for v, got in zip(vals, q[0]):
            best = min(range(-7, 8), key=lambda c: (abs(v - c * s), c % 2))
            assert int(got) == best, (trial, v, s, got, best)
    w = _bf16_words(rng, (48, 512), 3e-3)
    qn, en = bfp8.quantize(w, mantissa_bits=3)
    qc, ec = c_oracle.quantize(w, mantissa_bits=3)
    assert np.array_equal(qn, qc) and np.array_equal(en, ec)
    assert bfp8.bf8_exact(bfp8.dequantize(qn, en), mantissa_bits=3)


def test_bf4_tile_layout():
    """pack_tiles_bf4 is lossless and puts a value where the layout description says."""
    rng = np.random.RandomState(47)
    rows, cols = 32, 512
    q, e8 = bfp8.quantize(_bf16_words(rng, (rows, cols), 0.02), mantissa_bits=3)
    tiles, rowexp, flushed = bfp8.pack_tiles_bf4(q, e8)
    assert flushed == 0
    assert tiles.size + rows * 4 + bfp8.TRAILER_BYTES == bfp8.packed_bytes(rows, cols, "bf4")
    assert np.array_equal(bfp8.dequant_tiles_bf4(tiles, rowexp, rows, cols), bfp8.dequantize(q, e8))
    # spot check: row 21 (tile 1, r 5), K = 256 + 64*3 + 16*2 + 13 (sb 1, step 3, quarter 2, v13)
    r, k = 21, 256 + 64 * 3 + 16 * 2 + 13
    lane = 2 * 16 + 5
    blk = tiles.reshape(-1, bfp8.BF4_BLOCK_BYTES)[1 * (cols // 256) + 1]
    byte = blk[1024 * (3 // 2) + 16 * lane + 8 * (3 % 2) + 4 + (13 - 12)]  # second dword, u_{12+1} high nibble
    assert (byte >> 4) == q[r, k] + 8
    with pytest.raises(ValueError):
        bfp8.pack_tiles_bf4(np.full((16, 256), 9, np.int8), np.ones((16, 16), np.uint8))
