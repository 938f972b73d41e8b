"""bfloat16 bit helpers (oracle; test infrastructure only).

The reference rounds fp32 destination values to bf16 when it packs tiles.  Its register epilogue
documents the two rounding rules it considered (``scripts/ci/mlp_rounding_policy.py:62-68``,
``round_word``): round-to-nearest-even (bias ``0x7fff + lsb``) and ties-away (bias ``0x8000``).
The build rounds with nearest-even everywhere, like torch's ``.to(torch.bfloat16)``.
"""
import numpy as np


def bits_to_f32(bits):
    """bf16 storage words (uint16) -> float32 values (exact)."""
    bits = np.asarray(bits, dtype=np.uint16)
    return (bits.astype(np.uint32) << np.uint32(16)).view(np.float32)


def f32_to_bits(values, ties_away=False):
    """float32 -> bf16 storage words, round to nearest (even by default, ties-away on request).

    Same word arithmetic as ``round_word`` (``scripts/ci/mlp_rounding_policy.py:62-68``); NaNs are
    kept quiet.  Values that round past the largest finite bf16 become infinity, as in IEEE.
    """
    values = np.ascontiguousarray(values, dtype=np.float32)
    words = values.view(np.uint32).astype(np.uint64)
    if ties_away:
        bias = np.uint64(0x8000)
    else:
        bias = np.uint64(0x7FFF) + ((words >> np.uint64(16)) & np.uint64(1))
    rounded = ((words + bias) >> np.uint64(16)) & np.uint64(0xFFFF)
    nan = np.isnan(values)
    if nan.any():
        rounded[nan] = ((words[nan] >> np.uint64(16)) | np.uint64(0x40)) & np.uint64(0xFFFF)
    return rounded.astype(np.uint16)


def round_f32(values):
    """Round float32 values to the nearest bf16 value (nearest-even) and return them as float32."""
    return bits_to_f32(f32_to_bits(values))


def round_f64(values):
    """Round float64 values to the nearest bf16 value (nearest-even) once, returned as float64.

    Going through float32 with nearest-even would round twice and can land on a bf16 tie that the
    float64 value does not sit on.  The float32 step here rounds to odd instead (truncate toward
    zero, then set the last bit when anything was cut off), which keeps the later nearest-even
    rounding to bf16 exact because float32 carries more than two bits beyond bf16's 8 (Boldo and
    Melquiond, "Emulation of FMA and correctly rounded sums: proved algorithms using rounding to
    odd", IEEE Trans. Computers 57(4), 2008).  Finite inputs within the float32 range only.
    """
    v = np.asarray(values, dtype=np.float64)
    t = v.astype(np.float32)
    away = np.abs(t.astype(np.float64)) > np.abs(v)
    t = np.where(away, np.nextafter(t, np.float32(0)), t).astype(np.float32)  # truncated toward zero
    inexact = t.astype(np.float64) != v
    words = t.view(np.uint32) | inexact.astype(np.uint32)  # round to odd
    return round_f32(words.view(np.float32)).astype(np.float64)

