"""bfp8 block-float weight format (oracle; test infrastructure only).

Canonical format (the interchange format every test compares against)
-----------------------------------------------------------------------
A weight matrix ``W[rows, cols]`` (bf16, ``cols`` = the reduction dimension K) is cut into groups of
16 consecutive K values.  Each group stores

* one 8-bit exponent ``e8``: the scale of the group is ``2**(e8 - 127)``; ``e8 == 0`` is reserved
  for a group that dequantises to all zeros;
* 16 signed 8-bit mantissas ``q`` in ``[-127, 127]`` (1 sign + 7 magnitude bits).

Quantisation ("max-exponent-per-group rounding"): ``E`` is the largest ``frexp`` exponent of the
non-zero values of the group (so every ``|v| < 2**E``); the scale is ``2**(E - 7)``, i.e.
``e8 = E + 120``; ``q = round_half_even(v / scale)`` clamped to ``[-127, 127]``.  A group whose
``E + 120`` would fall below 1 keeps ``e8 = 1`` (values that small round towards zero).

This is the block-float rule of the reference's BF8_b check, ``bf8_exact``
(``scripts/ci/ordered_cache_hw_plan.py:243-260``): a group is exact when
``v * 2**(7 - shared) `` is an integer of magnitude below 2**7.  The reference groups 16 values
along the tile row (``BF8_GROUP = 16``, ``ordered_cache_hw_plan.py:25``); the GPU library groups
them along K so that one 16-byte load holds one group.

Device ("tiled") format
-----------------------
The GPU library re-encodes the canonical format losslessly for its kernels:

* rows are cut into 16-row tiles and K into 256-value superblocks; a (tile, superblock) block is
  4 K-steps x 1024 mantissa bytes followed by 256 exponent bytes (4352 bytes), blocks ordered
  tile-major;
* inside K-step ``j`` lane ``l`` (row ``r = l % 16``, quarter ``q = l // 16``) owns the 16 bytes at
  ``j*1024 + 16*l``: the mantissas of K values ``256*sb + 64*j + 16*q + (0..15)`` of row ``r``, stored
  excess-128 (``u = q + 128``);
* the exponent dword of lane ``l`` (bytes ``4096 + 4*l .. +3``) holds, for ``j = 0..3``, the scale of
  that lane's group in K-step ``j`` as the high byte of an IEEE half: ``E5 << 2`` with
  ``E5 = e8 - B + 20`` where ``B`` is the largest ``e8`` of the row (0 for an all-zero group);
* a per-row int32 ``rowexp = B - 132`` restores the true scale: ``w = (u - 128) * 2**(E5 - 15) *
  2**rowexp``.

Groups more than 19 binades below their row's largest group do not fit the half-precision window
and are reported (``flushed``); the test data never produces one.

bf4 (the reference's gate/up dtype)
-----------------------------------
The same canonical rule with 3 magnitude bits instead of 7 (``bf8_exact(values, 3)``): scale
``2**(E - 3)`` (``e8 = E + 124``), ``q`` in ``[-7, 7]``.  Its device block (2304 bytes) holds the
mantissas as 4-bit nibbles ``u = q + 8``: for K-step ``j`` of lane ``l`` the 16 values ``v0..v15``
take 8 bytes at ``1024*(j // 2) + 16*l + 8*(j % 2)``; byte ``b`` of the first dword is
``u_b | u_{b+4} << 4`` (``b = 0..3``), of the second ``u_{8+b} | u_{12+b} << 4``; then the same 256
exponent bytes as bfp8 at offset 2048.
"""
import numpy as np

from . import bf16

GROUP = 16
TILE_ROWS = 16
SUPER_K = 256
STEPS = 4
BLOCK_BYTES = STEPS * 1024 + 256
BF4_BLOCK_BYTES = STEPS * 512 + 256
BF16_BLOCK_BYTES = STEPS * 2048
MANTISSA_BITS = {"bfp8": 7, "bf4": 3}
TRAILER_BYTES = 256


def _check_shape(rows, cols):
    if rows <= 0 or cols <= 0 or rows % TILE_ROWS or cols % SUPER_K:
        raise ValueError(f"rows must be a multiple of {TILE_ROWS} and cols of {SUPER_K}: {rows}x{cols}")


def quantize(w_bits, mantissa_bits=7):
    """Canonical block-float quantisation of a bf16 matrix given as uint16 words: bfp8 with 7
    magnitude bits, bf4 with 3.

    Returns ``(q, e8)`` with ``q`` int8 ``[rows, cols]`` and ``e8`` uint8 ``[rows, cols // 16]``.
    Follows the shared-exponent rule of ``scripts/ci/ordered_cache_hw_plan.py:243-260``.
    """
    w_bits = np.asarray(w_bits, dtype=np.uint16)
    rows, cols = w_bits.shape
    if cols % GROUP:
        raise ValueError("cols must be a multiple of 16")
    v = bf16.bits_to_f32(w_bits).astype(np.float64).reshape(rows, cols // GROUP, GROUP)
    if not np.isfinite(v).all():
        raise ValueError("non-finite weight")
    _, ex = np.frexp(v)
    nonzero = v != 0
    shared = np.where(nonzero, ex, -100000).max(axis=2)
    zero_group = ~nonzero.any(axis=2)
    qmax = 2 ** mantissa_bits - 1
    e8 = np.clip(shared + 127 - mantissa_bits, 1, 254)
    e8 = np.where(zero_group, 0, e8)
    scale = np.ldexp(1.0, np.where(zero_group, 1, e8) - 127)
    q = np.clip(np.rint(v / scale[..., None]), -qmax, qmax)
    q = np.where(zero_group[..., None], 0, q)
    return q.astype(np.int8).reshape(rows, cols), e8.astype(np.uint8)


def dequantize(q, e8):
    """Canonical bfp8 -> float32 ``q * 2**(e8 - 127)`` (exact; ``e8 == 0`` gives zeros).

    Computed in float32 when every product is a float32 number (|q| < 2**7 times a power of two
    no larger than 2**121, i.e. ``e8 <= 248``, which covers every bf16 input), else in float64 and
    rounded.  Both give the same bits wherever float32 can hold the exact value
    (``dequantize_f64`` keeps the float64 form as the check)."""
    q = np.asarray(q, dtype=np.int8)
    e8 = np.asarray(e8, dtype=np.uint8)
    if e8.size and int(e8.max()) > 248:
        return dequantize_f64(q, e8)
    rows, cols = q.shape
    table = np.zeros(256, dtype=np.float32)
    table[1:249] = np.ldexp(np.float32(1.0), np.arange(1, 249, dtype=np.int32) - 127)
    out = q.astype(np.float32)
    np.multiply(out.reshape(rows, cols // GROUP, GROUP), table[e8][..., None], out=out.reshape(rows, cols // GROUP, GROUP))
    return out


def dequantize_f64(q, e8):
    """The float64 form of ``dequantize`` (rounded to float32 at the end)."""
    q = np.asarray(q, dtype=np.int8)
    e8 = np.asarray(e8, dtype=np.uint8)
    rows, cols = q.shape
    scale = np.ldexp(1.0, e8.astype(np.int64) - 127)
    scale = np.where(e8 == 0, 0.0, scale)
    out = q.astype(np.float64).reshape(rows, cols // GROUP, GROUP) * scale[..., None]
    return out.reshape(rows, cols).astype(np.float32)


def bf8_exact(values, mantissa_bits=7):
    """True when every 16-group is representable with one shared exponent and ``mantissa_bits``
    magnitude bits.  Same predicate as ``bf8_exact`` in ``scripts/ci/ordered_cache_hw_plan.py:243-260``
    (restated in numpy)."""
    flat = np.asarray(values, dtype=np.float64).reshape(-1, GROUP)
    if not np.isfinite(flat).all():
        return False
    _, exponent = np.frexp(flat)
    nonzero = flat != 0
    if not nonzero.any():
        return True
    shared = np.where(nonzero, exponent, -100000).max(axis=1, keepdims=True)
    scaled = flat * np.ldexp(1.0, (mantissa_bits - shared))
    representable = (scaled == np.round(scaled)) & (np.abs(scaled) < 2 ** mantissa_bits)
    return bool(representable[nonzero].all())


def row_base(e8):
    """Largest exponent of each row (0 for an all-zero row)."""
    return np.asarray(e8, dtype=np.uint8).max(axis=1).astype(np.int32)


def packed_bytes(rows, cols, fmt):
    """Size of the device buffer for one matrix: tiles, then int32 rowexp, then a 256-byte trailer."""
    _check_shape(rows, cols)
    block = {"bfp8": BLOCK_BYTES, "bf4": BF4_BLOCK_BYTES, "bf16": BF16_BLOCK_BYTES}[fmt]
    return (rows // TILE_ROWS) * (cols // SUPER_K) * block + rows * 4 + TRAILER_BYTES


def _device_exponents(e8):
    """Per-group device exponent bytes ``E5 << 2``, the per-row base, and the flush count."""
    base = row_base(e8)
    e5 = e8.astype(np.int32) - base[:, None] + 20
    live = e8 != 0
    flushed = int((live & (e5 < 1)).sum())
    return np.where(live & (e5 >= 1), e5 << 2, 0).astype(np.uint8), base, flushed


def _exponent_block(dev_e, T, C):
    # group index = 16*sb + 4*j + quarter -> lane-major dwords [T, C, quarter, row, step]
    return dev_e.reshape(T, TILE_ROWS, C, STEPS, 4).transpose(0, 2, 4, 1, 3).reshape(T, C, 256)


def pack_tiles_bf4(q, e8):
    """bf4 device tile bytes + per-row exponent + flush count for canonical (q, e8), q in [-7, 7].

    Returns ``(tiles uint8[T*C*2304], rowexp int32[rows], flushed int)``.
    """
    q = np.asarray(q, dtype=np.int8)
    e8 = np.asarray(e8, dtype=np.uint8)
    rows, cols = q.shape
    _check_shape(rows, cols)
    if np.abs(q.astype(np.int16)).max(initial=0) > 7:
        raise ValueError("bf4 mantissas must lie in [-7, 7]")
    T, C = rows // TILE_ROWS, cols // SUPER_K
    dev_e, base, flushed = _device_exponents(e8)
    u = (q.astype(np.int16) + 8).astype(np.uint8)
    # [T, row, C, step, quarter, 16] -> [T, C, step, quarter, row, 16]
    v = u.reshape(T, TILE_ROWS, C, STEPS, 4, GROUP).transpose(0, 2, 3, 4, 1, 5)
    nib = np.concatenate([v[..., 0:4] | (v[..., 4:8] << 4), v[..., 8:12] | (v[..., 12:16] << 4)], axis=-1)
    # [T, C, step, lane, 8] -> [T, C, pair, sub, lane, 8] -> [T, C, pair, lane, sub, 8]
    nib = nib.reshape(T, C, 2, 2, 64, 8).transpose(0, 1, 2, 4, 3, 5).reshape(T, C, 2048)
    tiles = np.concatenate([nib, _exponent_block(dev_e, T, C)], axis=2).reshape(-1)
    return tiles, (base - 132).astype(np.int32), flushed


def dequant_tiles_bf4(tiles, rowexp, rows, cols):
    """Inverse of ``pack_tiles_bf4`` evaluated on the values: float32 ``[rows, cols]``."""
    T, C = rows // TILE_ROWS, cols // SUPER_K
    blk = np.asarray(tiles, dtype=np.uint8).reshape(T, C, BF4_BLOCK_BYTES)
    nib = blk[:, :, :2048].reshape(T, C, 2, 64, 2, 8).transpose(0, 1, 2, 4, 3, 5).reshape(T, C, STEPS, 64, 8)
    lo, hi = nib & 0x0F, nib >> 4
    v = np.concatenate([lo[..., 0:4], hi[..., 0:4], lo[..., 4:8], hi[..., 4:8]], axis=-1)  # [T, C, step, lane, 16]
    v = v.reshape(T, C, STEPS, 4, TILE_ROWS, GROUP).transpose(0, 4, 1, 2, 3, 5)
    v = v.reshape(rows, cols // GROUP, GROUP).astype(np.float64) - 8.0
    ex = blk[:, :, 2048:].reshape(T, C, 4, TILE_ROWS, STEPS).transpose(0, 3, 1, 4, 2)
    e5 = ex.reshape(rows, cols // GROUP).astype(np.int64) >> 2
    scale = np.where(e5 == 0, 0.0, np.ldexp(1.0, e5 - 15))
    rs = np.ldexp(1.0, np.asarray(rowexp, dtype=np.int64))[:, None, None]
    return (v * scale[..., None] * rs).reshape(rows, cols).astype(np.float32)


def pack_tiles(q, e8):
    """Device tile bytes + per-row exponent + flush count for canonical (q, e8).

    Returns ``(tiles uint8[T*C*4352], rowexp int32[rows], flushed int)``.
    """
    q = np.asarray(q, dtype=np.int8)
    e8 = np.asarray(e8, dtype=np.uint8)
    rows, cols = q.shape
    _check_shape(rows, cols)
    T, C = rows // TILE_ROWS, cols // SUPER_K
    base = row_base(e8)
    e5 = e8.astype(np.int32) - base[:, None] + 20
    live = e8 != 0
    flushed = int((live & (e5 < 1)).sum())
    dev_e = np.where(live & (e5 >= 1), e5 << 2, 0).astype(np.uint8)  # [rows, cols/16]
    u = (q.astype(np.int16) + 128).astype(np.uint8)                  # excess-128
    # mantissa: [T, 16 rows, C, 4 steps, 4 quarters, 16] -> [T, C, steps, quarter, row, 16]
    m = u.reshape(T, TILE_ROWS, C, STEPS, 4, GROUP).transpose(0, 2, 3, 4, 1, 5)
    m = m.reshape(T, C, STEPS * 1024)
    # exponents: group index = 16*sb + 4*j + q -> lane-major dwords [T, C, quarter, row, step]
    ex = dev_e.reshape(T, TILE_ROWS, C, STEPS, 4).transpose(0, 2, 4, 1, 3).reshape(T, C, 256)
    tiles = np.concatenate([m, ex], axis=2).reshape(-1)
    return tiles, (base - 132).astype(np.int32), flushed


def pack_tiles_bf16(w_bits):
    """Device tile bytes for bf16 weights: per (tile, superblock, K-step) two 1024-byte halves;
    lane ``l`` owns values ``0..7`` of its 16 in the first half and ``8..15`` in the second."""
    w_bits = np.asarray(w_bits, dtype=np.uint16)
    rows, cols = w_bits.shape
    _check_shape(rows, cols)
    T, C = rows // TILE_ROWS, cols // SUPER_K
    w = w_bits.reshape(T, TILE_ROWS, C, STEPS, 4, 2, 8)       # [.., quarter, half, 8]
    w = w.transpose(0, 2, 3, 5, 4, 1, 6)                      # [T, C, step, half, quarter, row, 8]
    return np.ascontiguousarray(w).reshape(-1).view(np.uint8)


def dequant_tiles(tiles, rowexp, rows, cols):
    """Inverse of ``pack_tiles`` evaluated on the values: float32 ``[rows, cols]``."""
    T, C = rows // TILE_ROWS, cols // SUPER_K
    blk = np.asarray(tiles, dtype=np.uint8).reshape(T, C, BLOCK_BYTES)
    u = blk[:, :, :4096].reshape(T, C, STEPS, 4, TILE_ROWS, GROUP).transpose(0, 4, 1, 2, 3, 5)
    u = u.reshape(rows, cols // GROUP, GROUP).astype(np.float64) - 128.0
    ex = blk[:, :, 4096:].reshape(T, C, 4, TILE_ROWS, STEPS).transpose(0, 3, 1, 4, 2)
    ex = ex.reshape(rows, cols // GROUP).astype(np.int64)
    e5 = ex >> 2
    scale = np.where(e5 == 0, 0.0, np.ldexp(1.0, e5 - 15))
    rs = np.ldexp(1.0, np.asarray(rowexp, dtype=np.int64))[:, None, None]
    return (u * scale[..., None] * rs).reshape(rows, cols).astype(np.float32)


def row_norms(w):
    """L2 norm of every row of a float matrix, in float64."""
    w = np.asarray(w, dtype=np.float64)
    return np.sqrt((w * w).sum(axis=1))
