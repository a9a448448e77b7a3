"""Independent OCP e4m3fn codec in numpy (test infrastructure only).

ORACLE — used only by tests/, __graft_entry__.smoke() and bench.py's CPU
baseline, to check results against; never by the product path.

Purpose: pin torch's ``Tensor.to(torch.float8_e4m3fn)`` — the byte-level
authority of the reference's FP8 append (attention.py:190, cast after the
clamp at :187-188; dtype chosen at model_runner.py:247) — against a
restatement of the format from its definition (OCP 8-bit floating point
specification, E4M3 "fn" variant):

* 1 sign bit, 4 exponent bits (bias 7), 3 mantissa bits;
* exponent field 0 encodes subnormals m * 2**-9;
* no infinities; S.1111.111 is NaN, so the largest finite value is
  1.110b * 2**8 = 448;
* float -> e4m3fn rounds to nearest, ties to even.  Out-of-range finite
  values are not saturated by torch's cast (they become NaN); inputs here
  are already clamped to +-448 by the reference, so the encoder maps
  |x| > 448 (after rounding) to NaN like torch does.
"""
from __future__ import annotations

import numpy as np

E4M3_MAX = 448.0


def decode_e4m3fn(byte_values: np.ndarray) -> np.ndarray:
    """Bytes (uint8) -> float64 values from the format definition."""
    b = np.asarray(byte_values, dtype=np.uint8).astype(np.int64)
    sign = np.where(b & 0x80, -1.0, 1.0)
    e = (b >> 3) & 0xF
    m = b & 0x7
    sub = m * 2.0 ** -9
    norm = (1.0 + m / 8.0) * np.exp2(e - 7.0)
    val = np.where(e == 0, sub, norm)
    val = np.where((e == 0xF) & (m == 0x7), np.nan, val)
    return sign * val


def _all_finite_codes() -> tuple[np.ndarray, np.ndarray]:
    codes = np.arange(0, 0x7F, dtype=np.int64)  # 0x00 .. 0x7e: +0 .. +448
    return codes, decode_e4m3fn(codes.astype(np.uint8))


def encode_e4m3fn(x: np.ndarray) -> np.ndarray:
    """float32/float64 values -> e4m3fn bytes, round to nearest even.

    Implemented by nearest-neighbour search over the 127 non-negative finite
    codes (exact in float64), with ties broken towards the even code, then
    the sign bit applied.  Deliberately unlike a bit-twiddling encoder so
    that it is an independent check.
    """
    with np.errstate(invalid="ignore"):
        x = np.asarray(x, dtype=np.float64)
    codes, vals = _all_finite_codes()
    ax = np.abs(x)
    idx = np.searchsorted(vals, ax, side="left")  # first code with value >= |x|
    idx = np.clip(idx, 0, len(vals) - 1)
    lo = np.clip(idx - 1, 0, len(vals) - 1)
    d_hi = np.abs(vals[idx] - ax)
    d_lo = np.abs(ax - vals[lo])
    pick_lo = (d_lo < d_hi) | ((d_lo == d_hi) & (codes[lo] % 2 == 0))
    code = np.where(pick_lo, codes[lo], codes[idx])
    # Beyond 448: the midpoint to the (NaN) next code is 464; torch rounds
    # 448 < |x| <= 464 down to 448 and anything larger to NaN.
    code = np.where(ax > 464.0, 0x7F, code)
    code = np.where(np.isnan(x), 0x7F, code)
    sign = np.signbit(x)
    return (code | np.where(sign, 0x80, 0)).astype(np.uint8)


def quantize_per_tensor(x: np.ndarray, scale: float) -> np.ndarray:
    """clamp(float32(x) / float32(scale), -448, 448) -> e4m3fn bytes, with the
    divide done in float32 (IEEE, correctly rounded) like the reference's
    x.float() / scale (attention.py:187-188)."""
    xf = np.asarray(x, dtype=np.float32)
    q = (xf / np.float32(scale)).astype(np.float32)
    q = np.where(np.isnan(q), q, np.clip(q, -E4M3_MAX, E4M3_MAX)).astype(np.float32)
    return encode_e4m3fn(q)
