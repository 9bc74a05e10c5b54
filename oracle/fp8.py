"""OCP fp8 e4m3fn and bf16 conversions in numpy, written from the format definitions.

e4m3fn: 1 sign, 4 exponent bits (bias 7), 3 mantissa bits; exponent 0 is subnormal with a
2^-9 grid; there are no infinities and S.1111.111 is NaN; the largest finite value is 448.
The fp32 -> e4m3fn rounding is to nearest even and does not saturate: values whose rounding
would pass 448 (|x| > 464; 464 itself is a tie and rounds to the even 448), infinities and NaN
become NaN (0x7F | sign), which is what
torch's float -> float8_e4m3fn cast does (the reference generates fp8 with that cast,
hcu_ops/tests/test_mqa_hist.py:36,49).
"""
import numpy as np


def fp8_decode_table():
    """float32 value of every e4m3fn code 0..255."""
    codes = np.arange(256, dtype=np.uint32)
    e = (codes >> 3) & 0xF
    m = (codes & 7).astype(np.float64)
    mag = np.where(e == 0, m * 2.0 ** -9, (1.0 + m / 8.0) * 2.0 ** (e.astype(np.float64) - 7.0))
    mag = np.where((e == 15) & ((codes & 7) == 7), np.nan, mag)
    val = np.where(codes & 0x80, -mag, mag)
    return val.astype(np.float32)


_TABLE = fp8_decode_table()


def fp8_decode(codes):
    """uint8 codes -> float32 values (exact)."""
    return _TABLE[np.asarray(codes, dtype=np.uint8)]


def fp8_encode(x):
    """float32 -> uint8 e4m3fn codes, round to nearest even, non-saturating (NaN above 464)."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32)
    sign = ((u >> 24) & 0x80).astype(np.uint32)
    a = u & np.uint32(0x7FFFFFFF)
    absx = a.view(np.float32)
    # subnormal grid 2^-9 below 2^-6: round |x| * 512 to the nearest even integer
    sub = np.rint(np.fmin(absx.astype(np.float64), 1.0) * 512.0).astype(np.uint32)
    # normal: keep 3 mantissa bits, RNE on the 20 dropped ones, rebias 127 -> 7
    t = a.astype(np.uint64) + 0x7FFFF + ((a >> 20) & 1)
    nrm = ((t >> 20) - (120 << 3)).astype(np.uint32)
    code = np.where(a < 0x3C800000, sub, nrm)
    code = np.where(a > 0x43E80000, np.uint32(0x7F), code)
    return (code | sign).astype(np.uint8)


def bf16_rne(x):
    """float32 -> bf16 bit patterns (uint16), round to nearest even, NaN -> 0x7FC0."""
    x = np.asarray(x, dtype=np.float32)
    u = x.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(np.isnan(x), np.uint16(0x7FC0), r)


def bf16_to_f32(b):
    """bf16 bit patterns (uint16) -> float32."""
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def float_key(x):
    """Order-preserving uint32 key of float32 scores (sparse_mask_topk.cu:40-43)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32)
    return np.where(b & 0x80000000, ~b, b | np.uint32(0x80000000)).astype(np.uint32)
