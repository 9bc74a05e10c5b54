"""Pins the oracle's fp8 / bf16 conversions (oracle/fp8.py) against torch's independent
implementations and the closed-form values of the formats."""
import numpy as np
import torch

from oracle.fp8 import bf16_rne, float_key, fp8_decode, fp8_decode_table, fp8_encode


def test_fp8_decode_table_matches_torch_all_codes():
    codes = torch.arange(256, dtype=torch.int32).to(torch.uint8)
    ref = codes.view(torch.float8_e4m3fn).float().numpy()
    got = fp8_decode_table()
    nan = np.isnan(ref)
    assert np.array_equal(nan, np.isnan(got))
    assert np.array_equal(ref[~nan].view(np.uint32), got[~nan].view(np.uint32))


def test_fp8_decode_closed_form():
    t = fp8_decode_table()
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0  # largest finite
    assert t[0x01] == 2.0 ** -9  # smallest subnormal
    assert t[0x07] == 7 * 2.0 ** -9  # largest subnormal
    assert t[0x08] == 2.0 ** -6  # smallest normal
    assert t[0x38] == 1.0 and t[0x39] == 1.125
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    assert t[0x80] == 0.0 and np.signbit(t[0x80])
    # 254 finite values, 2 NaNs; the finite ones are strictly increasing over 0x00..0x7E
    pos = t[:0x7F]
    assert np.all(np.diff(pos) > 0)


def test_fp8_encode_matches_torch_random_and_edges():
    g = torch.Generator().manual_seed(7)
    parts = [
        torch.randn(200000, generator=g) * 100,
        torch.randn(50000, generator=g) * 1e-2,
        torch.randn(50000, generator=g) * 1e-3,  # subnormal range of e4m3
        torch.rand(20000, generator=g) * 40 + 440,  # around the 448 / 464 boundary
    ]
    # every exact code value and every midpoint between consecutive codes (RNE ties)
    t = torch.from_numpy(fp8_decode_table()[:0x7F].astype(np.float32))
    mids = (t[1:] + t[:-1]) / 2
    parts += [t, -t, mids, -mids, torch.tensor([0.0, -0.0, 463.99, 464.0, 470.0, 480.0, 1e30, float("inf"),
                                                -float("inf"), float("nan"), 2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11])]
    x = torch.cat(parts).float()
    ref = x.to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    got = fp8_encode(x.numpy())
    # torch maps NaN / overflow to 0x7F or 0xFF; compare NaN-ness separately from the code bits
    ref_nan = (ref & 0x7F) == 0x7F
    got_nan = (got & 0x7F) == 0x7F
    assert np.array_equal(ref_nan, got_nan)
    assert np.array_equal(ref[~ref_nan], got[~ref_nan])


def test_fp8_encode_round_trip_is_identity_on_codes():
    t = fp8_decode_table()
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    assert np.array_equal(fp8_encode(t[codes]), codes)


def test_bf16_rne_matches_torch():
    g = torch.Generator().manual_seed(3)
    x = torch.cat([torch.randn(300000, generator=g) * 10, torch.randn(1000, generator=g) * 1e-38,
                   torch.tensor([0.0, -0.0, float("inf"), -float("inf"), 3.0e38, -3.0e38]),
                   # exact ties: low 16 bits == 0x8000 with even and odd kept bit
                   torch.tensor([0x3F808000, 0x3F818000, 0xBF808000, 0x7F7F8000], dtype=torch.int64)
                   .to(torch.int32).view(torch.float32)]).float()
    ref = x.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    got = bf16_rne(x.numpy())
    assert np.array_equal(ref, got)
    assert bf16_rne(np.array([np.nan], dtype=np.float32))[0] == 0x7FC0


def test_float_key_orders_like_floats():
    g = torch.Generator().manual_seed(5)
    x = torch.cat([torch.randn(10000, generator=g), torch.tensor([0.0, -0.0, float("inf"), -float("inf")])]).numpy()
    k = float_key(x)
    order_k = np.argsort(k, kind="stable")
    xs = x[order_k]
    assert np.all(np.diff(xs) >= 0)
    assert float_key(np.array([0.0], dtype=np.float32))[0] == 0x80000000
    assert float_key(np.array([-0.0], dtype=np.float32))[0] == 0x7FFFFFFF
