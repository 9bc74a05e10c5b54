"""CPU checks of the tests' nonzero-mask checker (gpu_util.check_mask): it accepts a kernel zero at a
logit within the tolerance of zero, and rejects a mask that disagrees with the kernel's own logits
or with the oracle at a logit away from zero."""
import numpy as np
import pytest

from oracle import indexer as O
from gpu_util import check_mask


def _case():
    width = 32
    lens = np.array([30, 17])
    ref = np.full((2, width), np.nan)
    ref[0, :30] = np.linspace(-3, 3, 30)
    ref[1, :17] = np.linspace(1, 2, 17)
    ref[0, 5] = 0.0
    mag = np.where(np.isnan(ref), 0.0, np.abs(np.nan_to_num(ref)) + 1.0)
    got = np.nan_to_num(ref).astype(np.float32)
    return width, lens, ref, mag, got


def _mask(got, lens, width):
    bits = (np.arange(width)[None, :] < lens[:, None]) & (got.view(np.uint32) != 0)
    return O.pack_mask(bits)


def test_check_mask_accepts_consistent_and_near_zero():
    width, lens, ref, mag, got = _case()
    assert check_mask(_mask(got, lens, width), got, ref, mag, lens) == 0
    ref2 = ref.copy()
    ref2[1, 3] = 5e-4 * mag[1, 3]  # exact logit within RTOL * A_t of zero; the kernel gives 0.0
    got2 = got.copy()
    got2[1, 3] = 0.0
    assert check_mask(_mask(got2, lens, width), got2, ref2, mag, lens) == 1


def test_check_mask_rejects_mismatches():
    width, lens, ref, mag, got = _case()
    bad = _mask(got, lens, width)
    bad[0, 0] ^= 1  # a bit that does not follow the kernel's own logit
    with pytest.raises(AssertionError):
        check_mask(bad, got, ref, mag, lens)
    got3 = got.copy()
    got3[1, 4] = 0.0  # a zero where the exact logit is far from zero
    with pytest.raises(AssertionError):
        check_mask(_mask(got3, lens, width), got3, ref, mag, lens)
