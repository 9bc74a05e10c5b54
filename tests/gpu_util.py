"""Shared helpers of the GPU parity tests (imported by tests only)."""
import numpy as np
import torch

from oracle import indexer as O
from oracle.fp8 import fp8_decode

# Logits tolerance (fp8 MFMA + fp32 epilogue vs the exact fp64 oracle):
#  (a) every token: |gpu - oracle| <= RTOL * A_t, where A_t = s_t * sum_h |w_h| relu(acc_h) is the
#      magnitude of the weighted ReLU sum (A_t = |logit| when the head weights share a sign);
#  (b) tokens whose logit is cancelled by at most CANCEL, across heads (|logit| >= A_t / CANCEL)
#      and inside the dot products (|logit| >= M_t / CANCEL, M_t = s_t sum_h |w_h| sum_d
#      |q8_hd k8_td|): the plain relative bound |gpu - oracle| <= RTOL * |oracle|.
# One v_mfma_f32_16x16x128_f8f6f4 is not an fp32 sum of its 128 exact products: measured on
# gfx950 its result is off by up to 1.5e-5 (normal keys) and 5.0e-5 (Student-t(4) keys) of the
# summed |products| (a sequential fp32 sum: 5e-8), so a logit whose dot products cancel carries
# that error relative to M_t, not to |logit|; (b) leaves such tokens to (a), as it leaves the
# ones whose heads cancel.
RTOL = 1e-3
CANCEL = 20.0


def kv_np(kv):
    return kv.view(kv.shape[0], -1).cpu().numpy()


def q_bits(q_bf16):
    return q_bf16.view(torch.int16).cpu().numpy().view(np.uint16)


def check_logits(got, ref, mag, dmag, what=""):
    """Asserts the tolerance above (mag = A_t, dmag = M_t); returns (max err / A_t, max relative
    err over (b))."""
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - ref)
    bad = err > RTOL * mag + 1e-30
    worst_mag = float((err / np.maximum(mag, 1e-30)).max()) if err.size else 0.0
    assert not bad.any(), f"{what}: {int(bad.sum())} logits outside {RTOL} * magnitude; worst {worst_mag:.3e}"
    plain = (np.abs(ref) >= np.maximum(mag, dmag) / CANCEL) & (mag > 0)  # exact zeros are covered by (a)
    rel = err[plain] / np.abs(ref[plain]) if plain.any() else np.zeros(1)
    worst_rel = float(rel.max())
    assert worst_rel <= RTOL, f"{what}: relative error {worst_rel:.3e} > {RTOL} on an uncancelled logit"
    return worst_mag, worst_rel


def check_mask(got_mask, got_logits, ref_logits, mag, lens, what=""):
    """The nonzero mask (mqa_hist.cu:209-218: bit = t < len && the logit's bits != 0) against the
    kernel's own logits, exactly; and against the oracle's mask everywhere except at tokens whose
    exact logit lies within the logits tolerance of zero (RTOL * A_t), where the fp32 epilogue
    of cancelling heads may land on 0.0 exactly (measured once: a token at -3.7e-4 with A_t =
    71 came out as 0.0) -- the logit there is still checked against the oracle by check_logits.
    Returns the number of such tokens."""
    got_mask = np.asarray(got_mask)
    width = got_mask.shape[1] * 16
    bits = O.unpack_mask(got_mask, width)
    t = np.arange(width)[None, :]
    inside = t < np.asarray(lens, dtype=np.int64)[:, None]
    nonzero_bits = np.ascontiguousarray(np.asarray(got_logits, dtype=np.float32)[:, :width]).view(np.uint32) != 0
    own = inside & nonzero_bits
    assert np.array_equal(bits, own), f"{what}: mask bits differ from the kernel's own nonzero logits"
    ref_bits = inside & ~np.isnan(ref_logits) & (np.nan_to_num(ref_logits) != 0.0)
    differ = bits != ref_bits
    near_zero = np.abs(np.nan_to_num(ref_logits)) <= RTOL * np.asarray(mag)
    assert not (differ & ~near_zero).any(), f"{what}: mask differs from the oracle's at a logit away from zero"
    return int(differ.sum())


def sorted_rows(a):
    return np.sort(np.asarray(a), axis=1)


def oracle_decode(case, q8, w):
    return O.mqa_logits_decode(q8, w, kv_np(case.kv), case.context_lens.numpy(), case.block_table.numpy(),
                               case.group, case.width)


def oracle_q(case):
    return O.quant_q(q_bits(case.q), case.w.numpy())


__all__ = ["RTOL", "CANCEL", "kv_np", "q_bits", "check_logits", "check_mask", "sorted_rows", "oracle_decode", "oracle_q",
           "fp8_decode"]
