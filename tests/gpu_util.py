"""Shared helpers of the GPU parity tests (imported by tests only)."""
import numpy as np
import torch

from oracle import indexer as O
from oracle.fp8 import fp8_decode

# Logits tolerance: |gpu - oracle| <= RTOL * A_t, where A_t = s_t * sum_h |w_h| relu(acc_h) is the
# magnitude of the weighted ReLU sum (A_t = |logit| when the head weights share a sign, A_t >=
# |logit| otherwise); in addition at least STRICT_FRAC of the tokens must meet the plain
# relative bound |gpu - oracle| <= RTOL * |oracle|.
RTOL = 1e-3
STRICT_FRAC = 0.999


def kv_np(kv):
    return kv.view(kv.shape[0], -1).cpu().numpy()


def q_bits(q_bf16):
    return q_bf16.view(torch.int16).cpu().numpy().view(np.uint16)


def check_logits(got, ref, mag, what=""):
    got = np.asarray(got, dtype=np.float64)
    err = np.abs(got - ref)
    bad = err > RTOL * mag + 1e-30
    assert not bad.any(), f"{what}: {int(bad.sum())} logits outside {RTOL} * magnitude; worst " \
                          f"{float((err / np.maximum(mag, 1e-30)).max()):.3e}"
    strict = (err <= RTOL * np.abs(ref)).mean() if ref.size else 1.0
    assert strict >= STRICT_FRAC, f"{what}: only {strict:.5f} of logits within {RTOL} relative"


def sorted_rows(a):
    return np.sort(np.asarray(a), axis=1)


def oracle_decode(case, q8, w):
    return O.mqa_logits_decode(q8, w, kv_np(case.kv), case.context_lens.numpy(), case.block_table.numpy(),
                               case.group, case.width)


def oracle_q(case):
    return O.quant_q(q_bits(case.q), case.w.numpy())


__all__ = ["RTOL", "STRICT_FRAC", "kv_np", "q_bits", "check_logits", "sorted_rows", "oracle_decode", "oracle_q",
           "fp8_decode"]
