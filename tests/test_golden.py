"""The oracle against the known-answer fixtures of tests/golden/ (written by
tests/golden/make_golden.py from torch's fp8 / bf16 casts, exact float64 dot products and a
brute-force top-k on the reference's key order, none of it from oracle/): the C radix top-k row
for row, order included; the numpy top-k as a set; q quantisation, the K-cache writer, both
dequants and the mask bit-exact; the logits to float64 rounding."""
import os

import numpy as np

from oracle import indexer as O
from oracle.topk_c import topk_radix

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_golden_topk_oracles():
    d = _load("topk_small.npz")
    W = int(d["width"])
    got = np.asarray(topk_radix(d["score"], d["mask"], d["lengths"], d["page_table"], W))
    assert np.array_equal(got, d["expected"])
    sets = O.topk_transform(d["score"], d["mask"], d["lengths"], d["page_table"], W)
    assert np.array_equal(np.sort(sets, axis=1), np.sort(d["expected"], axis=1))


def test_golden_quant_dequant_logits_oracles():
    d = _load("indexer_small.npz")
    q8, w_eff = O.quant_q(d["q_bf16"], d["w"])
    assert np.array_equal(q8, d["q8"])
    assert np.array_equal(w_eff.view(np.uint32), d["w_eff"].view(np.uint32))
    assert np.array_equal(O.dequant_k_paged(d["kv_cache"], d["slots"]), d["dequant_bf16"])
    logits, mag, _, mask = O.mqa_logits_decode(d["q8"], d["w_eff"], d["kv_cache"], d["context_lens"],
                                               d["block_table"], int(d["group"]), int(d["width"]))
    written = ~np.isnan(d["logits"])
    assert np.array_equal(written, ~np.isnan(logits))
    np.testing.assert_allclose(logits[written], d["logits"][written], rtol=1e-12, atol=0)
    np.testing.assert_allclose(mag[written], d["magnitude"][written], rtol=1e-12, atol=0)
    assert np.array_equal(mask, d["mask"])


def test_golden_k_writer_and_mla_oracles():
    d = _load("indexer_small.npz")
    keep = d["k_slots"] >= 0
    kf = (d["k_bf16"].astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(O.build_kv_cache(kf[keep], d["k_slots"][keep], 2), d["k_cache_written"])
    m = _load("mla_small.npz")
    assert np.array_equal(O.dequant_mla(m["cache"], m["slots"]), m["expected"])


def test_golden_topk_rows_catch_plausible_mistakes():
    """Planted mistakes in a restatement of the selection (on the CPU) each change some fixture row:
    no +0 fast-path order, ties taken from the top token down, masked tokens keeping their score,
    the -0.0 / +0 order swapped."""
    d = _load("topk_small.npz")
    x, mask, lengths, pt = d["score"], d["mask"], d["lengths"], d["page_table"]
    bits = O.unpack_mask(mask, x.shape[1])

    def rows(fast_path=True, ties_desc=False, use_mask=True, neg_zero_high=False):
        out = []
        for r in range(x.shape[0]):
            L = int(lengths[r])
            if L <= 2048:
                out.append(np.array([pt[r, i] if i < L else -1 for i in range(2048)], dtype=np.int32))
                continue
            b = x[r, :L].view(np.uint32).astype(np.int64)
            k = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
            if neg_zero_high:
                k = np.where(b == 0x80000000, 0x80000001, k)
            if use_mask:
                k = np.where(bits[r, :L], k, 0x80000000)
            order = sorted(range(L), key=lambda t: (-int(k[t]), t))
            chosen = order[:2048]
            if fast_path and int((k > 0x80000000).sum()) == 2048:
                sel = sorted(chosen)
            else:
                thr = k[order[2047]]
                ties = [t for t in range(L) if k[t] == thr]
                ties = sorted(ties, reverse=ties_desc)[:2048 - sum(1 for t in chosen if k[t] > thr)]
                sel = sorted(t for t in chosen if k[t] > thr) + sorted(ties)
            out.append(pt[r, sel].astype(np.int32))
        return np.stack(out)

    assert np.array_equal(rows(), d["expected"])  # the restatement itself agrees
    for planted in ({"fast_path": False}, {"ties_desc": True}, {"use_mask": False}, {"neg_zero_high": True}):
        assert not np.array_equal(rows(**planted), d["expected"]), planted


def test_golden_logits_catch_plausible_mistakes():
    """Planted mistakes in a restatement of the logits (on the CPU) each move some fixture logit
    by more than the GPU tolerance (1e-3 of its magnitude): ReLU after the head weight, no key
    scale, the other row's head weights, the key of the next token."""
    from oracle.fp8 import fp8_decode
    d = _load("indexer_small.npz")
    q = fp8_decode(d["q8"]).astype(np.float64)
    kv = d["kv_cache"]
    slots = d["slots"].astype(np.int64)
    codes = kv[slots // 64][np.arange(len(slots))[:, None], (slots % 64)[:, None] * 128 + np.arange(128)]
    scale = np.ascontiguousarray(kv[slots // 64][np.arange(len(slots))[:, None],
                                                  8192 + (slots % 64)[:, None] * 4 + np.arange(4)]).view(np.float32)[:, 0]
    k = fp8_decode(codes).astype(np.float64)
    w = d["w_eff"].astype(np.float64)
    exact, mag = d["logits"], d["magnitude"]

    def logits(relu_after_w=False, no_scale=False, swap_w=False, shift_key=False):
        out = np.full_like(exact, np.nan)
        kk = np.roll(k, -1, axis=0) if shift_key else k
        for r in range(2):
            L = int(d["context_lens"][r])
            acc = q[r] @ kk[:L].T
            wr = w[1 - r] if swap_w else w[r]
            v = (np.maximum(wr[:, None] * acc, 0.0)).sum(0) if relu_after_w else wr @ np.maximum(acc, 0.0)
            out[r, :L] = v * (1.0 if no_scale else scale[:L])
        return out

    written = ~np.isnan(exact)
    assert (np.abs(logits()[written] - exact[written]) <= 1e-9 * mag[written] + 1e-300).all()
    for planted in ({"relu_after_w": True}, {"no_scale": True}, {"swap_w": True}, {"shift_key": True}):
        err = np.abs(logits(**planted)[written] - exact[written])
        assert (err > 1e-3 * mag[written]).any(), planted
