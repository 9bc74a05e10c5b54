"""The consumer wire format of the top-k output (tests/wire_format.py), pinned on the CPU: the
oracle's rows keep it, and each plausible mistake planted into them (a pad inside the row, token
ids where slot ids belong, a slot of the wrong page offset, a duplicate, a scrambled order, a
short row out of order, a wider integer type) is reported.  The sparse-MLA consumer is pinned by
the identity that attention over the listed slots equals dense attention over every token with
the unlisted ones masked out, whatever the list order."""
import numpy as np

import workloads as wl
from oracle.topk_c import topk_radix
from wire_format import TOPK, slot_table, sparse_mla_decode, wire_format_problems


def _case(seed=3):
    lens = np.array([0, 5, 2048, 2049, 9000, 30000], dtype=np.int32)
    B = lens.size
    L = int(lens.max())
    W = L + 64
    x, mask, _, _ = wl.topk_scores(B, L, "mixed", W=W, seed=seed)
    rng = np.random.default_rng(seed)
    n_pages = (W + 63) // 64
    bts = [rng.permutation(B * n_pages)[:n_pages] for _ in range(B)]  # distinct pages per row
    pt = np.stack([slot_table(bt, W) for bt in bts]).astype(np.int32)
    out = topk_radix(x.numpy(), mask.numpy(), lens, pt, W)
    return out, lens, pt


def test_oracle_rows_keep_the_wire_format():
    out, lens, pt = _case()
    assert wire_format_problems(out, lens, lambda r: pt[r]) == []
    assert (out[0] == -1).all() and (out[1, 5:] == -1).all() and (out[1, :5] == pt[1, :5]).all()


def test_planted_mistakes_are_reported():
    out, lens, pt = _case()
    slots = lambda r: pt[r]

    def problems(mut):
        bad = out.copy()
        mut(bad)
        return wire_format_problems(bad, lens, slots)

    def pad_inside(a):
        a[4, 100] = -1

    def token_ids(a):
        a[5] = np.sort(np.argsort(-np.arange(30000))[:TOPK]).astype(np.int32)

    def wrong_offset(a):
        a[3, 17] = a[3, 17] + 64 * 10**6

    def duplicate(a):
        a[4, 11] = a[4, 10]

    def scrambled(a):
        a[5, :] = a[5, ::-1]

    def short_out_of_order(a):
        a[1, :5] = a[1, [1, 0, 2, 3, 4]]

    def pad_first(a):
        a[1, :6] = np.concatenate([[-1], a[1, :5]])

    for mut in (pad_inside, token_ids, wrong_offset, duplicate, scrambled, short_out_of_order, pad_first):
        assert problems(mut), mut.__name__
    assert wire_format_problems(out.astype(np.int64), lens, slots)
    assert wire_format_problems(out[:, :TOPK - 1], lens, slots)


def test_sparse_consumer_equals_masked_dense_attention():
    rng = np.random.default_rng(1)
    n_tok, H = 5000, 16
    k = rng.standard_normal((n_tok, 576))
    q = rng.standard_normal((H, 576))
    sel = np.sort(rng.choice(n_tok, TOPK, replace=False))
    scale = 576 ** -0.5
    o, lse = sparse_mla_decode(q, k[sel], scale)
    s = (q @ k.T) * scale
    s[:, np.setdiff1d(np.arange(n_tok), sel)] = -np.inf
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    want_o = (p / p.sum(axis=1, keepdims=True)) @ k[:, :512]
    want_lse = np.log(p.sum(axis=1)) + m[:, 0]
    assert np.allclose(o, want_o, rtol=1e-12, atol=1e-12) and np.allclose(lse, want_lse, rtol=1e-12)
    perm = rng.permutation(TOPK)
    o2, _ = sparse_mla_decode(q, k[sel[perm]], scale)
    assert np.allclose(o2, o, rtol=1e-12, atol=1e-12)
    # a consumer that let a pad index the last slot (-1 in Python) would differ
    o3, _ = sparse_mla_decode(q, k[np.append(sel, -1)], scale)
    assert not np.allclose(o3, o, rtol=1e-6, atol=0)
