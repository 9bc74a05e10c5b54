"""Seeded random top-k cases against the C radix oracle, row for row and order included: random
row counts (1-300), widths (2,000-200,000 tokens, on both sides of the 81,920-token list switch),
the ten score distributions, masks or dense scores, ragged lengths, split counts 1-16, the
block-table form, and rows whose sampled threshold sits low in the row (4,600-9,000 keys pass
it, past the candidate lists: the second collection pass).  Longer runs of the same generator
(over 16,000 cases) matched the oracle everywhere."""
import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C
import workloads as wl
from oracle.topk_c import topk_radix

pytestmark = pytest.mark.gpu

N_CASES = 120


def _case(seed):
    rng = np.random.default_rng(seed)
    B = int(rng.choice([1, 2, 5, 16, 64, 128, 300]))
    W = int(rng.choice([2000, 4096, 9000, 16384, 40000, 65536, 81920, 98304, 131072, 200000]))
    B = max(1, min(B, 40_000_000 // W))
    dist = str(rng.choice(wl.TOPK_DISTS))
    ragged = bool(rng.integers(2))
    x, mask, lengths, pt = wl.topk_scores(B, W - 7 if ragged else W, dist, W=W, ragged=ragged, seed=seed)
    low = bool(rng.integers(4) == 0) and W > 4096 and dist in ("pos", "mixed", "relu_sum", "narrow")
    if low:
        target = int(rng.choice([4600, 6000, 9000]))
        t = 1.0 - target / W
        xs = torch.rand(B, W, generator=torch.Generator().manual_seed(seed)) * 0.999 + 0.001
        c = np.arange(256)
        for r in range(B):
            L = int(lengths[r])
            if L <= 4096:
                continue
            st = np.minimum((((2 * c + 1) * L) // 512) & ~15, (L - 16) & ~15)  # the sampled chunks
            idx = torch.from_numpy((st[:, None] + np.arange(16)[None, :]).reshape(-1))
            xs[r, idx] = t + torch.rand(idx.numel(), generator=torch.Generator().manual_seed(seed + r)) * 1e-3
        x = torch.where(torch.isnan(x), x, xs)
    use_mask = bool(rng.integers(3) > 0)
    blocks = bool(rng.integers(4) == 0)
    bt = None
    if blocks:
        pages = (W + 63) // 64
        bt = torch.from_numpy(rng.permutation(B * pages + 3)[:B * pages].reshape(B, pages).astype(np.int32))
        tok = torch.arange(pages * 64, dtype=torch.int64)
        pt = (bt.long()[:, tok // 64] * 64 + tok % 64).to(torch.int32)
    splits = int(rng.choice([1, 2, 4, 8, 16]))
    return B, W, dist, x, (mask if use_mask else None), lengths, pt, bt, splits, low


@pytest.mark.parametrize("chunk", range(4))
def test_topk_random_cases(gpu, chunk):
    for seed in range(5000 + chunk * (N_CASES // 4), 5000 + (chunk + 1) * (N_CASES // 4)):
        B, W, dist, x, m, lengths, pt, bt, splits, low = _case(seed)
        ref = np.asarray(topk_radix(x.numpy(), None if m is None else m.numpy(), lengths.numpy(), pt.numpy(), W))
        xg, lg, pg = x.to(gpu), lengths.to(gpu), pt.to(gpu)
        mg = None if m is None else m.to(gpu)
        cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
        if bt is not None:
            got = _C.sparse_mask_topk_transform_blocks(xg, mg, lg, bt.to(gpu), cu, 2048, splits, None, False)
        elif mg is None:
            got = hcu_ops.topk_transform(xg, lg, pg, cu, max_splits=splits)
        elif splits == 1:
            got = _C.sparse_mask_topk_transform(xg, mg, lg, pg, cu, 2048)
        else:
            got = _C.sparse_mask_topk_transform_split(xg, mg, lg, pg, cu, 2048, splits)
        assert np.array_equal(got.cpu().numpy(), ref), (
            f"seed {seed}: B={B} W={W} {dist} mask={m is not None} blocks={bt is not None} splits={splits} low={low}")
