"""GPU parity of the top-2048 at the reference's production shapes (hcu_ops/tests/test_rows.py:9-30):
relu_sum scores of 6 / 12 / 24 / 36 / 48 / 192 ragged rows (MTP verify batches) of 16K / 64K / 128K
tokens in a score block 1M wide (the page-table capacity), and 1,536 ragged rows of 16K tokens.
Every path -- one CTA per row, 2 / 8 / 16 splits, and the split top-k on a paired logits
workspace (counters only, sampled threshold) -- is compared with the oracle's C radix select,
set and order.

Only the first L columns of a row are drawn (on the CPU, seeded); the GPU block is 1M wide with
NaN garbage past L and clear mask bits there, as unwritten production storage would be.  The
page table holds arange + 7 + 10^6 * row over the L columns a row can select."""
import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C
from oracle.topk_c import topk_radix

pytestmark = pytest.mark.gpu

W_PROD = 1 << 20
BATCHES = (6, 12, 24, 36, 48, 192)
LENGTHS = (16384, 65536, 131072)


def relu_sum_rows(B, L, seed):
    """(scores f32 [B, L] with NaN at zero scores, mask i16 [B, L/16], lengths i32 [B], pt i32 [B, L]):
    the reference's relu_sum distribution, sum of 8 ReLU'd normals with one weight vector
    (hcu_ops/tests/topk_lib.py:16-18), ragged rows L - 37 i - 3."""
    g = torch.Generator().manual_seed(seed)
    c = torch.rand(8, generator=g) - 0.3
    x = torch.empty(B, L)
    for r in range(B):  # row by row: the [B, L, 8] normals never exist at once
        x[r] = (torch.relu(torch.randn(L, 8, generator=g)) * c).sum(-1)
    nz = x != 0
    w16 = torch.tensor([1 << i for i in range(16)], dtype=torch.int32)
    bits = (nz.view(B, -1, 16).to(torch.int32) * w16).sum(-1, dtype=torch.int32)
    mask = torch.where(bits > 32767, bits - 65536, bits).to(torch.int16).contiguous()
    x = torch.where(nz, x, torch.full_like(x, float("nan"))).contiguous()
    lengths = (L - torch.arange(B) * 37 - 3).clamp(min=1).to(torch.int32)
    pt = (torch.arange(L, dtype=torch.int32).unsqueeze(0) + 7
          + 1000000 * torch.arange(B, dtype=torch.int32).unsqueeze(1)).contiguous()
    return x, mask, lengths, pt


def on_gpu_padded(x, mask, W, dev):
    """[B, W] scores and [B, W/16] mask on the GPU: the first L columns from x / mask, NaN scores and
    clear mask bits past them."""
    B, L = x.shape
    xg = torch.full((B, W), float("nan"), device=dev)
    xg[:, :L] = x.to(dev)
    mg = torch.zeros(B, W // 16, dtype=torch.int16, device=dev)
    mg[:, :L // 16] = mask.to(dev)
    return xg, mg


def paired_split(x, m, l, p, c):
    """The split top-k on a logits call's workspace with only its counters zeroed (the paired decode
    mode without the fused histogram)."""
    zws = torch.zeros(x.shape[0] * (2 * 4096 + 2), dtype=torch.int32, device=x.device)
    return _C.sparse_mask_topk_transform_split_pre(x, m, l, p, c, 2048, 8, zws, False)


IMPLS = {
    "single": lambda x, m, l, p, c: _C.sparse_mask_topk_transform(x, m, l, p, c, 2048),
    "s2": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 2),
    "s8": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 8),
    "s16": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 16),
    "split_pre": paired_split,
    "default": lambda x, m, l, p, c: hcu_ops.sparse_mask_topk_transform(x, m, l, p, c, 2048),
}


@pytest.mark.parametrize("L", LENGTHS)
def test_topk_production_rows(gpu, L):
    for B in BATCHES:
        x, mask, lengths, pt = relu_sum_rows(B, L, seed=B * 7 + L)
        ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), L)
        xg, mg = on_gpu_padded(x, mask, W_PROD, gpu)
        lg, pg = lengths.to(gpu), pt.to(gpu)
        cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
        for name, fn in IMPLS.items():
            got = fn(xg, mg, lg, pg, cu).cpu().numpy()
            assert np.array_equal(got, ref), f"relu_sum rows={B} L={L} W=1M impl={name}"
        del xg, mg
        torch.cuda.empty_cache()


def test_topk_production_1536_rows(gpu):
    """The reference's eager large batch: 1,536 ragged rows of 16K tokens in a 16,448-wide block
    (one CTA per row: the split needs at most 512 rows)."""
    B, L, W = 1536, 16384, 16448
    x, mask, lengths, pt = relu_sum_rows(B, L, seed=1536)
    ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), L)
    xg, mg = on_gpu_padded(x, mask, W, gpu)
    lg, pg = lengths.to(gpu), pt.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    assert _C.topk_splits(B, W, 8) == 1
    for name in ("single", "s8", "default"):
        got = IMPLS[name](xg, mg, lg, pg, cu).cpu().numpy()
        assert np.array_equal(got, ref), f"relu_sum rows=1536 impl={name}"
