"""GPU parity of the block-table form of the top-k transform (dsa_topk_transform_blocks,
hcu_ops.sparse_mask_topk_transform_blocks): token t of a row maps to
block_table[row][t // 64] * 64 + t % 64, the entry page_table_size_1 holds when it expands the
64-token-page block table (reference sparse_mask_topk.cu:348,751,804-807 gather that expansion).
Every path is compared, set and order, with the C radix oracle run on the expanded table: one
CTA per row (short rows, the sampled row kernel, the wide-list instantiation), the sampled split,
the split paired with a logits workspace, the varlen layout, and a block table covering fewer
tokens than the scores (tokens past it map to -1)."""
import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C
import workloads as wl
from oracle.topk_c import topk_radix

pytestmark = pytest.mark.gpu


def random_blocks(n_rows, pages, seed):
    """int32 [n_rows, pages]: distinct shuffled physical pages (one pool for all rows)."""
    g = torch.Generator().manual_seed(seed)
    return torch.randperm(n_rows * pages + 17, generator=g)[:n_rows * pages].view(n_rows, pages).to(torch.int32)


def expand(bt):
    """page_table_size_1 of a block table: [rows, pages * 64], entry page * 64 + t % 64."""
    t = torch.arange(bt.shape[1] * 64, dtype=torch.int64)
    return (bt.long()[:, t // 64] * 64 + t % 64).to(torch.int32)


def run_blocks(x, mask, lengths, bt, cu, splits, zws=None, gpu=None):
    return _C.sparse_mask_topk_transform_blocks(x.to(gpu), None if mask is None else mask.to(gpu), lengths.to(gpu),
                                                bt.to(gpu), cu.to(gpu), 2048, splits, zws, False).cpu().numpy()


@pytest.mark.parametrize("B,W,dist", [(6, 65536, "relu_sum"), (6, 65536, "narrow"), (24, 16384, "sparse2"),
                                      (600, 5056, "mixed"), (520, 98304, "pos")])
def test_blocks_equal_expanded_table(gpu, B, W, dist):
    """Ragged rows: one CTA per row and the sampled split (decode layout); 520 rows of 96K take
    the one-CTA-per-row kernel with the 5120-entry list; rows of 600 x ~5K include rows of at most
    2048 tokens (copied)."""
    x, mask, lengths, _ = wl.topk_scores(B, W - 9, dist, W=W, ragged=True, seed=B + W)
    if B == 600:
        lengths[::7] = torch.randint(1, 2049, (len(lengths[::7]),), generator=torch.Generator().manual_seed(3),
                                     dtype=torch.int32)
    bt = random_blocks(B, W // 64, seed=B)
    ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), expand(bt).numpy(), W)
    cu = torch.arange(B + 1, dtype=torch.int32)
    for splits in (1, 2, 8):
        got = run_blocks(x, mask, lengths, bt, cu, splits, gpu=gpu)
        assert np.array_equal(got, ref), f"{dist} B={B} W={W} splits={splits}"


def test_blocks_paired_and_python_surface(gpu):
    """The split top-k on a logits call's workspace (counters zeroed, sampled threshold), through
    the C binding and through hcu_ops after mqa_logits(..., hist_lens): the real decode pairing."""
    case = wl.decode_case(21, [40000, 9000, 65000, 2100, 30000, 1500, 64000, 12000], group=2, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens = case.context_lens.to(gpu)
    bt = case.block_table.to(gpu)
    cu = torch.arange(case.rows + 1, dtype=torch.int32, device=gpu)
    lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), case.kv.to(gpu), w, lens, bt, case.width, 2, hist_lens=lens)
    got = hcu_ops.sparse_mask_topk_transform_blocks(lg, mask, lens, bt, cu).cpu().numpy()
    assert hcu_ops._MQA_HIST is None
    ref = topk_radix(lg.cpu().numpy(), mask.cpu().numpy(), case.context_lens.numpy(), case.page_table_1().numpy(),
                     case.width)
    assert np.array_equal(got, ref)
    zws = torch.zeros(case.rows * (2 * 4096 + 2), dtype=torch.int32, device=gpu)
    got2 = _C.sparse_mask_topk_transform_blocks(lg, mask, lens, bt, cu, 2048, 8, zws, False).cpu().numpy()
    assert np.array_equal(got2, ref)
    # the reference form on the expanded table gives the same rows
    got3 = hcu_ops.sparse_mask_topk_transform(lg, mask, lens, case.page_table_1().to(gpu), cu).cpu().numpy()
    assert np.array_equal(got3, ref)


def test_blocks_varlen_and_narrow_table(gpu):
    """Varlen layout (rows map to their request's block-table row through cu_seqlens_q), dense
    scores, and a block table of fewer pages than the scores are wide: tokens past its last page
    map to -1, as they do past the columns of page_table_size_1."""
    W = 9024
    x, _, _, _ = wl.topk_scores(7, W, "mixed", seed=5)
    x[[0, 4], 7600:9000] = torch.nan_to_num(x[[0, 4], 7600:9000]).abs() + 1000.0  # selected past the table's end
    lengths = torch.tensor([9000, 3000, 2048, 2049, 8999, 100, 6000], dtype=torch.int32)
    cu = torch.tensor([0, 3, 4, 7], dtype=torch.int32)
    bt = random_blocks(3, 120, seed=9)  # 7680 tokens < 9024
    ref = topk_radix(x.numpy(), None, lengths.numpy(), expand(bt).numpy(), W, cu_seqlens_q=cu.numpy())
    assert (ref[[0, 4]] == -1).any(), "rows past the table's last page must select tokens without a slot"
    for splits in (1, 4):
        got = run_blocks(x, None, lengths, bt, cu, splits, gpu=gpu)
        assert np.array_equal(got, ref), f"splits={splits}"
