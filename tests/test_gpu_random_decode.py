"""Seeded random decode batches through the whole step -- q quantisation, paged logits with the
top-k pass-1 pairing (hist_lens), top-2048 + page-table transform -- against the oracle: q8 and the
nonzero mask bit-exact, logits within the documented tolerance, and every top-k row (set and
order) identical to the oracle's selection on the GPU logits.  Each case draws its group size,
rows per CTA, head count, request count, lengths (short rows, rows within two tokens of 2048,
longer rows) and block-table capacity from its seed, so the sweep reaches combinations the
hand-picked cases do not (reference shapes: hcu_ops/tests/test_mqa_hist.py:25-61)."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle.topk_c import topk_radix

from gpu_util import check_logits, check_mask, oracle_decode, oracle_q

pytestmark = pytest.mark.gpu


def _draw(seed):
    rng = np.random.default_rng(seed)
    group = int(rng.choice([1, 2, 3, 4, 6, 8]))
    rpc = int(rng.choice([r for r in (1, 2, 3, 4, 8) if group % r == 0]))
    heads = int(rng.choice([32, 64]))
    lens = []
    for kind in rng.integers(0, 4, int(rng.integers(1, 13))):
        if kind == 0:
            lens.append(int(rng.integers(1, 2049)))
        elif kind == 1:
            lens.append(2048 + int(rng.integers(-2, 3)))
        else:
            lens.append(int(rng.integers(2049, 6001)))
    return group, rpc, heads, lens, int(rng.integers(0, 4))


@pytest.mark.parametrize("seed", range(12))
def test_random_decode_step(gpu, seed):
    group, rpc, heads, lens, slack = _draw(1000 + seed)
    what = f"seed {seed}: group {group} rpc {rpc} heads {heads} lens {lens}"
    case = wl.decode_case(2000 + seed, lens, group=group, heads=heads,
                          bt_pages=max((L + group + 63) // 64 for L in lens) + slack)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens_g = case.context_lens.to(gpu)
    lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), case.kv.to(gpu), w, lens_g, case.block_table.to(gpu), case.width,
                                  case.group, hist_lens=lens_g, rows_per_cta=rpc)
    pt = case.page_table_1()
    out = hcu_ops.sparse_mask_topk_transform(lg, mask, lens_g, pt.to(gpu),
                                             torch.arange(case.rows + 1, dtype=torch.int32, device=gpu))
    rq8, rw = oracle_q(case)
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rq8), f"{what}: q8"
    ref, mag, dmag, ref_mask = oracle_decode(case, rq8, rw)
    got_mask = mask.cpu().numpy()
    got = lg.cpu().numpy()
    check_mask(got_mask, got, ref, mag, case.context_lens.numpy(), f"{what}: mask")
    for r in range(case.rows):
        L = int(case.context_lens[r])
        check_logits(got[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"{what} row {r}")
    want = topk_radix(got.astype(np.float32), got_mask, case.context_lens.numpy(), pt.numpy(), case.width)
    assert np.array_equal(out.cpu().numpy(), want), f"{what}: top-k rows"
