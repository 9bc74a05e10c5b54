"""Seeded random prefill requests through quant_q_fp8 -> prefill_indexer (the slab loop under a
memory budget and a slab row limit) against the oracle: q8 bit-exact, every row's logits within
the documented tolerance, and every top-k row (set and order) identical to the oracle's selection
on the GPU logits.  Each case draws its row count, cached prefix (none, short, or past 2048
tokens: rows on both sides of 2048 keys), head count, K distribution, slab limits and page-table
map (the block table's slots, or an arbitrary token -> value map) from its seed."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix

from gpu_util import check_logits, kv_np, q_bits

pytestmark = pytest.mark.gpu


def _draw(seed):
    rng = np.random.default_rng(seed)
    rows = int(rng.integers(1, 65))
    prefix = [0, int(rng.integers(1, 2048)), int(rng.integers(2048, 4001))][int(rng.integers(0, 3))]
    heads = int(rng.choice([32, 64]))
    dist = ["normal", "student_t4"][int(rng.integers(0, 2))]
    slab = int(rng.integers(1, rows + 1))
    budget_rows = int(rng.integers(1, rows + 1))
    remap = bool(rng.integers(0, 2))
    return rows, prefix, heads, dist, slab, budget_rows, remap


@pytest.mark.parametrize("seed", range(8))
def test_random_prefill_indexer(gpu, seed):
    rows, prefix, heads, dist, slab, budget_rows, remap = _draw(3000 + seed)
    what = (f"seed {seed}: {rows} rows, prefix {prefix}, heads {heads}, {dist}, slab {slab}, "
            f"budget {budget_rows} rows, remap {remap}")
    case = wl.prefill_case(4000 + seed, rows, prefix, heads=heads, dist=dist)
    width = case.n_keys
    g = lambda t: t.to(gpu)
    kv, bt, lens = g(case.kv), g(case.block_table), g(case.lens)
    q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
    if remap:
        gen = torch.Generator().manual_seed(5000 + seed)
        pt = torch.randperm(3 * width, generator=gen)[:width].to(torch.int32)
    else:
        pt = case.slots()
    out = hcu_ops.prefill_indexer(q8, w, kv, bt, lens, width, g(pt) if remap else None,
                                  memory_budget_bytes=budget_rows * width * 4, max_slab_rows=slab)
    lg = hcu_ops.mqa_logits_prefill(q8, w, kv, bt, lens, width).cpu().numpy()

    rq8, rw = O.quant_q(q_bits(case.q), case.w.numpy())
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rq8), f"{what}: q8"
    ref, mag, dmag = O.mqa_logits_prefill(rq8, rw, kv_np(case.kv), case.block_table.numpy(), case.lens.numpy(), width)
    for r in range(rows):
        L = int(case.lens[r])
        check_logits(lg[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"{what} row {r}")
    want = topk_radix(lg.astype(np.float32), None, case.lens.numpy(), pt.numpy()[None, :], width,
                      cu_seqlens_q=np.array([0, rows], dtype=np.int32))
    assert np.array_equal(out.cpu().numpy(), want), f"{what}: top-k rows"


@pytest.mark.parametrize("rows,prefix,slab", [(600, 1500, 600), (700, 5000, 560), (1100, 20000, 1024)])
def test_prefill_indexer_medium_slabs(gpu, rows, prefix, slab):
    """Slabs of hundreds of rows (one top-k CTA a row) and a smaller tail slab through
    prefill_indexer, the rows' keys on both sides of 2048 and 4096, against the oracle's selection
    on the same logits."""
    case = wl.prefill_case(7000 + rows, rows, prefix, heads=64)
    width = case.n_keys
    g = lambda t: t.to(gpu)
    kv, bt, lens = g(case.kv), g(case.block_table), g(case.lens)
    q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
    pt = case.slots()
    out = hcu_ops.prefill_indexer(q8, w, kv, bt, lens, width, g(pt), memory_budget_bytes=slab * width * 4,
                                  max_slab_rows=slab)
    lg = hcu_ops.mqa_logits_prefill(q8, w, kv, bt, lens, width).cpu().numpy()
    want = topk_radix(lg.astype(np.float32), None, case.lens.numpy(), pt.numpy()[None, :], width,
                      cu_seqlens_q=np.array([0, rows], dtype=np.int32))
    got = out.cpu().numpy()
    bad = [r for r in range(rows) if not np.array_equal(got[r], want[r])]
    assert not bad, f"rows {bad[:8]} of {rows} (prefix {prefix}, slab {slab}) differ from the oracle"
