"""Parity at the full sizes of the five benchmark workloads, through the exact steps bench.py
times (the reference's own tests run production shapes too: hcu_ops/tests/test_mqa_hist.py:25-61,
150-180 at 64K context and graph-capacity width, hcu_ops/tests/test_topk.py:17-54 up to 1M-wide
rows).

Decode (decode_1x4k, decode_32x16k, decode_mtp64 -- the headline): quant_q_fp8 -> mqa_logits(
hist_lens=lens) -> sparse_mask_topk_transform on every row: q8 and the folded weights bit-exact,
the nonzero mask bit-exact, every logit within the tolerance of tests/gpu_util.py against the
exact fp64 oracle, every top-k row identical (set and order) to the oracle's C radix select
on the same logits.

Prefill (prefill_8k_64k, prefill_16k_128k with Student-t K): quant_q_fp8 -> prefill_indexer in
4096-row slabs.  Every row of every slab equals an exact selection computed by torch on the GPU
from the same logits (int64 composite keys (key << 21) | (2^21 - 1 - token), i.e. key
descending, token ascending), put in the reference's order.  About 32 rows spread over the
slabs (the first and last row of each slab among them): q8 / weights bit-exact, logits against the fp64 oracle, and the
top-k row equal to the oracle's C radix select."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix

from gpu_util import check_logits, kv_np, oracle_decode, oracle_q, q_bits

pytestmark = pytest.mark.gpu

SLAB = 4096


def _log(msg):
    print(f"[configs] {msg}", flush=True)


@pytest.mark.timeout(900)
@pytest.mark.parametrize("name", ["decode_1x4k", "decode_32x16k", "decode_mtp64"])
def test_decode_config_full_size(gpu, name):
    case = getattr(wl, name)()
    _log(f"{name}: {case.rows} rows, width {case.width}, {case.tokens_scored()} keys scored")
    g = lambda t: t.to(gpu)
    lens = g(case.context_lens)
    pt = case.page_table_1()
    cu = torch.arange(case.rows + 1, dtype=torch.int32, device=gpu)
    q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
    logits, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), g(case.kv), w, lens, g(case.block_table), case.width,
                                      case.group, hist_lens=lens)
    out = hcu_ops.sparse_mask_topk_transform(logits, mask, lens, g(pt), cu)
    torch.cuda.synchronize()

    rq8, rw = oracle_q(case)
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rq8), "q8 differs from the oracle"
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw.view(np.uint32)), "folded weights differ"
    ref, mag, ref_mask = oracle_decode(case, rq8, rw)
    got_mask = mask.cpu().numpy()
    assert np.array_equal(got_mask, ref_mask), "nonzero mask differs from the oracle"
    got = logits.cpu().numpy()
    worst = 0.0
    for r in range(case.rows):
        L = int(case.context_lens[r])
        wm, _ = check_logits(got[r, :L], ref[r, :L], mag[r, :L], f"{name} row {r}")
        worst = max(worst, wm)
    want = topk_radix(got, got_mask, case.context_lens.numpy(), pt.numpy(), case.width)
    sel = out.cpu().numpy()
    bad = [r for r in range(case.rows) if not np.array_equal(sel[r], want[r])]
    assert not bad, f"{name}: top-k rows {bad[:8]} differ from the oracle's selection"
    _log(f"{name}: {case.rows} rows match; worst logit error / magnitude {worst:.2e}")


def _exact_topk_torch(lg, lens, pt):
    """int32 [rows, 2048]: each row's top-2048 in the reference's output order -- the tokens with
    key > thr ascending, then the ties taken ascending (-1 padded below 2048 tokens) -- as page_table
    entries, computed with torch on the GPU from the logits lg [rows, width] (every entry below
    the row length valid).  The selection is a top-k of int64 composite keys
    (key << 21) | (2^21 - 1 - token): key descending, token ascending."""
    rows, width = lg.shape
    assert width < (1 << 21)
    b = lg.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    key = torch.where(b >= 0x80000000, b ^ 0xFFFFFFFF, b | 0x80000000)
    del b
    t = torch.arange(width, device=lg.device, dtype=torch.int64)
    comp = (key << 21) | ((1 << 21) - 1 - t)[None, :]
    comp.masked_fill_(t[None, :] >= lens.long()[:, None], -1)
    k = min(2048, width)
    _, idx = torch.topk(comp, k, dim=1, sorted=False)
    del comp
    idx = idx.sort(dim=1).values                       # ascending token
    ksel = key.gather(1, idx)
    valid = idx < lens.long()[:, None]
    # the threshold: +0 when positives <= 2048 <= positives + zeros (the reference's sparse fast
    # path), else the 2048th largest key; a short row is copied in order
    inrow = t[None, :] < lens.long()[:, None]
    pos = ((key > 0x80000000) & inrow).sum(dim=1, keepdim=True)
    zeros = ((key == 0x80000000) & inrow).sum(dim=1, keepdim=True)
    thr = torch.where(valid, ksel, torch.full_like(ksel, 1 << 40)).min(dim=1, keepdim=True).values
    thr = torch.where((pos <= 2048) & (pos + zeros >= 2048), torch.full_like(thr, 0x80000000), thr)
    tie = (ksel == thr) & valid & (lens.long()[:, None] > 2048)
    order = torch.sort(tie.to(torch.int8) + 2 * (~valid).to(torch.int8), dim=1, stable=True).indices
    idx = idx.gather(1, order)
    valid = valid.gather(1, order)
    del key, inrow
    sel = torch.where(valid, pt.long()[idx], torch.full_like(idx, -1))
    out = torch.full((rows, 2048), -1, dtype=torch.int64, device=lg.device)
    out[:, :k] = sel
    return out.to(torch.int32)


@pytest.mark.timeout(1200)
@pytest.mark.parametrize("name", ["prefill_8k_64k", "prefill_16k_128k"])
def test_prefill_config_full_size(gpu, name):
    case = getattr(wl, name)()
    rows, width = case.rows, case.n_keys
    _log(f"{name}: {rows} rows x {width} keys (causal), {case.tokens_scored()} keys scored")
    g = lambda t: t.to(gpu)
    kv, bt, lens = g(case.kv), g(case.block_table), g(case.lens)
    pt = case.slots()
    ptg = g(pt)
    q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
    out = hcu_ops.prefill_indexer(q8, w, kv, bt, lens, width, ptg, memory_budget_bytes=SLAB * width * 4,
                                  max_slab_rows=SLAB)
    torch.cuda.synchronize()

    n_slabs = (rows + SLAB - 1) // SLAB
    picks = set(np.linspace(0, rows - 1, 32 - 2 * n_slabs).astype(int).tolist())
    for s in range(n_slabs):
        picks |= {s * SLAB, min(rows, (s + 1) * SLAB) - 1}
    picks = sorted(picks)
    kept = {}
    for s in range(n_slabs):
        r0, r1 = s * SLAB, min(rows, (s + 1) * SLAB)
        lg = hcu_ops.mqa_logits_prefill(q8[r0:r1], w[r0:r1], kv, bt, lens[r0:r1], width)
        want = _exact_topk_torch(lg, lens[r0:r1], ptg)
        diff = (out[r0:r1] != want).any(dim=1).nonzero().flatten()
        assert diff.numel() == 0, f"{name}: slab {s} rows {(diff[:8] + r0).tolist()} differ from the exact selection"
        for r in picks:
            if r0 <= r < r1:
                kept[r] = lg[r - r0].cpu().numpy()
        del lg, want
        _log(f"{name}: slab {s} ({r1 - r0} rows) top-k rows exact")

    idx = np.array(picks)
    rq8, rw = O.quant_q(q_bits(case.q[idx]), case.w[idx].numpy())
    assert np.array_equal(q8[idx].view(torch.uint8).cpu().numpy(), rq8), "q8 differs from the oracle"
    assert np.array_equal(w[idx].cpu().numpy().view(np.uint32), rw.view(np.uint32)), "folded weights differ"
    codes, scale = O.kv_tokens(kv_np(case.kv), O.slots_of(case.block_table.numpy(), width))
    sel = out[idx].cpu().numpy()
    worst = 0.0
    for i, r in enumerate(picks):
        L = int(case.lens[r])
        ref, mag = O.logits_row(rq8[i], rw[i], codes[:L], scale[:L])
        wm, _ = check_logits(kept[r][:L], ref, mag, f"{name} row {r}")
        worst = max(worst, wm)
        want = topk_radix(kept[r][None, :], None, np.array([L], dtype=np.int32), pt.numpy()[None, :], width)
        assert np.array_equal(sel[i], want[0]), f"{name}: row {r} differs from the oracle"
    _log(f"{name}: {len(picks)} sampled rows match the oracle; worst logit error / magnitude {worst:.2e}")
