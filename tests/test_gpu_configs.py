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
slabs (the first and last row of each slab among them): logits against the CPU fp64 oracle
(indexer.logits_row) and the top-k row equal to the oracle's C radix select.  Every row: q8 /
weights bit-exact against the oracle, and every logit within the tolerance against the same
fp64 closed form evaluated on the GPU (chunks of rows, one fp64 matmul per chunk), itself checked
against indexer.logits_row on the sampled rows."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix

from gpu_util import check_logits, check_mask, kv_np, oracle_decode, oracle_q, q_bits

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
    ref, mag, dmag, ref_mask = oracle_decode(case, rq8, rw)
    got_mask = mask.cpu().numpy()
    got = logits.cpu().numpy()
    check_mask(got_mask, got, ref, mag, case.context_lens.numpy(), f"{name} nonzero mask")
    worst = 0.0
    for r in range(case.rows):
        L = int(case.context_lens[r])
        wm, _ = check_logits(got[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"{name} row {r}")
        worst = max(worst, wm)
    want = topk_radix(got, got_mask, case.context_lens.numpy(), pt.numpy(), case.width)
    sel = out.cpu().numpy()
    bad = [r for r in range(case.rows) if not np.array_equal(sel[r], want[r])]
    assert not bad, f"{name}: top-k rows {bad[:8]} differ from the oracle's selection"
    _log(f"{name}: {case.rows} rows match; worst logit error / magnitude {worst:.2e}")


def _ref_logits_gpu(q8, w, k8, kscale, lens):
    """fp64 (logits, magnitude, dot magnitude) [rows, width] of indexer.logits_row on the GPU:
    q8 [rows, H, 128] and k8 [width, 128] fp8 codes decoded exactly, acc = q8 . k8 per head, then
    scale_t * sum_h w_h relu(acc), scale_t * sum_h |w_h| relu(acc) and scale_t * sum_h |w_h|
    |q8| . |k8|; NaN at t >= lens[r]."""
    rows, H, D = q8.shape
    qd = q8.view(torch.float8_e4m3fn).to(torch.float64).reshape(rows * H, D)
    acc = torch.matmul(qd, k8).view(rows, H, -1).clamp_min_(0.0)  # k8: [128, width] fp64, contiguous
    wd = w.to(torch.float64).unsqueeze(1).contiguous()  # [rows, 1, H] @ [rows, H, width]
    wa = wd.abs().contiguous()
    lg = torch.bmm(wd, acc).squeeze(1) * kscale[None, :]
    mag = torch.bmm(wa, acc).squeeze(1) * kscale[None, :]
    del acc
    dots = torch.matmul(qd.abs(), k8.abs()).view(rows, H, -1)
    dmag = torch.bmm(wa, dots).squeeze(1) * kscale[None, :]
    del dots
    t = torch.arange(lg.shape[1], device=lg.device)
    out = t[None, :] >= lens.long()[:, None]
    nan = float("nan")
    return lg.masked_fill_(out, nan), mag.masked_fill_(out, nan), dmag.masked_fill_(out, nan)


def _check_logits_gpu(got, ref, mag, dmag, what):
    """check_logits on the GPU over the finite reference entries: |got - ref| <= RTOL * magnitude,
    and the relative error <= RTOL where the logit is not cancelled (|ref| >= max(magnitude, dot
    magnitude) / CANCEL)."""
    from gpu_util import CANCEL, RTOL
    ok = ~torch.isnan(ref)
    err = (got.to(torch.float64) - ref).abs()
    bad = ok & (err > RTOL * mag + 1e-30)
    assert not bool(bad.any()), f"{what}: {int(bad.sum())} logits outside {RTOL} * magnitude"
    plain = ok & (ref.abs() >= torch.maximum(mag, dmag) / CANCEL) & (mag > 0)
    rel = torch.where(plain, err / ref.abs().clamp_min(1e-300), torch.zeros_like(err))
    worst = float(rel.max()) if rel.numel() else 0.0
    assert worst <= RTOL, f"{what}: relative error {worst:.3e} > {RTOL} on an uncancelled logit"
    return float(torch.where(ok, err / mag.clamp_min(1e-30), torch.zeros_like(err)).max())


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

    # q8 / weights of every row against the oracle; the keys as fp64 for the GPU restatement
    rq8_all, rw_all = O.quant_q(q_bits(case.q), case.w.numpy())
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rq8_all), "q8 differs from the oracle"
    assert np.array_equal(w.cpu().numpy().view(np.uint32), rw_all.view(np.uint32)), "folded weights differ"
    del rq8_all, rw_all
    codes, scale = O.kv_tokens(kv_np(case.kv), O.slots_of(case.block_table.numpy(), width))
    k8 = torch.from_numpy(np.ascontiguousarray(codes)).to(gpu).view(torch.float8_e4m3fn).to(torch.float64)
    k8 = k8.t().contiguous()
    ks = torch.from_numpy(scale).to(gpu).to(torch.float64)
    chunk = 8

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
        worst_all = 0.0
        for c0 in range(r0, r1, chunk):
            c1 = min(r1, c0 + chunk)
            ref, mag, dmag = _ref_logits_gpu(q8[c0:c1], w[c0:c1], k8, ks, lens[c0:c1])
            worst_all = max(worst_all, _check_logits_gpu(lg[c0 - r0:c1 - r0], ref, mag, dmag,
                                                         f"{name} rows {c0}..{c1 - 1}"))
            for r in picks:  # the GPU restatement is the CPU oracle's closed form
                if c0 <= r < c1:
                    L = int(case.lens[r])
                    kept_ref = (ref[r - c0, :L].cpu().numpy(), mag[r - c0, :L].cpu().numpy())
                    kept[("ref", r)] = kept_ref
            del ref, mag, dmag
        del lg, want
        _log(f"{name}: slab {s} ({r1 - r0} rows) top-k rows exact; every logit within tolerance "
             f"(worst error / magnitude {worst_all:.2e})")

    idx = np.array(picks)
    rq8, rw = O.quant_q(q_bits(case.q[idx]), case.w[idx].numpy())
    sel = out[idx].cpu().numpy()
    worst = 0.0
    for i, r in enumerate(picks):
        L = int(case.lens[r])
        ref, mag, dmag = O.logits_row(rq8[i], rw[i], codes[:L], scale[:L])
        gref, gmag = kept[("ref", r)]
        # the same fp64 sums in another order: within a few ulps of the magnitude (the logit itself
        # may cancel)
        d = float((np.abs(gref - ref) / np.maximum(mag, 1e-300)).max())
        assert d <= 1e-12 and np.allclose(gmag, mag, rtol=1e-12, atol=1e-300), \
            f"{name} row {r}: the GPU fp64 restatement differs from indexer.logits_row ({d:.2e} of the magnitude)"
        wm, _ = check_logits(kept[r][:L], ref, mag, dmag, f"{name} row {r}")
        worst = max(worst, wm)
        want = topk_radix(kept[r][None, :], None, np.array([L], dtype=np.int32), pt.numpy()[None, :], width)
        assert np.array_equal(sel[i], want[0]), f"{name}: row {r} differs from the oracle"
    _log(f"{name}: {len(picks)} sampled rows match the oracle; worst logit error / magnitude {worst:.2e}")
