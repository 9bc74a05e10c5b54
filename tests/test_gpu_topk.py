"""GPU parity of the exact top-2048 + page-table transform: every output row is identical to
the oracle's C restatement of the reference single kernel (hcu_ops/csrc/sparse_mask_topk.cu:
141-349) on the same scores -- the same set and the same order (keys above the threshold in
ascending token order, then the ties taken in ascending token order) -- for the reference's ten
score distributions (hcu_ops/tests/topk_lib.py:8-51), ragged / padded rows, the 1M-wide
production layout, every split count, the fused pass-1 path and the varlen layout."""
import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix


pytestmark = pytest.mark.gpu


def _oracle(x, mask, lengths, pt, W, cu=None):
    return topk_radix(x.numpy(), None if mask is None else mask.numpy(), lengths.numpy(), pt.numpy(), W,
                      cu_seqlens_q=None if cu is None else cu.numpy())


IMPLS = {
    "single": lambda x, m, l, p, c: _C.sparse_mask_topk_transform(x, m, l, p, c, 2048),
    "s2": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 2),
    "s8": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 8),
    "s16": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 16),
}


@pytest.mark.parametrize("dist", wl.TOPK_DISTS)
@pytest.mark.parametrize("B", [6, 24])
def test_topk_distributions(gpu, dist, B):
    for L in [1000, 2048, 2049, 4096, 16384, 65536]:
        for ragged in [False, True]:
            W = 2 * L + 64 if ragged and L >= 16384 else L + 64
            x, mask, lengths, pt = wl.topk_scores(B, L, dist, W=W, ragged=ragged, seed=L + B)
            ref = np.asarray(_oracle(x, mask, lengths, pt, W))
            xg, mg, lg, pg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu)
            cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
            for name, fn in IMPLS.items():
                got = np.asarray(fn(xg, mg, lg, pg, cu).cpu().numpy())
                assert np.array_equal(got, ref), f"{dist} B={B} L={L} ragged={ragged} impl={name}"


@pytest.mark.parametrize("dist", wl.TOPK_DISTS)
def test_topk_one_cta_rows_to_16k(gpu, dist):
    """One CTA per row (widths up to 32K never split) at 16,384 tokens wide, one short of it
    (unaligned: scalar loads) and a middle width; full and ragged rows."""
    for W in [16384, 16383, 9000]:
        for ragged in [False, True]:
            L = W if not ragged else W - 5
            x, mask, lengths, pt = wl.topk_scores(24, L, dist, W=W, ragged=ragged, seed=W + ragged)
            ref = np.asarray(_oracle(x, mask, lengths, pt, W))
            xg, mg, lg, pg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu)
            cu = torch.arange(25, dtype=torch.int32, device=gpu)
            got = np.asarray(IMPLS["single"](xg, mg, lg, pg, cu).cpu().numpy())
            assert np.array_equal(got, ref), f"{dist} W={W} ragged={ragged}"


@pytest.mark.parametrize("dist", ["relu_sum", "narrow", "sparse2"])
def test_topk_production_width(gpu, dist):
    """Score width = page-table capacity (1M) with ragged rows of 16K..128K tokens."""
    for L in [16384, 131072]:
        x, mask, lengths, pt = wl.topk_scores(6, L, dist, W=1 << 20, ragged=True, seed=L)
        ref = np.asarray(_oracle(x, mask, lengths, pt, 1 << 20))
        xg, mg, lg, pg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu)
        cu = torch.arange(7, dtype=torch.int32, device=gpu)
        for name, fn in IMPLS.items():
            got = np.asarray(fn(xg, mg, lg, pg, cu).cpu().numpy())
            assert np.array_equal(got, ref), f"W1M {dist} L={L} impl={name}"
        del xg, mg, pg


def _sample_chunks(L):
    """First tokens of the 256 sampled 16-token chunks of a row longer than 4096 tokens (the
    kernel's fixed sample: chunk c starts at ((2c + 1) L / 512) rounded down to 16)."""
    c = np.arange(256)
    return np.minimum((((2 * c + 1) * L) // 512) & ~15, (L - 16) & ~15)


@pytest.mark.parametrize("target", [4600, 7000])
def test_topk_wide_rows_sample_misses(gpu, target):
    """Rows of 131,072 tokens (scores wider than 80K: the one-CTA-per-row and split kernels with
    their larger candidate list) whose sample sits in a narrow band low in the row's distribution, so that the
    sample's threshold collects about `target` keys: 4600 lies past 4096 but within the wide
    list, 7000 past it (the threshold raised from the stored or published keys, the row collected
    once more).  The set and order must equal the oracle's either way (U(0, 1) scores, the
    sample's tokens in [t, t + 1e-3] with t leaving ~target keys above)."""
    L, B = 131072, 4
    g = torch.Generator().manual_seed(target)
    x = torch.rand(B, L, generator=g) * 0.999 + 0.001
    t = 1.0 - target / L
    idx = torch.from_numpy((_sample_chunks(L)[:, None] + np.arange(16)[None, :]).reshape(-1))
    for r in range(B):
        x[r, idx] = t + torch.rand(idx.numel(), generator=g) * 1e-3
    w16 = torch.tensor([1 << i for i in range(16)], dtype=torch.int32)
    bits = (torch.ones(B, L // 16, 16, dtype=torch.int32) * w16).sum(-1, dtype=torch.int32)
    mask = torch.where(bits > 32767, bits - 65536, bits).to(torch.int16).contiguous()
    lengths = torch.tensor([L, L - 5, L - 4096, L - 77], dtype=torch.int32)
    pt = (torch.arange(L, dtype=torch.int32)[None, :] + 11 + 1000000 * torch.arange(B, dtype=torch.int32)[:, None])
    ref = np.asarray(_oracle(x, mask, lengths, pt, L))
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name in ("single", "s2", "s8"):  # the row kernel and the split kernel, both with the wide list
        got = IMPLS[name](x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu), cu)
        assert np.array_equal(np.asarray(got.cpu().numpy()), ref), f"target {target} impl {name}"


@pytest.mark.parametrize("W,target", [(65536, 4600), (65536, 9000), (131072, 7000)])
def test_topk_second_pass_masked_blocks(gpu, W, target):
    """The second collection pass (rows whose sampled threshold collects more keys than the
    candidate list holds: 4096 entries up to 80K-wide scores, 5120 past it) on masked rows: 5% of
    the tokens are masked out and hold NaN or 5.0 (above every kept score), which neither pass may
    take.  Both list sizes, the row and split kernels, and the block-table form, whose table here
    expands to the page table the other forms read."""
    B = 4
    g = torch.Generator().manual_seed(W + target)
    x = torch.rand(B, W, generator=g) * 0.999 + 0.001
    t = 1.0 - target / W
    idx = torch.from_numpy((_sample_chunks(W)[:, None] + np.arange(16)[None, :]).reshape(-1))
    for r in range(B):
        x[r, idx] = t + torch.rand(idx.numel(), generator=g) * 1e-3
    keep = torch.rand(B, W, generator=g) >= 0.05
    drop = ~keep
    x[drop] = torch.where(torch.rand(int(drop.sum()), generator=g) < 0.5, torch.tensor(float("nan")),
                          torch.tensor(5.0))
    w16 = torch.tensor([1 << i for i in range(16)], dtype=torch.int32)
    bits = (keep.view(B, W // 16, 16).to(torch.int32) * w16).sum(-1, dtype=torch.int32)
    mask = torch.where(bits > 32767, bits - 65536, bits).to(torch.int16).contiguous()
    lengths = torch.tensor([W, W - 5, W - 4096, W - 77], dtype=torch.int32)
    bt = torch.randperm(B * W // 64 + 5, generator=g)[:B * W // 64].view(B, W // 64).to(torch.int32)
    tok = torch.arange(W, dtype=torch.int64)
    pt = (bt.long()[:, tok // 64] * 64 + tok % 64).to(torch.int32)
    ref = np.asarray(_oracle(x, mask, lengths, pt, W))
    xg, mg, lg, pg, bg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu), bt.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name in ("single", "s2", "s8"):
        got = IMPLS[name](xg, mg, lg, pg, cu)
        assert np.array_equal(np.asarray(got.cpu().numpy()), ref), f"W={W} target {target} impl {name}"
    for splits in (1, 8):
        got = _C.sparse_mask_topk_transform_blocks(xg, mg, lg, bg, cu, 2048, splits, None, False)
        assert np.array_equal(np.asarray(got.cpu().numpy()), ref), f"W={W} target {target} blocks, splits {splits}"


def test_topk_many_rows_and_empty(gpu):
    x, mask, lengths, pt = wl.topk_scores(600, 5000, "relu_sum", W=5056, ragged=True, seed=1)
    ref = np.asarray(_oracle(x, mask, lengths, pt, 5056))
    out = hcu_ops.sparse_mask_topk_transform(x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu),
                                             torch.arange(601, dtype=torch.int32, device=gpu))
    assert np.array_equal(np.asarray(out.cpu().numpy()), ref)
    e = torch.empty(0, 4096, device=gpu)
    out = hcu_ops.sparse_mask_topk_transform(e, torch.empty(0, 256, dtype=torch.int16, device=gpu),
                                             torch.empty(0, dtype=torch.int32, device=gpu),
                                             torch.empty(0, 4096, dtype=torch.int32, device=gpu),
                                             torch.zeros(1, dtype=torch.int32, device=gpu))
    assert tuple(out.shape) == (0, 2048)


def test_topk_dense_and_varlen(gpu):
    """Dense scores (no mask) with the varlen layout: rows map to their request's page table."""
    x, _, lengths, _ = wl.topk_scores(7, 9000, "mixed", seed=5)
    lengths = torch.tensor([9000, 3000, 2048, 2049, 8999, 100, 6000], dtype=torch.int32)
    cu = torch.tensor([0, 3, 4, 7], dtype=torch.int32)
    pt = (torch.arange(9000, dtype=torch.int32)[None, :] + 100000 * torch.arange(3, dtype=torch.int32)[:, None])
    ref = np.asarray(_oracle(x, None, lengths, pt, 9000, cu=cu))
    for splits in [1, 4]:
        got = hcu_ops.topk_transform(x.to(gpu), lengths.to(gpu), pt.contiguous().to(gpu), cu.to(gpu),
                                     max_splits=splits)
        assert np.array_equal(np.asarray(got.cpu().numpy()), ref), f"splits={splits}"


@pytest.mark.parametrize("fused", [False, True])
@pytest.mark.parametrize("group,lens", [(1, [40000, 12000, 4000, 1000]), (2, [65536, 60000, 3000, 2100, 900, 20000])])
def test_topk_pass1_pairing(gpu, monkeypatch, fused, group, lens):
    """mqa_logits(hist_lens=lengths) -> sparse_mask_topk_transform consumes the paired pass-1
    workspace (zeroed by the logits call, or filled by it when fused) and gives the same set as
    the top-k with its own pass 1 on the same logits."""
    monkeypatch.setattr(hcu_ops, "_MQA_HIST_MAX_ROWS", 1000 if fused else 0)
    monkeypatch.setattr(hcu_ops, "_MQA_HIST_MAX_ROWS_G6", 1000 if fused else 0)
    case = wl.decode_case(17, lens, group=group, heads=64)
    gl = lambda t: t.to(gpu)
    q8, w = hcu_ops.quant_q_fp8(gl(case.q), gl(case.w))
    lens = gl(case.context_lens)
    pt = gl(case.page_table_1())
    cu = torch.arange(case.rows + 1, dtype=torch.int32, device=gpu)
    lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), gl(case.kv), w, lens, gl(case.block_table), case.width, group,
                                  hist_lens=lens)
    assert hcu_ops._MQA_HIST is not None and hcu_ops._MQA_HIST[3] == fused
    paired = hcu_ops.sparse_mask_topk_transform(lg, mask, lens, pt, cu)
    assert hcu_ops._MQA_HIST is None
    plain = _C.sparse_mask_topk_transform(lg, mask, lens, pt, cu, 2048)
    ref = _oracle(lg.cpu(), mask.cpu(), case.context_lens, case.page_table_1(), case.width)
    assert np.array_equal(np.asarray(paired.cpu().numpy()), np.asarray(ref))
    assert np.array_equal(np.asarray(plain.cpu().numpy()), np.asarray(ref))


def _sample_tokens(L):
    """Tokens the sampled threshold reads in a row of L > 4096 tokens: 256 chunks of 16 aligned
    tokens at ((2c + 1) L / 512) & ~15, the last ones clamped to (L - 16) & ~15."""
    starts = [min(((2 * c + 1) * L // 512) & ~15, (L - 16) & ~15) for c in range(256)]
    return np.unique(np.concatenate([np.arange(s, s + 16) for s in starts]))


@pytest.mark.parametrize("pattern", ["sample_high", "sample_low"])
def test_topk_sampled_threshold_fallback(gpu, pattern):
    """Scores placed against the sample: high exactly where it looks (K* lands above all but a
    few hundred keys: too few collected) or low there (K* lands below almost every key: too many
    collected).  Both take the exact path; the sets still match the oracle for every split."""
    B, W = 6, 65536 + 64
    g = torch.Generator().manual_seed(11)
    x = torch.rand(B, W, generator=g)
    lengths = torch.tensor([65536, 40000, 16384, 9000, 4097, 70000 - 9000], dtype=torch.int32)
    for b in range(B):
        L = int(lengths[b])
        s = torch.from_numpy(_sample_tokens(L))
        if pattern == "sample_high":
            x[b, s] += 10.0
        else:
            keep = torch.ones(W, dtype=torch.bool)
            keep[s] = False
            x[b, keep] += 10.0
    mask = torch.full((B, (W + 15) // 16), -1, dtype=torch.int16)
    pt = (torch.arange(W, dtype=torch.int32)[None, :] + 7 + 1000000 * torch.arange(B, dtype=torch.int32)[:, None])
    ref = np.asarray(_oracle(x, mask, lengths, pt, W))
    xg, mg, lg, pg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = np.asarray(fn(xg, mg, lg, pg, cu).cpu().numpy())
        assert np.array_equal(got, ref), f"{pattern} impl={name}"
    got = hcu_ops.topk_transform(xg, lg, pg, cu, max_splits=1)
    assert np.array_equal(np.asarray(got.cpu().numpy()), ref), f"{pattern} dense"
    # into a caller's buffer: rows 1.. of a larger output, the other rows untouched
    buf = torch.full((B + 1, 2048), -7, dtype=torch.int32, device=gpu)
    ret = hcu_ops.topk_transform(xg, lg, pg, cu, max_splits=1, out=buf[1:])
    assert ret.data_ptr() == buf[1:].data_ptr()
    assert np.array_equal(np.asarray(buf[1:].cpu().numpy()), ref), f"{pattern} dense into out"
    assert (buf[0] == -7).all()


def _crowded_row(g, L, m, need, kind):
    """A row of L tokens whose threshold 12-bit digit (key[31:20]) holds exactly m members, of
    which `need` are taken: 2048 - need tokens far above (>= 4.0), m members in [1.0, 1.125)
    (low 20 key bits u: distinct, five values, one value, or one key[19:10] bucket), the rest
    below 1.0; positions shuffled."""
    if kind == "distinct":
        u = torch.randperm(1 << 20, generator=g)[:m]
    elif kind == "ties5":
        u = torch.randperm(1 << 20, generator=g)[:5][torch.randint(0, 5, (m,), generator=g)]
    elif kind == "equal":
        u = torch.full((m,), 12345)
    else:  # "bucket": one key[19:10] value, the order settled by key[9:0] alone
        u = 777 * 1024 + torch.randint(0, 1024, (m,), generator=g)
    members = (torch.full((m,), 0x3F800000, dtype=torch.int32) + u.to(torch.int32)).view(torch.float32)
    above = 4.0 + torch.randperm(2048 - need, generator=g).float()
    rest = torch.rand(L - (2048 - need) - m, generator=g) * 1.8 - 0.9
    vals = torch.cat([above, members, rest])
    return vals[torch.randperm(L, generator=g)]


@pytest.mark.parametrize("W", [4160, 4161, 40000, 40001])
def test_topk_short_rows_crowded_threshold_digit(gpu, W):
    """Rows of 2049..4096 tokens (resolved whole in one CTA on key[31:20]) whose threshold digit
    holds 1 to 513 members -- distinct keys, five keys, one key, or one key[19:10] bucket -- with
    1, half or all of them taken: the selection among the members (by register ranking up to 64,
    pairwise LDS ranking up to 128, two radix passes over key[19:0] up to 512, the heavy-tie path
    past it) matches the oracle, set and order, for every implementation.  Blocks 4160 / 4161
    tokens wide take the one-CTA-per-row kernel, 40000 / 40001 the split kernel (its short-row
    path, as for the short rows of a wide decode batch); the odd widths take the buffer loads."""
    g = torch.Generator().manual_seed(23)
    rows = []
    for m in [1, 2, 63, 64, 65, 128, 129, 300, 512, 513]:
        for need in sorted({1, max(1, m // 2), m}):
            for kind in ["distinct", "ties5", "equal", "bucket"]:
                lo = 2048 - need + m
                L = max(2049, int(torch.randint(lo, 4097, (1,), generator=g)))
                rows.append((L, m, need, kind))
    B = len(rows)
    x = torch.full((B, W), 1e30)  # past a row's length: never read as a score
    for b, (L, m, need, kind) in enumerate(rows):
        x[b, :L] = _crowded_row(g, L, m, need, kind)
    lengths = torch.tensor([r[0] for r in rows], dtype=torch.int32)
    mask = torch.full((B, (W + 15) // 16), -1, dtype=torch.int16)
    pt = torch.arange(W, dtype=torch.int32)[None, :] + 3 + 100000 * torch.arange(B, dtype=torch.int32)[:, None]
    ref = np.asarray(_oracle(x, mask, lengths, pt, W))
    xg, mg, lg, pg = x.to(gpu), mask.to(gpu), lengths.to(gpu), pt.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = np.asarray(fn(xg, mg, lg, pg, cu).cpu().numpy())
        bad = [rows[b] for b in range(B) if not np.array_equal(got[b], ref[b])]
        assert not bad, f"W={W} impl={name}: rows (L, members, taken, keys) {bad[:4]}"
    got = np.asarray(hcu_ops.topk_transform(xg, lg, pg, cu, max_splits=1).cpu().numpy())
    assert np.array_equal(got, ref), f"W={W} dense"


def test_topk_page_table_without_columns(gpu):
    """A page table whose rows hold no entries (a zero-column view of a real table): every selected
    or copied token maps to -1, on every path, without reading the table."""
    x, mask, lengths, _ = wl.topk_scores(3, 5000, "mixed", W=5056, ragged=False, seed=77)
    lengths = torch.tensor([5000, 100, 3000], dtype=torch.int32)
    base = torch.arange(3 * 64, dtype=torch.int32).view(3, 64).to(gpu)
    pt = base[:, :0]
    cu = torch.arange(4, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = fn(x.to(gpu), mask.to(gpu), lengths.to(gpu), pt, cu).cpu().numpy()
        assert (got == -1).all(), name
