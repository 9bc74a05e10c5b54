"""Pins the oracle's indexer functions (oracle/indexer.py, oracle/topk_radix.c) against
independent restatements: torch-CPU closed forms, pure-Python loops on tiny inputs, the
C radix select, and invariants of the mathematics."""
import numpy as np
import pytest
import torch

import workloads as wl
from oracle import indexer as O
from oracle.fp8 import bf16_rne, float_key, fp8_decode
from oracle.topk_c import topk_radix


def _kv_np(case):
    return case.kv.view(case.kv.shape[0], -1).numpy()


def _torch_tokens(kv, pages, off):
    """fp8 values (as float32) and scales of tokens (pages[i], off[i]) of the paged layout
    [64 x 128 fp8][64 x f32] with torch ops."""
    flat = kv.view(kv.shape[0], -1)
    cols = off[:, None] * 128 + torch.arange(128)[None, :]
    k8 = flat[pages[:, None], cols].contiguous().view(torch.float8_e4m3fn).float()
    sc = flat[pages[:, None], 8192 + off[:, None] * 4 + torch.arange(4)[None, :]].contiguous().view(torch.float32)
    return k8, sc.flatten()


# ---------------------------------------------------------------------------------------------
# dequant / quant

def test_dequant_matches_torch_closed_form():
    case = wl.decode_case(11, [300, 200], group=1, heads=32)
    kv = _kv_np(case)
    slots = torch.randperm(kv.shape[0] * 64, generator=torch.Generator().manual_seed(1))[:500].numpy()
    got = O.dequant_k_paged(kv, slots)
    page, off = slots // 64, slots % 64
    k8, sc = _torch_tokens(case.kv, torch.from_numpy(page), torch.from_numpy(off))
    ref = (k8 * sc[:, None]).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, ref)


def test_dequant_all_codes_and_edge_scales():
    # one page per scale; even tokens hold codes 0..127, odd tokens codes 128..255
    scales = np.array([1.0, 2.0 ** -20, 3.0e-3, 1.7e5, 2.0 ** -126, 6.1e-5, 0.0, 448.0], dtype=np.float32)
    kv = np.zeros((len(scales), 64 * 132), dtype=np.uint8)
    for p, s in enumerate(scales):
        for t in range(64):
            kv[p, t * 128:(t + 1) * 128] = (np.arange(128) + 128 * (t % 2)).astype(np.uint8)
            kv[p, 8192 + t * 4:8192 + t * 4 + 4] = np.array([s], dtype=np.float32).view(np.uint8)
    slots = np.arange(len(scales) * 64)
    got = O.dequant_k_paged(kv, slots)
    codes = torch.from_numpy(kv[:, :8192].reshape(-1, 128).copy())
    sc = torch.from_numpy(np.repeat(scales, 64))
    ref = (codes.view(torch.float8_e4m3fn).float() * sc[:, None]).to(torch.bfloat16).view(torch.int16).numpy()
    ref = ref.view(np.uint16)
    # NaN codes (0x7F / 0xFF) and 0 * NaN: any bf16 NaN is a NaN (torch's vectorised cast does not
    # canonicalise it; the oracle and the kernels emit 0x7FC0); every other value bit-exact.
    is_nan = lambda b: ((b & 0x7F80) == 0x7F80) & ((b & 0x7F) != 0)
    assert np.array_equal(is_nan(got), is_nan(ref))
    assert np.all(got[is_nan(got)] == 0x7FC0)
    assert np.array_equal(got[~is_nan(ref)], ref[~is_nan(ref)])


def test_dequant_mla_matches_torch_closed_form():
    g = torch.Generator().manual_seed(2)
    pool = 64
    cache = (torch.randn(pool, 656, generator=g) * 0.1).to(torch.float8_e4m3fn).view(torch.uint8)
    # realistic positive scales and a finite rope part
    cache[:, 512:528] = (torch.rand(pool, 4, generator=g) * 0.02 + 1e-3).view(torch.uint8)
    cache[:, 528:] = torch.randn(pool, 64, generator=g).to(torch.bfloat16).view(torch.uint8)
    slots = torch.randint(0, pool, (100,), generator=g)
    got = O.dequant_mla(cache.numpy(), slots.numpy())
    rows = cache[slots]
    nope = rows[:, :512].contiguous().view(torch.float8_e4m3fn).float().view(-1, 4, 128)
    sc = rows[:, 512:528].contiguous().view(torch.float32)
    ref_nope = (nope * sc[:, :, None]).view(-1, 512).to(torch.bfloat16)
    ref = torch.cat([ref_nope, rows[:, 528:].contiguous().view(torch.bfloat16)], 1)
    assert np.array_equal(got, ref.view(torch.int16).numpy().view(np.uint16))
    # padded entries (negative slots) are zero rows; the other rows are unchanged
    neg = slots.clone()
    neg[::7] = -1
    got2 = O.dequant_mla(cache.numpy(), neg.numpy())
    keep = neg.numpy() >= 0
    assert (got2[~keep] == 0).all() and np.array_equal(got2[keep], got[keep])


def test_cpu_dequant_torch_matches_numpy_oracle():
    """The torch-CPU dequant of the multi-thread CPU baseline gives the numpy oracle's bits (both
    layouts), so the baseline times the same computation."""
    case = wl.decode_case(12, [700, 300], group=1, heads=32)
    kv = _kv_np(case)
    slots = torch.randperm(kv.shape[0] * 64, generator=torch.Generator().manual_seed(3))[:900]
    got = O.cpu_dequant_torch(torch.from_numpy(kv), slots, mla=False).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, O.dequant_k_paged(kv, slots.numpy()))
    g = torch.Generator().manual_seed(4)
    pool = 50
    cache = (torch.randn(pool, 656, generator=g) * 0.1).to(torch.float8_e4m3fn).view(torch.uint8)
    cache[:, 512:528] = (torch.rand(pool, 4, generator=g) * 0.02 + 1e-3).view(torch.uint8)
    cache[:, 528:] = torch.randn(pool, 64, generator=g).to(torch.bfloat16).view(torch.uint8)
    slots = torch.randint(0, pool, (300,), generator=g)
    got = O.cpu_dequant_torch(cache, slots, mla=True).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, O.dequant_mla(cache.numpy(), slots.numpy()))


def test_quant_vectors_matches_torch_generator():
    g = torch.Generator().manual_seed(9)
    x = torch.cat([torch.randn(5000, 128, generator=g) * 3, torch.zeros(2, 128),
                   torch.randn(10, 128, generator=g) * 1e-30])
    ref8, ref_s = wl.quantize_tokens(x)
    codes, scale = O.quant_vectors(x.numpy())
    assert np.array_equal(codes, ref8.view(torch.uint8).numpy())
    assert np.array_equal(scale.view(np.uint32), ref_s.numpy().view(np.uint32))
    # invariants: |q| <= 448, the largest element of every nonzero row encodes to +-448
    vals = fp8_decode(codes)
    assert np.all(np.abs(vals) <= 448)
    nz = scale > 0
    assert np.all(np.abs(vals[nz]).max(-1) == 448)


def test_build_kv_cache_matches_workload_packing():
    g = torch.Generator().manual_seed(4)
    k = torch.randn(3 * 64, 128, generator=g)
    k8, sc = wl.quantize_tokens(k)
    packed = wl.pack_kv_pages(k8, sc, 3).view(3, -1).numpy()
    got = O.build_kv_cache(k.numpy(), np.arange(192), 3)
    assert np.array_equal(got, packed)


# ---------------------------------------------------------------------------------------------
# logits

def _torch_logits(case, r):
    """Independent torch fp32 restatement of one row (dequant -> matmul -> relu*w -> sum -> *s)."""
    L = int(case.context_lens[r])
    g0 = (r // case.group) * case.group
    t = torch.arange(L)
    pages = case.block_table[g0].long()[t // 64]
    off = t % 64
    k8, s = _torch_tokens(case.kv, pages, off)
    q8, w = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    q = torch.from_numpy(fp8_decode(q8[r]))
    acc = q @ k8.T
    return ((torch.relu(acc) * torch.from_numpy(w[r])[:, None]).sum(0) * s).double().numpy()


def test_logits_oracle_matches_torch_fp32():
    case = wl.decode_case(21, [700, 1500], group=2, heads=64)
    q8, w = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    lg, mag, _, mask = O.mqa_logits_decode(q8, w, _kv_np(case), case.context_lens.numpy(), case.block_table.numpy(),
                                        case.group, case.width)
    for r in range(case.rows):
        L = int(case.context_lens[r])
        ref = _torch_logits(case, r)
        err = np.abs(lg[r, :L] - ref)
        assert np.all(err <= 1e-5 * mag[r, :L] + 1e-30)
        assert np.all(np.isnan(lg[r, L:]))
    bits = O.unpack_mask(mask, case.width)
    assert np.array_equal(bits, np.nan_to_num(lg, nan=0.0) != 0)


def test_logits_oracle_pure_python_tiny():
    rng = np.random.default_rng(0)
    H, n = 3, 5
    q8 = rng.integers(0, 256, (H, 128)).astype(np.uint8)
    q8[(q8 & 0x7F) == 0x7F] = 0
    k8 = rng.integers(0, 256, (n, 128)).astype(np.uint8)
    k8[(k8 & 0x7F) == 0x7F] = 0
    w = rng.standard_normal(H).astype(np.float32)
    s = rng.random(n).astype(np.float32)
    lg, _, _ = O.logits_row(q8, w, k8, s)
    qv, kv = fp8_decode(q8).tolist(), fp8_decode(k8).tolist()
    for t in range(n):
        tot = 0.0
        for h in range(H):
            acc = 0.0
            for d in range(128):
                acc += float(qv[h][d]) * float(kv[t][d])
            tot += float(w[h]) * max(acc, 0.0)
        assert abs(tot * float(s[t]) - lg[t]) <= 1e-12 * max(1.0, abs(lg[t]))


def test_logits_linear_in_weights_and_scale():
    rng = np.random.default_rng(1)
    q8 = rng.integers(0, 126, (8, 128)).astype(np.uint8) ^ (rng.integers(0, 2, (8, 128)) * 0x80).astype(np.uint8)
    k8 = rng.integers(0, 126, (40, 128)).astype(np.uint8) ^ (rng.integers(0, 2, (40, 128)) * 0x80).astype(np.uint8)
    w1, w2 = rng.standard_normal(8).astype(np.float32), rng.standard_normal(8).astype(np.float32)
    s = rng.random(40).astype(np.float32)
    a, _, _ = O.logits_row(q8, w1, k8, s)
    b, _, _ = O.logits_row(q8, w2, k8, s)
    c, _, _ = O.logits_row(q8, (w1.astype(np.float64) + w2).astype(np.float32), k8, s)
    assert np.allclose(a + b, c, rtol=1e-6, atol=1e-6)
    d, _, _ = O.logits_row(q8, w1, k8, (2 * s).astype(np.float32))
    assert np.array_equal(d, 2 * a)
    # all dot products negative -> relu kills everything -> exact zeros (mask bit clear)
    neg = np.full((8, 128), 0x38, dtype=np.uint8)  # +1.0
    kneg = np.full((3, 128), 0xB8, dtype=np.uint8)  # -1.0
    z, _, _ = O.logits_row(neg, w1, kneg, s[:3])
    assert np.all(z == 0.0)


def test_quant_q_scale_folding():
    """w_eff * relu(q8 . k) reproduces w * relu(q . k) up to the fp8 rounding of q."""
    case = wl.decode_case(5, [256], group=1, heads=8)
    qb = case.q.view(torch.int16).numpy().view(np.uint16)
    q8, weff = O.quant_q(qb, case.w.numpy())
    qf = (qb.astype(np.uint32) << 16).view(np.float32)
    amax = np.abs(qf).max(-1)
    assert np.array_equal(weff, (case.w.numpy() * (amax / np.float32(448))).astype(np.float32))
    rel = np.abs(fp8_decode(q8) * (amax / 448)[..., None] - qf) / np.maximum(np.abs(qf), 1e-30)
    assert np.quantile(rel[np.abs(qf) > amax[..., None] / 8], 0.999) <= 2.0 ** -4


# ---------------------------------------------------------------------------------------------
# top-k

def _pure_python_topk(keys, k=2048):
    idx = sorted(range(len(keys)), key=lambda t: (-int(keys[t]), t))
    return sorted(idx[:k])


@pytest.mark.parametrize("dist", wl.TOPK_DISTS)
@pytest.mark.parametrize("L,ragged", [(1000, False), (2048, False), (2049, False), (4096, True), (9000, False),
                                      (20000, True)])
def test_topk_bruteforce_vs_c_radix(dist, L, ragged):
    W = L + 64 if not ragged else 2 * L + 64
    x, mask, lengths, pt = wl.topk_scores(4, L, dist, W=W, ragged=ragged, seed=L)
    xs, ms, ls, ps = x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy()
    brute = O.topk_transform(xs, ms, ls, ps, W)
    rad = topk_radix(xs, ms, ls, ps, W)
    assert np.array_equal(np.sort(brute, 1), np.sort(rad, 1))
    for r in range(4):
        n = min(int(ls[r]), W)
        if n <= 2048:
            assert np.array_equal(rad[r, :n], ps[r, :n]) and np.all(rad[r, n:] == -1)
            continue
        # invariants (topk_lib.py:70-89): unique, below the length, 2048 selected
        tok = rad[r] - 7 - 1000000 * r
        assert len(set(tok.tolist())) == 2048 and tok.min() >= 0 and tok.max() < n
        # every selected key >= every unselected key; ties at the threshold favour lower t
        keys = O.row_keys(xs[r], ms[r], n)
        sel = np.zeros(n, dtype=bool)
        sel[tok] = True
        thr = keys[sel].min()
        assert np.all(keys[~sel] <= thr)
        tie_sel = np.nonzero(sel & (keys == thr))[0]
        tie_uns = np.nonzero(~sel & (keys == thr))[0]
        if tie_uns.size:
            assert tie_sel.max() < tie_uns.min()


@pytest.mark.parametrize("dist", wl.TOPK_DISTS)
def test_topk_c_radix_output_order_is_reference_order(dist):
    """[keys > threshold, ascending t][ties, ascending t] (sparse_mask_topk.cu:301-348), the
    threshold being +0 whenever positives <= 2048 <= positives + zeros (the sparse fast path,
    :199-234; with exactly 2048 positives every selected key is above it) and the 2048th largest
    key otherwise: the C restatement's rows equal the brute-force selection put in that order.
    Rows with exactly 2048 positives (the smallest positive would otherwise count as a tie) are
    included on purpose."""
    x, mask, lengths, pt = wl.topk_scores(3, 6000, dist, W=6064, ragged=True, seed=3)
    xs, ms, ls, ps = x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy()
    x2 = np.random.default_rng(5).standard_normal((2, 5000)).astype(np.float32)
    x2[:, :2048] = np.abs(x2[:, :2048]) + 1e-3  # exactly 2048 positives
    x2[:, 2048:] = -np.abs(x2[:, 2048:])
    x2[1, 3000:3100] = 0.0                      # ... and some zeros
    x2 = np.ascontiguousarray(np.stack([np.random.default_rng(6 + i).permutation(x2[i]) for i in range(2)]))
    cases = [(xs, ms, ls, ps, 6064), (x2, None, np.array([5000, 5000], dtype=np.int32),
                                      np.tile(np.arange(5000, dtype=np.int32), (2, 1)) + 11, 5000)]
    for xs, ms, ls, ps, W in cases:
        out = topk_radix(xs, ms, ls, ps, W)
        for r in range(xs.shape[0]):
            n = min(int(ls[r]), W)
            keys = O.row_keys(xs[r], None if ms is None else ms[r], n)
            sel = O.topk_tokens(keys)  # ascending t
            pos, zeros = int((keys > O.ZERO_KEY).sum()), int((keys == O.ZERO_KEY).sum())
            thr = O.ZERO_KEY if pos <= 2048 <= pos + zeros else keys[sel].min()
            want = np.concatenate([sel[keys[sel] > thr], sel[keys[sel] == thr]])
            assert np.array_equal(out[r], ps[r][want])


def test_topk_pure_python_tiny():
    rng = np.random.default_rng(3)
    for trial in range(4):
        n = 2048 + int(rng.integers(1, 300))
        x = rng.integers(-20, 20, n).astype(np.float32) / 4  # heavy ties incl. +-0
        keys = float_key(x)
        assert O.topk_tokens(keys).tolist() == _pure_python_topk(keys)


def test_topk_varlen_layout():
    x, mask, lengths, _ = wl.topk_scores(6, 5000, "mixed", seed=1)
    cu = np.array([0, 2, 3, 6], dtype=np.int32)
    pt = (np.arange(5000)[None, :] + 100000 * np.arange(3)[:, None]).astype(np.int32)
    brute = O.topk_transform(x.numpy(), mask.numpy(), lengths.numpy(), pt, 5000, cu_seqlens_q=cu)
    rad = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt, 5000, cu_seqlens_q=cu)
    assert np.array_equal(np.sort(brute, 1), np.sort(rad, 1))
    assert np.all(brute[3:6] >= 200000) and np.all(brute[0:2] < 100000)


def test_topk_narrow_page_table():
    """A page-table row narrower than the row: tokens past its columns map to -1 in both oracles
    (brute force and the C radix), short rows included; the other entries are the table's."""
    x, mask, lengths, _ = wl.topk_scores(4, 6000, "mixed", seed=4)
    lengths = torch.tensor([6000, 5000, 1900, 4100], dtype=torch.int32)
    x[0, 4000:6000] = torch.nan_to_num(x[0, 4000:6000]).abs() + 1000.0  # row 0 selects past the table
    pt = (np.arange(4500)[None, :] * 3 + 7 + 100000 * np.arange(4)[:, None]).astype(np.int32)[:, :1800]
    brute = O.topk_transform(x.numpy(), mask.numpy(), lengths.numpy(), pt, 6000)
    rad = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt, 6000)
    assert np.array_equal(np.sort(brute, 1), np.sort(rad, 1))
    wide = (np.arange(6000)[None, :] * 3 + 7 + 100000 * np.arange(4)[:, None]).astype(np.int32)
    full = O.topk_transform(x.numpy(), mask.numpy(), lengths.numpy(), wide, 6000)
    expect = np.where((full - 7 - 100000 * np.arange(4)[:, None]) // 3 < 1800, full, -1)
    expect[full == -1] = -1
    assert np.array_equal(brute, expect)
    assert (brute[0] == -1).sum() > 0 and (brute[2, 1800:1900] == -1).all()


def test_pass1_hist_closed_form():
    """Histogram restated with torch ops exactly as hcu_ops/tests/test_mqa_hist.py:109-124."""
    x, mask, lengths, _ = wl.topk_scores(5, 6000, "relu_sum", W=8000, ragged=True, seed=2)
    lengths[2] = 1500
    W = 8000
    ws = O.pass1_hist(x.numpy(), mask.numpy(), lengths.numpy(), W)
    bits16 = torch.arange(16, dtype=torch.int32)
    mm = ((mask.int().unsqueeze(-1) >> bits16) & 1).flatten(1)[:, :W].bool()
    lg = torch.nan_to_num(x, nan=0.0)
    h = lengths.long().clamp(max=W)
    act = h > 2048
    sel = mm & (torch.arange(W) < h[:, None]) & act[:, None]
    b = lg.contiguous().view(torch.int32).long() & 0xFFFFFFFF
    key = torch.where(b >= 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    g1 = torch.zeros(5, 4096, dtype=torch.long)
    g1.scatter_add_(1, torch.where(sel, key >> 20, 0), sel.long())
    nz = sel.sum(1)
    zeros = torch.where(act, h - nz, 0)
    g1[:, 0x800] += zeros
    pos = (sel & (key > 0x80000000)).sum(1)
    ref = torch.cat([g1.flatten(), torch.zeros(5 * 4096, dtype=torch.long),
                     torch.stack([pos, zeros], 1).flatten()]).int().numpy()
    assert np.array_equal(ws, ref)


def test_cpu_baseline_row_matches_oracle():
    case = wl.decode_case(31, [5000], group=1, heads=64)
    q8, w = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    kv = _kv_np(case)
    lg, _, _, mask = O.mqa_logits_decode(q8, w, kv, case.context_lens.numpy(), case.block_table.numpy(), 1, case.width)
    pt = case.page_table_1().numpy()
    ref = O.topk_transform(lg.astype(np.float32), mask, case.context_lens.numpy(), pt, case.width)
    slots = O.slots_of(case.block_table.numpy()[0], 5000)
    codes, sc = O.kv_tokens(kv, slots)
    got = O.cpu_indexer_row_torch(torch.from_numpy(fp8_decode(q8[0])), torch.from_numpy(w[0]),
                                  torch.from_numpy(fp8_decode(codes)), torch.from_numpy(sc),
                                  torch.from_numpy(slots.astype(np.int32)))
    # fp32 vs fp64 logits may reorder near-ties at the threshold: compare the sets up to a few
    assert len(set(got.tolist()) ^ set(ref[0].tolist())) <= 8


def test_prefill_oracle_equals_decode_oracle_with_one_group():
    """The prefill logits of one request's rows equal the decode logits of those rows as one
    group sharing the request's block table (the same closed form, mqa_hist.cu:93-95,162): a
    wrong causal rule, row offset or page mapping in either restatement breaks the equality."""
    case = wl.prefill_case(31, 9, 700, heads=64)
    q8, w = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    kv = _kv_np(case)
    width = case.n_keys + 3
    bt = np.concatenate([case.block_table.numpy(), np.zeros(1, dtype=np.int32)])
    lens = case.lens.numpy().copy()
    lens[2] = 0
    lens[5] = width + 50  # clamped to the width by both
    pre, pre_mag, pre_dmag = O.mqa_logits_prefill(q8, w, kv, bt, lens, width)
    bt2 = np.tile(bt, (case.rows, 1))
    dec, dec_mag, dec_dmag, _ = O.mqa_logits_decode(q8, w, kv, lens, bt2, case.rows, width)
    assert np.array_equal(np.isnan(pre), np.isnan(dec))
    assert np.array_equal(pre[~np.isnan(pre)], dec[~np.isnan(dec)]) and np.array_equal(pre_mag, dec_mag)
    assert np.array_equal(pre_dmag, dec_dmag)
    # and a causal row sees exactly its prefix: row i's logits are row j's on their common keys
    L3, L4 = int(lens[3]), int(lens[4])
    assert L3 < L4 and np.isnan(pre[3, L3:]).all() and not np.isnan(pre[4, :L4]).any()


def test_logits_row_dot_magnitude_brute_force():
    """M_t = s_t sum_h |w_h| sum_d |q8_hd k8_td| by plain loops on a small case, and
    |logit| <= A_t <= M_t."""
    rng = np.random.default_rng(3)
    q8 = rng.integers(0, 256, size=(3, 128)).astype(np.uint8)
    q8[(q8 & 0x7F) == 0x7F] = 0x20  # no NaN codes
    k8 = rng.integers(0, 256, size=(5, 128)).astype(np.uint8)
    k8[(k8 & 0x7F) == 0x7F] = 0x31
    w = rng.normal(size=3).astype(np.float32)
    s = rng.uniform(0.1, 2.0, size=5).astype(np.float32)
    lg, mag, dmag = O.logits_row(q8, w, k8, s)
    qv, kv = fp8_decode(q8).astype(np.float64), fp8_decode(k8).astype(np.float64)
    for t in range(5):
        m = 0.0
        for h in range(3):
            m += abs(float(w[h])) * sum(abs(qv[h, d] * kv[t, d]) for d in range(128))
        assert abs(dmag[t] - m * float(s[t])) <= 1e-12 * dmag[t]
        assert abs(lg[t]) <= mag[t] * (1 + 1e-12) and mag[t] <= dmag[t] * (1 + 1e-12)


def test_quant_fmax_ignores_nan():
    """amax follows fmaxf from 0 (hcu_ops/csrc/norm_quant.cu:13-14): NaN elements do not count;
    an all-NaN vector has amax 0 (codes NaN, scale 0); inf gives scale inf and codes 0 / NaN."""
    x = np.zeros((4, 128), dtype=np.float32)
    x[0, :] = 1.0
    x[0, 5] = np.nan
    x[1, :] = np.nan
    x[2, 3] = np.inf
    x[2, 4] = 2.0
    codes, scale = O.quant_vectors(x)
    assert scale[0] == np.float32(1.0 / 448.0) and codes[0, 0] == 0x7E and codes[0, 5] in (0x7F, 0xFF)
    assert scale[1] == 0 and (codes[1] & 0x7F == 0x7F).all()
    assert np.isinf(scale[2]) and codes[2, 4] == 0 and codes[2, 3] & 0x7F == 0x7F
    assert scale[3] == 0 and (codes[3] == 0).all()
