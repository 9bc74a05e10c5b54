"""Edge cases of the reference's checklist for bit-exact claims (tools/ut_bench.py:11-14): NaN,
+-inf and -0.0 (unmasked scores and quantiser inputs), zero-length and padding rows, strided
inputs, a 131,072-token row in every score distribution, and extreme fp8 query codes whose
per-head dot products cancel (the fp32 MFMA accumulation error, bounded against the oracle)."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from hcu_ops import _C
from oracle import indexer as O
from oracle.fp8 import fp8_decode
from oracle.topk_c import topk_radix

from gpu_util import RTOL, kv_np, oracle_decode, oracle_q, q_bits

pytestmark = pytest.mark.gpu

IMPLS = {
    "single": lambda x, m, l, p, c: _C.sparse_mask_topk_transform(x, m, l, p, c, 2048),
    "s2": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 2),
    "s8": lambda x, m, l, p, c: _C.sparse_mask_topk_transform_split(x, m, l, p, c, 2048, 8),
}

F32_NAN_NEG = np.uint32(0xFFC00000).view(np.float32)


def _mask_of(bits):
    """bool [B, W] -> int16 [B, ceil(W / 16)]."""
    return torch.from_numpy(O.pack_mask(bits))


def _pt(B, W):
    return (torch.arange(W, dtype=torch.int32)[None, :] + 7 + 1000000 * torch.arange(B, dtype=torch.int32)[:, None])


@pytest.mark.parametrize("B,L", [(4, 5000), (4, 70000), (24, 9000), (4, 3000)])
def test_topk_nan_inf_signed_zero_unmasked(gpu, B, L):
    """NaN of both signs, +-inf, +-0.0 at unmasked positions rank by the key transform
    (sparse_mask_topk.cu:40-43): +NaN above +inf, -NaN below -inf, -0.0 just below +0; a masked
    NaN is +0.  One row is mostly +NaN of one payload: ties broken by the lower token."""
    rng = np.random.default_rng(L + B)
    W = L + 64
    x = rng.standard_normal((B, W)).astype(np.float32)
    bits = np.ones((B, W), dtype=bool)
    for b in range(B):
        idx = rng.permutation(L)
        x[b, idx[:300]] = np.nan
        x[b, idx[300:400]] = np.inf
        x[b, idx[400:500]] = -np.inf
        x[b, idx[500:600]] = F32_NAN_NEG
        x[b, idx[600:1200]] = -0.0
        x[b, idx[1200:1800]] = 0.0
        bits[b, idx[1800:2400]] = False  # masked out: counted as +0 whatever is stored
        x[b, idx[1800:2000]] = np.nan
    x[0, :L - 100] = np.nan  # heavy ties at the top (same NaN payload)
    x[1, :] = np.where(rng.random(W) < 0.5, -0.0, 0.0).astype(np.float32)  # only signed zeros
    lengths = torch.full((B,), L, dtype=torch.int32)
    mask = _mask_of(bits)
    pt = _pt(B, W)
    xt = torch.from_numpy(x)
    ref = topk_radix(x, mask.numpy(), lengths.numpy(), pt.numpy(), W)
    g = lambda t: t.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = fn(g(xt), g(mask), g(lengths), g(pt), cu).cpu().numpy()
        assert np.array_equal(got, ref), f"B={B} L={L} impl={name}"
    dense_ref = topk_radix(x, None, lengths.numpy(), pt.numpy(), W)
    got = hcu_ops.topk_transform(g(xt), g(lengths), g(pt), cu, max_splits=1).cpu().numpy()
    assert np.array_equal(got, dense_ref), f"B={B} L={L} dense"


def test_topk_zero_negative_and_short_lengths(gpu):
    """Lengths 0, negative, 1, 2048, 2049, the width and past it: short rows copy the page table
    and pad with -1; empty rows are all -1."""
    B, W = 9, 40000 + 64
    x, mask, _, pt = wl.topk_scores(B, 40000, "relu_sum", W=W, seed=2)
    lengths = torch.tensor([0, -5, 1, 2048, 2049, 40000, W, W + 1000, 3], dtype=torch.int32)
    ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), W)
    assert (ref[0] == -1).all() and (ref[1] == -1).all() and ref[2, 0] == pt[2, 0] and (ref[2, 1:] == -1).all()
    g = lambda t: t.to(gpu)
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = fn(g(x), g(mask), g(lengths), g(pt), cu).cpu().numpy()
        assert np.array_equal(got, ref), f"impl={name}"


@pytest.mark.parametrize("L", [30000, 3500])
@pytest.mark.parametrize("extra", [36, 37])
def test_topk_strided_score_mask_and_page_table(gpu, extra, L):
    """Score, mask and page-table rows that are views into wider buffers: row strides above the
    width (extra % 4 == 0 keeps the 16-B score loads, 37 takes the scalar path: buffer loads,
    rows of <= 4096 tokens on the exact path)."""
    B = 6
    W = L + 64
    x, mask, lengths, pt = wl.topk_scores(B, L, "mixed", W=W, ragged=True, seed=7)
    ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), W)
    xs = torch.full((B, W + extra), float("nan"))
    xs[:, :W] = x
    ms = torch.zeros(B, mask.shape[1] + 5, dtype=torch.int16)
    ms[:, :mask.shape[1]] = mask
    ps = torch.full((B, W + 123), -9, dtype=torch.int32)
    ps[:, :W] = pt
    g = lambda t: t.to(gpu)
    xv, mv, pv = g(xs)[:, :W], g(ms)[:, :mask.shape[1]], g(ps)[:, :W]
    assert xv.stride(0) == W + extra and pv.stride(0) == W + 123
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    for name, fn in IMPLS.items():
        got = fn(xv, mv, g(lengths), pv, cu).cpu().numpy()
        assert np.array_equal(got, ref), f"extra={extra} impl={name}"


@pytest.mark.parametrize("dist", wl.TOPK_DISTS)
def test_topk_distributions_128k(gpu, dist):
    """The reference's sweep length 131,072 (hcu_ops/tests/test_topk.py:19) in every distribution,
    plain and ragged."""
    for ragged in [False, True]:
        B, L = 6, 131072
        W = L + 64
        x, mask, lengths, pt = wl.topk_scores(B, L, dist, W=W, ragged=ragged, seed=17)
        ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), W)
        g = lambda t: t.to(gpu)
        cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
        for name, fn in IMPLS.items():
            got = fn(g(x), g(mask), g(lengths), g(pt), cu).cpu().numpy()
            assert np.array_equal(got, ref), f"{dist} ragged={ragged} impl={name}"


def test_quant_special_values(gpu):
    """NaN, +-inf, -0.0, all-zero and single-outlier vectors through the q quantiser: amax by fmaxf
    from 0 (NaN elements do not count; an all-NaN vector has amax 0), bit-exact with the oracle."""
    g = torch.Generator().manual_seed(9)
    q = torch.randn(6, 64, 128, generator=g)
    q[0, 0] = 0.0
    q[0, 1] = -0.0
    q[0, 2, 5] = float("nan")
    q[0, 3, :] = float("nan")
    q[0, 4, 7] = float("inf")
    q[0, 5, 9] = float("-inf")
    q[0, 6, 11] = -0.0
    q[1, 0, 3] = 3e4  # one huge outlier
    q[1, 1, :] = 1e-30  # a tiny (normal) vector: 448 / amax stays finite
    qb = q.to(torch.bfloat16)
    w = torch.randn(6, 64, generator=g)
    w[0, 4] = 0.0  # 0 * inf scale
    q8, weff = hcu_ops.quant_q_fp8(qb.to(gpu), w.to(gpu))
    rc, rw = O.quant_q(q_bits(qb), w.numpy())
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rc)
    got_w = weff.cpu().numpy()
    assert np.array_equal(np.isnan(got_w), np.isnan(rw))
    ok = ~np.isnan(rw)
    assert np.array_equal(got_w[ok].view(np.uint32), rw[ok].view(np.uint32))


def test_decode_logits_extreme_q_cancellation(gpu):
    """q vectors whose fp8 codes are all +-448 (every element at the vector's absmax): one head's
    128 products of up to 448 * 448 cancel to a small sum, and a relative bound on the logit cannot
    hold for every such input.  The fp8 MFMA's error is a fraction of the products it sums (one
    v_mfma_f32_16x16x128_f8f6f4 measured off by up to 1.5e-5 of sum_d |q_hd k_td| on normal keys,
    5e-5 on Student-t(4) keys); on these inputs (normal keys) the logits stay within
    |logit_gpu - logit| <= s_t * (2^-17 * sum_h |w_h| sum_d |q_hd k_td| + 1e-3 * sum_h |w_h|
    relu(acc_h)) -- an empirical bound here, the first term the scale of an fp32 sum of the 128
    products, the second covering the weighted head sum -- checked against the exact fp64 oracle."""
    case = wl.decode_case(23, [3000, 2600], group=1, heads=64)
    g = torch.Generator().manual_seed(23)
    signs = torch.where(torch.rand(case.rows, 32, 128, generator=g) < 0.5, -1.0, 1.0)
    case.q = case.q.clone()
    case.q[:, :32] = signs.to(torch.bfloat16)  # half the heads: codes all +-448
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens = case.context_lens.to(gpu)
    lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), case.kv.to(gpu), w, lens, case.block_table.to(gpu), case.width,
                                  case.group)
    rq8, rw = oracle_q(case)
    assert (np.abs(fp8_decode(rq8[:, :32])) == 448).all()
    ref, mag, _, ref_mask = oracle_decode(case, rq8, rw)
    got = lg.cpu().numpy()
    kvn = kv_np(case.kv)
    worst_plain = worst_bound = 0.0
    for r in range(case.rows):
        L = int(case.context_lens[r])
        codes, scale = O.kv_tokens(kvn, O.slots_of(case.block_table.numpy()[r], L))
        absdot = np.abs(fp8_decode(rq8[r]).astype(np.float64)) @ np.abs(fp8_decode(codes).astype(np.float64)).T
        bound = scale.astype(np.float64) * (2.0 ** -17 * (np.abs(rw[r]).astype(np.float64) @ absdot)) \
            + RTOL * mag[r, :L]
        err = np.abs(got[r, :L].astype(np.float64) - ref[r, :L])
        assert (err <= bound + 1e-30).all(), f"row {r}: worst err / bound {float((err / bound).max()):.3f}"
        worst_bound = max(worst_bound, float((err / bound).max()))
        worst_plain = max(worst_plain, float((err / np.maximum(mag[r, :L], 1e-30)).max()))
    print(f"[edge] extreme q: worst error / bound {worst_bound:.3f}, worst error / magnitude {worst_plain:.2e}")
