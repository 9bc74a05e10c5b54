"""The HIP path against the known-answer fixtures of tests/golden/ (see tests/golden/make_golden.py):
top-k rows bit-exact, order included, on the one-CTA-per-row and split kernels; q quantisation,
the K-cache writer and both dequants bit-exact; the mask words exact and the logits within 1e-3
of each token's magnitude A_t = s_t sum_h |w_h| relu(acc_h)."""
import os

import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _load(name):
    return np.load(os.path.join(GOLDEN, name))


def test_golden_topk(gpu):
    d = _load("topk_small.npz")
    x, m, L, pt = (torch.from_numpy(d[k]).to(gpu) for k in ("score", "mask", "lengths", "page_table"))
    cu = torch.arange(x.shape[0] + 1, dtype=torch.int32, device=gpu)
    got = hcu_ops.sparse_mask_topk_transform(x, m, L, pt, cu)
    assert np.array_equal(got.cpu().numpy(), d["expected"])
    for splits in (2, 8):
        got = _C.sparse_mask_topk_transform_split(x, m, L, pt, cu, 2048, splits)
        assert np.array_equal(got.cpu().numpy(), d["expected"]), f"splits={splits}"
    got = _C.sparse_mask_topk_transform(x, m, L, pt, cu, 2048)
    assert np.array_equal(got.cpu().numpy(), d["expected"])


def test_golden_quant_logits_dequant(gpu):
    d = _load("indexer_small.npz")
    q = torch.from_numpy(d["q_bf16"].view(np.int16)).view(torch.bfloat16).to(gpu)
    w = torch.from_numpy(d["w"]).to(gpu)
    q8, w_eff = hcu_ops.quant_q_fp8(q, w)
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), d["q8"])
    assert np.array_equal(w_eff.cpu().numpy().view(np.uint32), d["w_eff"].view(np.uint32))

    kv = torch.from_numpy(d["kv_cache"]).view(-1, 64, 1, 132).to(gpu)
    lens = torch.from_numpy(d["context_lens"]).to(gpu)
    bt = torch.from_numpy(d["block_table"]).to(gpu)
    logits, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), kv, w_eff, lens, bt, int(d["width"]), int(d["group"]))
    assert np.array_equal(mask.cpu().numpy(), d["mask"])
    exact, mag = d["logits"], d["magnitude"]
    written = ~np.isnan(exact)
    err = np.abs(logits.cpu().numpy().astype(np.float64)[written] - exact[written])
    assert (err <= 1e-3 * mag[written]).all(), float((err / np.maximum(mag[written], 1e-300)).max())

    deq = hcu_ops.dequant_k_paged(kv, torch.from_numpy(d["slots"]).to(gpu))
    assert np.array_equal(deq.view(torch.int16).cpu().numpy().view(np.uint16), d["dequant_bf16"])


def test_golden_k_writer_and_mla(gpu):
    d = _load("indexer_small.npz")
    k = torch.from_numpy(d["k_bf16"].view(np.int16)).view(torch.bfloat16).to(gpu)
    kv = torch.zeros(2, 64, 1, 132, dtype=torch.uint8, device=gpu)
    hcu_ops.store_k_cache(k, torch.from_numpy(d["k_slots"]).to(gpu), kv)
    assert np.array_equal(kv.view(2, -1).cpu().numpy(), d["k_cache_written"])
    m = _load("mla_small.npz")
    cache = torch.from_numpy(m["cache"]).view(torch.float8_e4m3fn).view(-1, 1, 656).to(gpu)
    got = hcu_ops.dequantize_k_cache_paged(cache, torch.from_numpy(m["slots"]).to(gpu))
    n = m["slots"].shape[0]
    assert np.array_equal(got.view(n, 576).view(torch.int16).cpu().numpy().view(np.uint16), m["expected"])
