"""The top-k output read by a sparse-MLA consumer (the [rows, 2048] int32 slot-id wire format of
tests/wire_format.py), on the decode step and on the prefill indexer.

Each product output keeps the wire format (pads only at the end, every id the slot of a token
below the row's length, no repeats, short rows in token order, long rows in at most two
ascending runs), equals the oracle's selection in the reference order, and is the same on a
second call.  A consumer then runs on it: the MLA K of the listed slots is dequantised on the
GPU (pads included, which dequantise to zero and are masked out) and a sparse MLA decode
attention (16 heads, 576-dim scores, 512-dim values) is computed in float32 on the GPU in list
order; it must match the float64 consumer on the oracle's slot list and the oracle's dequant to
within 2e-5 of the output's scale."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix
from wire_format import TOPK, bf16_bits_to_f32, slot_table, sparse_mla_decode, wire_format_problems

pytestmark = pytest.mark.gpu

H_MLA = 16
SM_SCALE = 576 ** -0.5


def _mla_pool(n_slots, seed):
    return wl.mla_dequant_case(seed, 1, pool=n_slots).cache


def _consume(gpu, pool, ids, q_mla):
    """float32 [rows, H, 512] from the GPU: dequant the listed slots, attention over the valid ones."""
    rows = ids.shape[0]
    kv = hcu_ops.dequantize_k_cache_paged(pool, ids.reshape(-1)).view(rows, TOPK, 576).float()
    valid = ids >= 0
    s = torch.matmul(q_mla, kv.transpose(1, 2).contiguous()) * SM_SCALE  # [rows, H, 2048]
    s = s.masked_fill(~valid[:, None, :], float("-inf"))
    p = torch.softmax(s, dim=2)
    p = torch.nan_to_num(p, nan=0.0)  # rows with no valid id
    return torch.matmul(p, kv[:, :, :512].contiguous())


def _check_consumer(gpu, pool, got_ids, want_ids, q_mla, what):
    o = _consume(gpu, pool, got_ids, q_mla).cpu().numpy()
    pool_np = pool.view(pool.shape[0], -1).cpu().numpy()
    qn = q_mla.cpu().numpy()
    worst = 0.0
    for r in range(want_ids.shape[0]):
        ids = want_ids[r][want_ids[r] >= 0]
        if ids.size == 0:
            assert np.abs(o[r]).max() == 0.0, f"{what} row {r}: output of an empty row"
            continue
        k = bf16_bits_to_f32(O.dequant_mla(pool_np, ids))
        ref, _ = sparse_mla_decode(qn[r], k, SM_SCALE)
        err = np.abs(o[r] - ref).max() / max(np.abs(ref).max(), 1e-30)
        worst = max(worst, float(err))
    assert worst <= 2e-5, f"{what}: consumer output off by {worst:.2e} of its scale"
    return worst


def test_decode_step_output_feeds_sparse_mla(gpu):
    case = wl.decode_case(41, [0, 700, 2047, 2048, 2049, 5000, 33000, 64000], group=2, bt_pages=1002)
    g = lambda t: t.to(gpu)
    lens = g(case.context_lens)
    pt = case.page_table_1()
    cu = torch.arange(case.rows + 1, dtype=torch.int32, device=gpu)

    def step():
        q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
        lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), g(case.kv), w, lens, g(case.block_table), case.width,
                                      case.group, hist_lens=lens)
        return lg, mask, hcu_ops.sparse_mask_topk_transform(lg, mask, lens, g(pt), cu)

    lg, mask, out = step()
    ids = out.cpu().numpy()
    bt = case.block_table.numpy()
    assert out.dtype == torch.int32 and out.is_contiguous() and tuple(out.shape) == (case.rows, TOPK)
    problems = wire_format_problems(ids, case.context_lens.numpy(), lambda r: slot_table(bt[r], case.width))
    assert problems == [], problems[:5]
    want = topk_radix(lg.cpu().numpy(), mask.cpu().numpy(), case.context_lens.numpy(), pt.numpy(), case.width)
    assert np.array_equal(ids, want), "decode: top-k rows differ from the oracle (set or order)"
    _, _, again = step()
    assert torch.equal(again, out), "decode: a second call changed the rows"

    n_slots = case.kv.shape[0] * 64
    pool = g(_mla_pool(n_slots, 41))
    q_mla = torch.randn(case.rows, H_MLA, 576, generator=torch.Generator().manual_seed(42)).to(gpu)
    q_mla = q_mla.to(torch.bfloat16).float()
    worst = _check_consumer(gpu, pool, out, want, q_mla, "decode")
    print(f"[consumer] decode: {case.rows} rows keep the wire format; consumer error {worst:.2e}", flush=True)


def test_prefill_indexer_output_feeds_sparse_mla(gpu):
    case = wl.prefill_case(43, 96, 3000)
    g = lambda t: t.to(gpu)
    q8, w = hcu_ops.quant_q_fp8(g(case.q), g(case.w))
    kv, bt, lens = g(case.kv), g(case.block_table), g(case.lens)
    out = hcu_ops.prefill_indexer(q8, w, kv, bt, lens, case.n_keys, max_slab_rows=40)  # slots from bt
    ids = out.cpu().numpy()
    slots = slot_table(case.block_table.numpy(), case.n_keys)
    problems = wire_format_problems(ids, case.lens.numpy(), lambda r: slots)
    assert problems == [], problems[:5]
    lg = hcu_ops.mqa_logits_prefill(q8, w, kv, bt, lens, case.n_keys)
    want = topk_radix(lg.cpu().numpy(), None, case.lens.numpy(), slots[None, :].astype(np.int32), case.n_keys,
                      cu_seqlens_q=np.array([0, case.rows], dtype=np.int32))
    assert np.array_equal(ids, want), "prefill: top-k rows differ from the oracle (set or order)"

    pool = g(_mla_pool(case.kv.shape[0] * 64, 43))
    q_mla = torch.randn(case.rows, H_MLA, 576, generator=torch.Generator().manual_seed(44)).to(torch.bfloat16)
    worst = _check_consumer(gpu, pool, out, want, q_mla.float().to(gpu), "prefill")
    print(f"[consumer] prefill: {case.rows} rows keep the wire format; consumer error {worst:.2e}", flush=True)
