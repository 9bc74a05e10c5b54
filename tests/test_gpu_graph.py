"""The decode step and the prefill indexer under hipGraph capture: captured once on static buffers, replayed with new
inputs copied into them (new queries, weights, K pages, lengths and block tables of the same
shapes), each replay bit-identical to an eager run of the same inputs (logits, mask and the
top-k rows, their order included) and identical to the oracle's selection.  The reference
captures its ops in graphs the same way (hcu_ops/tests/test_mqa_hist.py:78-99,
hcu_ops/tests/topk_lib.py:54-67) and promises a layout that does not change across replays
(hcu_ops/csrc/sparse_mask_topk.cu:4-7)."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle.topk_c import topk_radix

pytestmark = pytest.mark.gpu

N_REQ, GROUP, CAP_PAGES = 8, 2, 1026  # 8 requests x 2 MTP rows, capacity 65,664 tokens


def _case(seed):
    g = torch.Generator().manual_seed(seed)
    L = torch.randint(2048, 65536, (N_REQ,), generator=g).tolist()
    L[seed % N_REQ] = 1500 + seed  # a row below 2048 tokens
    return wl.decode_case(seed, L, group=GROUP, heads=64, bt_pages=CAP_PAGES)


class Step:
    """Static input / output buffers and the decode step over them."""

    def __init__(self, gpu, max_pages):
        B, W = N_REQ * GROUP, CAP_PAGES * 64
        self.q = torch.zeros(B, 64, 128, dtype=torch.bfloat16, device=gpu)
        self.w = torch.zeros(B, 64, device=gpu)
        self.kv = torch.zeros(max_pages, 64, 1, 132, dtype=torch.uint8, device=gpu)
        self.lens = torch.zeros(B, dtype=torch.int32, device=gpu)
        self.bt = torch.zeros(B, CAP_PAGES, dtype=torch.int32, device=gpu)
        self.pt = torch.zeros(B, W, dtype=torch.int32, device=gpu)
        self.cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
        self.width = W

    def load(self, case):
        self.q.copy_(case.q)
        self.w.copy_(case.w)
        self.kv.zero_()
        self.kv[:case.kv.shape[0]].copy_(case.kv)
        self.lens.copy_(case.context_lens)
        self.bt.copy_(case.block_table)
        self.pt.copy_(case.page_table_1())

    def __call__(self):
        q8, w = hcu_ops.quant_q_fp8(self.q, self.w)
        logits, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), self.kv, w, self.lens, self.bt, self.width, GROUP,
                                          hist_lens=self.lens)
        out = hcu_ops.sparse_mask_topk_transform(logits, mask, self.lens, self.pt, self.cu)
        return logits, mask, out


def test_decode_step_graph_replay(gpu):
    cases = [_case(s) for s in (31, 32, 33, 34)]
    step = Step(gpu, max(c.kv.shape[0] for c in cases))
    step.load(cases[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_logits, g_mask, g_out = step()
    torch.cuda.synchronize()
    for i, case in enumerate(cases[1:] + cases[:1]):
        step.load(case)
        e_logits, e_mask, e_out = step()  # eager run on the same inputs
        e_logits, e_mask, e_out = e_logits.clone(), e_mask.clone(), e_out.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        lens = case.context_lens.to(gpu)
        keep = torch.arange(step.width, device=gpu)[None, :] < lens[:, None]
        assert torch.equal(g_logits[keep].view(torch.int32), e_logits[keep].view(torch.int32)), f"replay {i}: logits"
        assert torch.equal(g_mask, e_mask), f"replay {i}: mask"
        assert torch.equal(g_out, e_out), f"replay {i}: top-k rows"
        want = topk_radix(g_logits.cpu().numpy(), g_mask.cpu().numpy(), case.context_lens.numpy(),
                          case.page_table_1().numpy(), step.width)
        assert np.array_equal(g_out.cpu().numpy(), want), f"replay {i}: top-k rows differ from the oracle"


P_ROWS, P_PREFIX, P_SLAB = 72, 5000, 24  # three 24-row slabs per replay


def test_prefill_indexer_graph_replay(gpu):
    """The prefill indexer (quant, then per slab: logits + top-2048) captured once and replayed
    with new queries, weights and K of the same shapes: every replay bit-identical to an eager
    run and to the oracle's selection (set and order)."""
    cases = [wl.prefill_case(s, P_ROWS, P_PREFIX) for s in (51, 52, 53)]
    n_keys = cases[0].n_keys
    c0 = cases[0]
    q = torch.zeros_like(c0.q, device=gpu)
    w = torch.zeros_like(c0.w, device=gpu)
    kv = torch.zeros_like(c0.kv, device=gpu)
    bt = c0.block_table.to(gpu)  # one page order for every case: the kv contents change
    lens = c0.lens.to(gpu)
    out = torch.empty(P_ROWS, 2048, dtype=torch.int32, device=gpu)

    def step():
        q8, w8 = hcu_ops.quant_q_fp8(q, w)
        return hcu_ops.prefill_indexer(q8, w8, kv, bt, lens, n_keys, max_slab_rows=P_SLAB, out=out), q8, w8

    def load(case):
        q.copy_(case.q)
        w.copy_(case.w)
        kv.copy_(case.kv)

    load(cases[0])
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step()
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out, g_q8, g_w8 = step()
    torch.cuda.synchronize()
    slots = (c0.block_table.long()[torch.arange(n_keys) // 64] * 64 + torch.arange(n_keys) % 64).to(torch.int32)
    for i, case in enumerate(cases[1:] + cases[:1]):
        load(case)
        e_out = step()[0].clone()  # eager run on the same inputs (writes `out` too)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, e_out), f"replay {i}: top-k rows differ from the eager run"
        lg = hcu_ops.mqa_logits_prefill(g_q8, g_w8, kv, bt, lens, n_keys)
        want = topk_radix(lg.cpu().numpy(), None, case.lens.numpy(), slots[None, :].numpy(), n_keys,
                          cu_seqlens_q=np.array([0, P_ROWS], dtype=np.int32))
        assert np.array_equal(g_out.cpu().numpy(), want), f"replay {i}: top-k rows differ from the oracle"
