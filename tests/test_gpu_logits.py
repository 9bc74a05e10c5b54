"""GPU parity of the MQA indexer logits (decode and prefill) against the oracle:
logits within the documented tolerance (tests/gpu_util.py), the 16-token nonzero mask and the
fused top-k pass-1 histogram bit-exact."""
import numpy as np
import pytest
import torch

import hcu_ops
from hcu_ops import _C
import workloads as wl
from oracle import indexer as O
from oracle.topk_c import topk_radix

from gpu_util import check_logits, check_mask, kv_np, oracle_decode, oracle_q

pytestmark = pytest.mark.gpu


def _run_decode(case, gpu, pctas=0, rpc=None, hist=False):
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens = case.context_lens.to(gpu)
    lg, mask = hcu_ops.mqa_logits(q8.unsqueeze(1), case.kv.to(gpu), w, lens, case.block_table.to(gpu), case.width,
                                  case.group, hist_lens=lens if hist else None, persistent_ctas=pctas,
                                  rows_per_cta=rpc)
    return q8, w, lg, mask


def _check_decode(case, lg, mask):
    q8, w = oracle_q(case)
    ref, mag, dmag, ref_mask = oracle_decode(case, q8, w)
    got_mask = mask.cpu().numpy()
    got = lg.cpu().numpy()
    check_mask(got_mask, got, ref, mag, case.context_lens.numpy(), "nonzero mask")
    for r in range(case.rows):
        L = int(case.context_lens[r])
        check_logits(got[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"row {r}")


@pytest.mark.parametrize("heads", [64, 32])
@pytest.mark.parametrize("group,lens,rpc", [
    (1, [4096], 1),
    (1, [5000, 130, 64, 65, 2049], 1),
    (2, [3000, 7000, 1], 1),
    (2, [3000, 7000, 1], 2),
    (6, [2500, 900], 1),
    (6, [2500, 900], 2),
    (6, [2500, 900], 3),
    (4, [1000, 1200], 4),
    (8, [3000, 70], 8),
])
def test_decode_logits(gpu, heads, group, lens, rpc):
    case = wl.decode_case(100 + len(lens) + group, lens, group=group, heads=heads,
                          bt_pages=max((L + group + 63) // 64 for L in lens) + 3)
    _, _, lg, mask = _run_decode(case, gpu, rpc=rpc)
    _check_decode(case, lg, mask)


@pytest.mark.parametrize("n_req,group", [(64, 1), (65, 1), (130, 1), (33, 2), (64, 2)])
def test_decode_logits_group_counts(gpu, n_req, group):
    """Up to 64 request groups every wave assigns its CTA's pages itself; past 64 the CTA does it
    with block scans: both sides of the boundary, with empty and one-token rows among them."""
    g = torch.Generator().manual_seed(n_req + group)
    lens = torch.randint(1, 2600, (n_req,), generator=g)
    lens[::7] = 0
    lens[3::11] = 1
    case = wl.decode_case(300 + n_req, lens.tolist(), group=group, heads=64, bt_pages=(2600 + group + 63) // 64 + 1)
    _, _, lg, mask = _run_decode(case, gpu, rpc=group)
    _check_decode(case, lg, mask)


@pytest.mark.parametrize("pctas", [1, 3, 64, 1000])
def test_decode_logits_cta_split(gpu, pctas):
    case = wl.decode_case(7, [9000, 4000], group=2, heads=64)
    _, _, lg, mask = _run_decode(case, gpu, pctas=pctas, rpc=2)
    _check_decode(case, lg, mask)


def test_decode_logits_sparse_and_negative_modes(gpu):
    """The reference's 'sparse' and 'neg' modes (test_mqa_hist.py:31-49): all-negative dot
    products give exact zeros (mask bit clear), all-negative weights give negative logits."""
    case = wl.decode_case(9, [3000, 2500], group=1, heads=64)
    kvf = case.kv.view(case.kv.shape[0], -1).clone()
    codes = kvf[:, :8192].contiguous().view(-1, 128)
    vals = codes.view(torch.float8_e4m3fn).float().abs()
    g = torch.Generator().manual_seed(1)
    pos = torch.rand(codes.shape[0], 1, generator=g) < 0.05
    signed = torch.where(pos, vals, -vals).to(torch.float8_e4m3fn).view(torch.uint8)
    kvf[:, :8192] = signed.view(kvf.shape[0], 8192)
    case.kv = kvf.view(case.kv.shape)
    case.q = case.q.abs()
    case.w = case.w.abs()
    _, _, lg, mask = _run_decode(case, gpu)
    _check_decode(case, lg, mask)
    bits = O.unpack_mask(mask.cpu().numpy(), case.width)
    assert 0 < bits.sum() < 0.2 * case.context_lens.sum()
    case.w = -case.w
    _, _, lg, mask = _run_decode(case, gpu)
    _check_decode(case, lg, mask)


@pytest.mark.parametrize("group,lens,rpc", [(1, [9000, 5000, 1500, 40000], 1), (2, [20000, 3000], 2),
                                            (2, [65536, 64000, 700, 0, 3000, 2049], 1),
                                            (6, [30000, 2100], 3)])
def test_decode_fused_histogram_reference_contract(gpu, group, lens, rpc):
    """_C.mqa_logits_hist called with the reference's ten arguments (hcu_ops/csrc/bind.cpp:36-44)
    and hist_lens leaves pass 1 in zws, checked as the reference's own test does
    (hcu_ops/tests/test_mqa_hist.py:166-174, ok_h): ghist1 and (positives, zeros) equal the
    closed form of test_mqa_hist.py:109-124 on the kernel's own logits, the second block is all
    zero; then _C.sparse_mask_topk_transform_split_pre with the reference's eight arguments
    consumes it and selects the oracle's set."""
    from hcu_ops import _C
    case = wl.decode_case(13, lens, group=group, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens_d = case.context_lens.to(gpu)
    B, W = case.rows, case.width
    lg, mask, zws = _C.mqa_logits_hist(q8.unsqueeze(1), case.kv.to(gpu), w, lens_d, case.block_table.to(gpu), W,
                                       group, 0, rpc, lens_d)
    z = zws.cpu().numpy()
    ref = O.pass1_hist(lg.cpu().numpy(), mask.cpu().numpy(), case.context_lens.numpy(), W)
    assert np.array_equal(z[:B * 4096], ref[:B * 4096]), "ghist1 differs"
    assert np.array_equal(z[2 * B * 4096:], ref[2 * B * 4096:]), "(positives, zeros) differ"
    assert not z[B * 4096:2 * B * 4096].any(), "second histogram block not all zero"
    _check_decode(case, lg, mask)
    pt = case.page_table_1()
    cu = torch.arange(B + 1, dtype=torch.int32, device=gpu)
    got = _C.sparse_mask_topk_transform_split_pre(lg, mask, lens_d, pt.to(gpu), cu, 2048, 8, zws)
    want = topk_radix(lg.cpu().numpy(), mask.cpu().numpy(), case.context_lens.numpy(), pt.numpy(), W)
    assert np.array_equal(got.cpu().numpy(), want)


def test_decode_logits_reference_arguments_reject_fused_r4(gpu):
    """The fused pass 1 keeps 8 KB of LDS counters per row: rows_per_cta > 3 with hist_lens is
    rejected unless fuse_pass1=False is passed (then only the counters are zeroed)."""
    from hcu_ops import _C
    case = wl.decode_case(15, [3000, 2500], group=4, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    lens_d = case.context_lens.to(gpu)
    args = (q8.unsqueeze(1), case.kv.to(gpu), w, lens_d, case.block_table.to(gpu), case.width, 4, 0, 4, lens_d)
    with pytest.raises(RuntimeError, match="rows_per_cta <= 3"):
        _C.mqa_logits_hist(*args)
    lg, mask, zws = _C.mqa_logits_hist(*args, fuse_pass1=False)
    _check_decode(case, lg, mask)


@pytest.mark.parametrize("group,lens", [(1, [9000, 100, 40000]), (2, [20000, 3000, 0, 0])])
def test_decode_topk_counters_zeroed(gpu, group, lens):
    """Without the fused pass 1 the logits call (C ABI, hist_ws given, fuse_pass1 = 0) zeroes
    exactly the paired top-k's per-row counters (words 0..2 of each row of the second block)
    and writes nothing else of the workspace."""
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(hcu_ops.__file__), "libdsa_indexer.so"))
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.dsa_mqa_logits_decode
    f.argtypes = [P, P, I, I64, I, P, I64, P, P, I64, I64, P, I64, P, I64, I, I, P, P, I, P]
    lib.dsa_last_error.restype = ctypes.c_char_p
    case = wl.decode_case(14, lens, group=group, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    kv, ctx, bt = case.kv.to(gpu), case.context_lens.to(gpu), case.block_table.to(gpu)
    B, W = case.rows, case.width
    lg = torch.empty(B, W, device=gpu)
    mask = torch.empty(B, W // 16, dtype=torch.int16, device=gpu)
    ws = torch.full((B * (2 * 4096 + 2),), -1, dtype=torch.int32, device=gpu)
    st = f(q8.data_ptr(), w.data_ptr(), 64, B, group, kv.data_ptr(), kv.stride(0), ctx.data_ptr(), bt.data_ptr(),
           bt.stride(0), bt.shape[1], lg.data_ptr(), lg.stride(0), mask.data_ptr(), mask.stride(0),
           1 if group == 1 else 2, 0, ctx.data_ptr(), ws.data_ptr(), 0, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.dsa_last_error()
    zws = ws.cpu().numpy()
    ctr = zws[B * 4096:2 * B * 4096].reshape(B, 4096)
    assert not ctr[:, :3].any(), "top-k counters not zeroed"
    assert (ctr[:, 3:] == -1).all() and (zws[:B * 4096] == -1).all() and (zws[2 * B * 4096:] == -1).all()
    _check_decode(case, lg, mask)


# row counts cover every launch split of the prefill entry: groups of 8, then of 4 and 1-3 rows
@pytest.mark.parametrize("heads,n_q,prefix", [(64, 40, 3000), (32, 9, 130), (64, 17, 0), (64, 15, 700),
                                              (32, 6, 4100), (64, 3, 64)])
def test_prefill_logits(gpu, heads, n_q, prefix):
    case = wl.prefill_case(21 + n_q, n_q, prefix, heads=heads)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    width = case.n_keys + 5
    bt = torch.cat([case.block_table, torch.zeros(1, dtype=torch.int32)])  # capacity for width
    lg = hcu_ops.mqa_logits_prefill(q8, w, case.kv.to(gpu), bt.to(gpu), case.lens.to(gpu), width)
    rq8, rw = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    ref, mag, dmag = O.mqa_logits_prefill(rq8, rw, kv_np(case.kv), bt.numpy(), case.lens.numpy(), width)
    got = lg.cpu().numpy()
    for r in range(case.rows):
        L = int(case.lens[r])
        check_logits(got[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"row {r}")


def test_prefill_writes_only_below_len(gpu):
    """Through the C ABI into a NaN-filled buffer wider than `width`: row r gets exactly the
    entries t < min(len[r], width); lengths include 0, negative and past `width`."""
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(hcu_ops.__file__), "libdsa_indexer.so"))
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.dsa_mqa_logits_prefill
    f.argtypes = [P, P, I, I64, P, I64, P, I64, P, P, I64, I64, P]
    lib.dsa_last_error.restype = ctypes.c_char_p
    case = wl.prefill_case(5, 13, 900, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    width = case.n_keys - 37
    lens = case.lens.clone()
    lens[0], lens[5], lens[12] = 0, -3, width + 500
    kv, bt, lens_d = case.kv.to(gpu), case.block_table.to(gpu), lens.to(gpu)
    out = torch.full((case.rows, width + 19), float("nan"), device=gpu)
    st = f(q8.data_ptr(), w.data_ptr(), 64, case.rows, kv.data_ptr(), kv.stride(0), bt.data_ptr(), bt.numel(),
           lens_d.data_ptr(), out.data_ptr(), out.stride(0), width, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.dsa_last_error()
    got = out.cpu().numpy()
    ref = hcu_ops.mqa_logits_prefill(q8, w, kv, bt, lens_d, width).cpu().numpy()
    for r in range(case.rows):
        L = max(0, min(int(lens[r]), width))
        assert not np.isnan(got[r, :L]).any(), f"row {r}: entries below len not written"
        assert np.isnan(got[r, L:]).all(), f"row {r}: entries at or past min(len, width) written"
        assert np.array_equal(got[r, :L], ref[r, :L]), f"row {r}: differs from the torch binding"


def test_decode_wide_block_nontemporal_stores(gpu):
    """A logits block above 16 MB (64 rows x 70,400-token capacity, 18 MB) takes the kernel's
    nontemporal-store path: same bits as the same rows in a narrow block (cached stores), and the
    oracle's values; entries past each row's length stay untouched."""
    lens = [900 + 37 * i for i in range(32)]
    wide = wl.decode_case(41, lens, group=2, heads=64, bt_pages=1100)
    narrow = wl.decode_case(41, lens, group=2, heads=64)
    assert wide.rows * wide.width * 4 > (16 << 20) and narrow.rows * narrow.width * 4 < (16 << 20)
    _, _, lg_w, mask_w = _run_decode(wide, gpu, rpc=2)
    _, _, lg_n, mask_n = _run_decode(narrow, gpu, rpc=2)
    keep = torch.arange(narrow.width, device=gpu)[None, :] < narrow.context_lens.to(gpu)[:, None]
    assert torch.equal(lg_w[:, :narrow.width][keep].view(torch.int32), lg_n[keep].view(torch.int32))
    assert torch.equal(mask_w[:, :narrow.width // 16], mask_n)
    assert not mask_w[:, narrow.width // 16 + 1:].any()
    _check_decode(wide, lg_w, mask_w)


def test_prefill_wide_block_nontemporal_stores(gpu):
    """Prefill into a 64-row x 70,016-wide block (17.9 MB, nontemporal stores) with short causal
    rows: the oracle's values below each row's length, nothing written past it."""
    case = wl.prefill_case(43, 64, 1000, heads=64)
    q8, w = hcu_ops.quant_q_fp8(case.q.to(gpu), case.w.to(gpu))
    width = 70016
    assert case.rows * width * 4 > (16 << 20)
    bt = torch.cat([case.block_table, torch.zeros(width // 64 - case.block_table.numel(), dtype=torch.int32)])
    out = torch.full((case.rows, width), float("nan"), device=gpu)
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(hcu_ops.__file__), "libdsa_indexer.so"))
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.dsa_mqa_logits_prefill
    f.argtypes = [P, P, I, I64, P, I64, P, I64, P, P, I64, I64, P]
    lib.dsa_last_error.restype = ctypes.c_char_p
    kv, btd, lens = case.kv.to(gpu), bt.to(gpu), case.lens.to(gpu)
    st = f(q8.data_ptr(), w.data_ptr(), 64, case.rows, kv.data_ptr(), kv.stride(0), btd.data_ptr(), btd.numel(),
           lens.data_ptr(), out.data_ptr(), out.stride(0), width, torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.dsa_last_error()
    rq8, rw = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    ref, mag, dmag = O.mqa_logits_prefill(rq8, rw, kv_np(case.kv), bt.numpy(), case.lens.numpy(), case.n_keys)
    got = out.cpu().numpy()
    for r in range(case.rows):
        L = int(case.lens[r])
        check_logits(got[r, :L], ref[r, :L], mag[r, :L], dmag[r, :L], f"row {r}")
        assert np.isnan(got[r, L:]).all(), f"row {r}: entries past len written"


def test_mfma_probe_runs_on_random_fp8(gpu):
    """The MFMA throughput probe the bench reports beside the published fp8 peak: every VALU count
    per MFMA runs, keeps finite results and reads both clocks."""
    g = torch.Generator().manual_seed(5)
    codes = torch.randint(0, 254, (4 * 16384,), generator=g, dtype=torch.int32)
    codes = (codes + (codes >= 0x7F).int()).to(torch.uint8)
    ops = codes.view(torch.int32).to(gpu)
    for epi in (0, 1, 4, 8, 16):
        sink, clocks = _C.mfma_fp8_probe(ops, 64, 20, epi)
        torch.cuda.synchronize()
        assert torch.isfinite(sink).all(), f"epilogue={epi}"
        c = clocks.cpu().tolist()
        assert c[0] > 0 and c[1] > 0, f"epilogue={epi}: clocks {c}"
