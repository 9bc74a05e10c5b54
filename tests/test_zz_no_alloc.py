"""dsa_topk_transform_noalloc (the top-k entry point that allocates nothing: its split workspace
is a built-in device array) against dsa_topk_transform with a caller workspace, through the C
ABI: its first call in the process made inside a hipGraph capture and replayed with new scores;
then two eager calls in a row, the second with a smaller input; every call taking the split path
that uses the workspace, each equal to the existing entry point's rows and to the oracle's."""
import ctypes
import os

import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle.topk_c import topk_radix

pytestmark = pytest.mark.gpu

P, I64, I, SZ = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t


def _lib():
    lib = ctypes.CDLL(os.path.join(os.path.dirname(hcu_ops.__file__), "libdsa_indexer.so"))
    lib.dsa_topk_transform.argtypes = [P, I64, I64, P, I64, P, I64, P, I64, I64, P, I64, I, I, P, SZ, P, P]
    lib.dsa_topk_transform_noalloc.argtypes = [P, I64, I64, P, I64, P, I64, P, I64, I64, P, I64, I, I, P, P]
    lib.dsa_topk_workspace_bytes.argtypes = [I64, I64, I, I]
    lib.dsa_topk_workspace_bytes.restype = SZ
    lib.dsa_topk_noalloc_max_bytes.restype = SZ
    lib.dsa_last_error.restype = ctypes.c_char_p
    return lib


def test_topk_noalloc_first_call_under_capture(gpu):
    """The process's first no-alloc call (the one that looks up the device array's address) is made
    inside a hipGraph capture; the graph is then replayed with new scores copied into its static
    inputs, each replay equal to the workspace entry point's eager rows and to the oracle's."""
    lib = _lib()
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    B, L = 12, 40000
    W = L + 64
    assert 0 < lib.dsa_topk_workspace_bytes(B, W, 8, n_cu) <= lib.dsa_topk_noalloc_max_bytes()
    xg = torch.zeros(B, W, device=gpu)
    mg = torch.zeros(B, (W + 15) // 16, dtype=torch.int16, device=gpu)
    lg = torch.zeros(B, dtype=torch.int32, device=gpu)
    pg = torch.zeros(B, W, dtype=torch.int32, device=gpu)
    out_na = torch.full((B, 2048), -7, dtype=torch.int32, device=gpu)
    args = (xg.data_ptr(), xg.stride(0), W, mg.data_ptr(), mg.stride(0), lg.data_ptr(), B, pg.data_ptr(),
            pg.stride(0), W, None, B, 8, n_cu)
    g = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.graph(g, stream=side):
        st = lib.dsa_topk_transform_noalloc(*args, out_na.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert st == 0, lib.dsa_last_error()
    torch.cuda.synchronize()
    need = lib.dsa_topk_workspace_bytes(B, W, 8, n_cu)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    out_ws = torch.empty(B, 2048, dtype=torch.int32, device=gpu)
    stream = torch.cuda.current_stream().cuda_stream
    for seed, dist in ((3, "relu_sum"), (4, "mixed"), (5, "ties"), (6, "relu_sum")):
        x, mask, lengths, pt = wl.topk_scores(B, L, dist, W=W, ragged=True, seed=seed)
        xg.copy_(x)
        mg.copy_(mask)
        lg.copy_(lengths)
        pg.copy_(pt)
        out_na.fill_(-7)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert lib.dsa_topk_transform(*args, ws.data_ptr(), need, out_ws.data_ptr(), stream) == 0, \
            lib.dsa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), f"replay {dist} seed={seed}: rows differ from the workspace entry's"
        ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), W)
        assert np.array_equal(out_na.cpu().numpy(), ref), f"replay {dist} seed={seed}: rows differ from the oracle"


def test_topk_noalloc_matches_workspace_entry(gpu):
    lib = _lib()
    n_cu = torch.cuda.get_device_properties(0).multi_processor_count
    stream = torch.cuda.current_stream().cuda_stream
    for B, L in [(16, 65536), (6, 40000)]:
        W = L + 64
        x, mask, lengths, pt = wl.topk_scores(B, L, "relu_sum", W=W, ragged=True, seed=B)
        need = lib.dsa_topk_workspace_bytes(B, W, 8, n_cu)
        assert 0 < need <= lib.dsa_topk_noalloc_max_bytes(), "the case must take the split path"
        xg, mg, lg, pg = (t.to(gpu) for t in (x, mask, lengths, pt))
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        out_ws = torch.full((B, 2048), -7, dtype=torch.int32, device=gpu)
        out_na = torch.full((B, 2048), -7, dtype=torch.int32, device=gpu)
        args = (xg.data_ptr(), xg.stride(0), W, mg.data_ptr(), mg.stride(0), lg.data_ptr(), B, pg.data_ptr(),
                pg.stride(0), W, None, B, 8, n_cu)
        assert lib.dsa_topk_transform(*args, ws.data_ptr(), need, out_ws.data_ptr(), stream) == 0, \
            lib.dsa_last_error()
        assert lib.dsa_topk_transform_noalloc(*args, out_na.data_ptr(), stream) == 0, lib.dsa_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), f"B={B} L={L}: no-alloc rows differ from the workspace entry's"
        ref = topk_radix(x.numpy(), mask.numpy(), lengths.numpy(), pt.numpy(), W)
        assert np.array_equal(out_na.cpu().numpy(), ref), f"B={B} L={L}: rows differ from the oracle"
