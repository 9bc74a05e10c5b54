"""CPU checks of the drop-in boundary: the C-ABI library loads and exports every entry point
include/dsa_indexer.h declares; host-side contract checks reject bad arguments without touching
a GPU; the torch bind rejects CPU tensors and bad shapes with the reference's messages."""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "dsa_indexer.h")
LIB = os.path.join(ROOT, "sglang0.5.18-opt_amd", "hcu_ops", "libdsa_indexer.so")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(dsa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    assert os.path.exists(LIB), "build first: python sglang0.5.18-opt_amd/build.py"
    return ctypes.CDLL(LIB)


def test_header_declares_the_path():
    names = declared_functions()
    for n in ["dsa_dequant_k_paged", "dsa_gather_k_paged", "dsa_dequant_mla_paged", "dsa_quant_q_fp8",
              "dsa_store_k_cache", "dsa_mqa_logits_decode", "dsa_mqa_logits_prefill", "dsa_topk_workspace_bytes",
              "dsa_topk_transform", "dsa_topk_transform_pre", "dsa_topk_split_count", "dsa_prefill_slab_rows",
              "dsa_prefill_indexer_workspace_bytes", "dsa_prefill_indexer", "dsa_topk_transform_noalloc",
              "dsa_topk_noalloc_max_bytes", "dsa_last_error", "dsa_device_cu_count", "dsa_mfma_fp8_probe"]:
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/dsa_indexer.h but not exported"


def test_mfma_probe_rejects_bad_arguments_on_the_host(lib):
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.dsa_mfma_fp8_probe
    f.argtypes = [P, I64, P, P, I, I, I, P]
    assert f(P(16), 16383, P(16), P(16), 8, 10, 0, None) == 1
    assert "16384" in _err(lib)
    assert f(None, 16384, P(16), P(16), 8, 10, 0, None) == 1
    assert f(P(16), 16384, P(16), P(16), 0, 10, 0, None) == 1
    assert f(P(16), 16384, P(16), P(16), 8, 10, 3, None) == 1  # 3 VALU operations per MFMA: not a probe mode
    assert "epilogue" in _err(lib)


def _err(lib):
    lib.dsa_last_error.restype = ctypes.c_char_p
    return lib.dsa_last_error().decode()


def test_contract_violations_are_rejected_on_the_host(lib):
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    f = lib.dsa_dequant_k_paged
    f.argtypes = [P, I64, P, I64, P, I64, P]
    assert f(None, 8448, None, -1, None, 128, None) == 1
    assert "n_tokens" in _err(lib)
    assert f(None, 8448, None, 0, None, 128, None) == 0  # empty: nothing to do
    assert f(P(16), 8000, P(16), 4, P(16), 128, None) == 1  # page stride below 8448
    assert "8448" in _err(lib)
    g = lib.dsa_mqa_logits_decode
    g.argtypes = [P, P, I, I64, I, P, I64, P, P, I64, I64, P, I64, P, I64, I, I, P, P, I, P]
    assert g(P(16), P(16), 48, 2, 1, P(16), 8448, P(16), P(16), 4, 4, P(16), 256, P(16), 16, 1, 0, None, None, 0,
             None) == 1
    assert "heads" in _err(lib)
    assert g(P(16), P(16), 64, 3, 2, P(16), 8448, P(16), P(16), 4, 4, P(16), 256, P(16), 16, 1, 0, None, None, 0,
             None) == 1
    assert "group_size" in _err(lib)
    assert g(P(16), P(16), 64, 2, 1, P(16), 8448, P(16), P(16), 4, 4, P(16), 256, P(16), 16, 1, 0, None, P(16), 1,
             None) == 1
    assert "fuse_pass1" in _err(lib)
    t = lib.dsa_topk_transform
    t.argtypes = [P, I64, I64, P, I64, P, I64, P, I64, I64, P, I64, I, I, P, ctypes.c_size_t, P, P]
    lib.dsa_topk_workspace_bytes.argtypes = [I64, I64, I, I]
    lib.dsa_topk_workspace_bytes.restype = ctypes.c_size_t
    need = lib.dsa_topk_workspace_bytes(4, 65536, 8, 256)
    assert need > 0 and lib.dsa_topk_workspace_bytes(4, 65536, 1, 256) == 0
    assert lib.dsa_topk_workspace_bytes(600, 65536, 8, 256) == 0  # rows >= CUs: one CTA per row
    assert t(P(16), 65536, 65536, None, 0, P(16), 4, P(16), 65536, 65536, None, 4, 8, 256, P(256), need - 1,
             P(16), None) == 1
    assert "workspace" in _err(lib)


def test_torch_bind_rejects_bad_operands():
    import hcu_ops
    from hcu_ops import _C
    q = torch.zeros(2, 1, 64, 128, dtype=torch.float8_e4m3fn)
    kv = torch.zeros(4, 64, 1, 132, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="q must be contiguous fp8"):
        _C.mqa_logits_hist(q, kv, torch.zeros(2, 64), torch.zeros(2, dtype=torch.int32),
                           torch.zeros(2, 4, dtype=torch.int32), 256, 1, 0, 1, None)
    with pytest.raises(RuntimeError, match="topk=2048"):
        _C.sparse_mask_topk_transform(torch.zeros(1, 16), torch.zeros(1, 1, dtype=torch.int16),
                                      torch.zeros(1, dtype=torch.int32), torch.zeros(1, 16, dtype=torch.int32),
                                      torch.zeros(2, dtype=torch.int32), 1024)
    with pytest.raises(RuntimeError, match="score must be row-contiguous float32"):
        _C.sparse_mask_topk_transform(torch.zeros(1, 16), torch.zeros(1, 1, dtype=torch.int16),
                                      torch.zeros(1, dtype=torch.int32), torch.zeros(1, 16, dtype=torch.int32),
                                      torch.zeros(2, dtype=torch.int32), 2048)
    # operand gate used by the sglang call site: CPU-checkable shapes / dtypes
    w = torch.zeros(2, 64)
    assert hcu_ops.mqa_logits_supported(q, kv, w, 1)
    assert hcu_ops.mqa_logits_supported(q, kv, w, 2)
    assert not hcu_ops.mqa_logits_supported(q, kv, w, 3)
    assert not hcu_ops.mqa_logits_supported(q.view(torch.uint8), kv, w, 1)
    assert not hcu_ops.mqa_logits_supported(torch.zeros(2, 1, 48, 128, dtype=torch.float8_e4m3fn), kv,
                                            torch.zeros(2, 48), 1)
    assert not hcu_ops.mqa_logits_supported(q, kv, w, 1, block_table=torch.zeros(2, 4, dtype=torch.int32),
                                            max_context_len=300)


def test_prefill_slab_policy(lib):
    """Slab rows for a byte budget: a multiple of 8 rows when at least 8 fit, capped at the cap and
    at the rows; the workspace holds one slab of f32 logits (256-B aligned) plus the top-k's."""
    I64, I = ctypes.c_int64, ctypes.c_int
    lib.dsa_prefill_slab_rows.argtypes = [I64, I64, I64, I64]
    lib.dsa_prefill_slab_rows.restype = I64
    lib.dsa_prefill_indexer_workspace_bytes.argtypes = [I64, I64, I64, I, I]
    lib.dsa_prefill_indexer_workspace_bytes.restype = ctypes.c_size_t
    width = 147456
    assert lib.dsa_prefill_slab_rows(16384, width, 4096, 2 << 30) == 3640  # 2 GiB of logits rows
    assert lib.dsa_prefill_slab_rows(16384, width, 4096, 4096 * width * 4) == 4096
    assert lib.dsa_prefill_slab_rows(16384, width, 4096, 0) == 4096  # no budget: the cap
    assert lib.dsa_prefill_slab_rows(5, width, 4096, 1 << 40) == 5
    assert lib.dsa_prefill_slab_rows(100, width, 0, 13 * width * 4) == 8
    assert lib.dsa_prefill_slab_rows(100, width, 0, 3 * width * 4) == 3
    assert lib.dsa_prefill_slab_rows(100, width, 0, 1) == 1
    need = lib.dsa_prefill_indexer_workspace_bytes(16384, width, 4096, 8, 256)
    assert need == 4096 * width * 4  # 4096-row slabs: one CTA a row, no top-k workspace
    small = lib.dsa_prefill_indexer_workspace_bytes(4, 70000, 4, 8, 256)
    assert small > (4 * 70000 * 4 + 255) // 256 * 256  # four 70K rows split: the top-k's workspace too


def test_reference_knob_gate(monkeypatch):
    """mqa_logits pairs with the top-k only where the reference's gate would: the split top-k
    must split rows (reference hcu_ops/hcu_ops/__init__.py:96-98).  MI355X: 256 CUs."""
    import hcu_ops
    monkeypatch.setattr(hcu_ops, "_N_CU", 256)
    assert hcu_ops._topk_splits(128, 65536) > 1
    assert hcu_ops._topk_splits(32, 16384) == 1
    assert hcu_ops._topk_splits(1, 4096) == 1
    assert hcu_ops._topk_splits(600, 65536) == 1


def test_noalloc_topk_rejects_oversize_on_the_host(lib):
    """The allocation-free top-k refuses inputs whose split workspace exceeds its built-in array,
    before touching a device: 300 rows of 64K split in two need ~14.7 MB."""
    P, I64, I = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.dsa_topk_noalloc_max_bytes.restype = ctypes.c_size_t
    lib.dsa_topk_workspace_bytes.argtypes = [I64, I64, I, I]
    lib.dsa_topk_workspace_bytes.restype = ctypes.c_size_t
    cap = lib.dsa_topk_noalloc_max_bytes()
    assert cap == 4096 + 3 * 256 * 4096 * 4  # counters, then keys, tokens and page-table entries of 256 rows
    assert lib.dsa_topk_workspace_bytes(256, 65536, 8, 256) == cap
    assert lib.dsa_topk_workspace_bytes(300, 65536, 8, 256) > cap
    # scores wider than 81,920 tokens: 5120-entry lists, so 204 split rows fit and 205 do not
    assert lib.dsa_topk_workspace_bytes(204, 131072, 8, 256) <= cap < lib.dsa_topk_workspace_bytes(205, 131072, 8, 256)
    assert lib.dsa_topk_workspace_bytes(204, 131072, 8, 256) > lib.dsa_topk_workspace_bytes(204, 81920, 8, 256)
    f = lib.dsa_topk_transform_noalloc
    f.argtypes = [P, I64, I64, P, I64, P, I64, P, I64, I64, P, I64, I, I, P, P]
    assert f(P(16), 65536, 65536, None, 0, P(16), 300, P(16), 65536, 65536, None, 300, 8, 256, P(16), None) == 2
    assert "built-in" in _err(lib)
