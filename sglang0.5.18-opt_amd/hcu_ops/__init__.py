"""MI355X (gfx950) DSA indexer operators, drop-in for the reference's ``hcu_ops`` surface.

Operator names, signatures and the env-switch conventions follow
hcu_ops/hcu_ops/__init__.py:1-105 of the reference: ``mqa_logits_supported`` / ``mqa_logits``
(called by sglang's dsa_indexer paged branch), ``sparse_mask_topk_transform`` (called by
dsa_indexer_metadata's top-k transform) and the logits -> top-k pairing that lets the top-k
reuse the pass-1 histogram built inside the logits kernel.  Additions: H = 64 heads (the
reference hard-codes 32), the bf16 q quantisation step, paged K dequant / gather, the K-cache
writer, prefill logits and a dense-score top-k with the varlen (cu_seqlens_q) layout.

All compute runs in the HIP library ``libdsa_indexer.so`` through the ``_C`` bind; importing this
package fails if the extension has not been built (python build.py): there is no fallback.
"""
import os

import torch  # noqa: F401  (loads libtorch / the HIP runtime before the extension)

from . import _C

# HCU_TOPK_IMPL: "split" (default) lets the top-k spread a row over up to HCU_TOPK_SPLITS CTAs while
# the rows are few; "single" keeps one CTA per row.
_TOPK_IMPL = os.environ.get("HCU_TOPK_IMPL", "split")
_TOPK_SPLITS = int(os.environ.get("HCU_TOPK_SPLITS", "8"))

# Logits launch and its pairing with the top-k (the reference's knob names and meanings):
#   HCU_MQA_PCTAS[_G1]   CTAs per request row-set for grouped [single] rows; <= 0 takes every CTA that
#                        is resident at once (on gfx950 that beats the reference's -1 policy of 64 per
#                        row-set for few rows: the balanced grid spreads the pages over the whole chip).
#   HCU_MQA_RPC          rows of a group sharing one K page stream (must divide the group).
#   HCU_MQA_HIST_MAX_ROWS[_G6]  up to this many single [grouped] rows, when the paired top-k will split
#                        rows, mqa_logits(..., hist_lens) builds the top-k's pass-1 histogram inside the
#                        logits kernel (rows_per_cta <= 3).
#   HCU_MQA_PAIR_MAX_ROWS (this build's addition) otherwise, up to this many rows, the logits kernel
#                        only zeroes the paired split top-k's per-row counters on its way, which saves
#                        the top-k its zeroing launch; the top-k then selects against its sampled
#                        threshold.  Measured on gfx950, the fused histogram loses everywhere, hence
#                        0 for both (the reference fuses up to 8 single rows): its 8 KB of LDS
#                        counters per row cost the logits kernel occupancy, and the exact-bin top-k
#                        after it is slower than the sampled one.  Decode steps (logits + top-k) of
#                        1 / 8 single rows of 65,536 tokens, H = 64: 86.7 / 116.3 us fused,
#                        24.7 / 34.2 us with the counters only; the 64-request MTP decode (G = 2):
#                        logits 54.8 -> 58.7 us fused.
_MQA_PCTAS = int(os.environ.get("HCU_MQA_PCTAS", "0"))
_MQA_PCTAS_G1 = int(os.environ.get("HCU_MQA_PCTAS_G1", str(_MQA_PCTAS)))
_MQA_RPC = int(os.environ.get("HCU_MQA_RPC", "2"))
_MQA_HIST_MAX_ROWS = int(os.environ.get("HCU_MQA_HIST_MAX_ROWS", "0"))
_MQA_HIST_MAX_ROWS_G6 = int(os.environ.get("HCU_MQA_HIST_MAX_ROWS_G6", "0"))
_MQA_PAIR_MAX_ROWS = int(os.environ.get("HCU_MQA_PAIR_MAX_ROWS", "256"))
_MQA_HIST = None  # (logits, hist_lens, zws, pass1_done) of the last mqa_logits with hist_lens
_N_CU = None
# Prefill: SGLANG_NSA_MQA_LOGITS_MEMORY_BUDGET_GB bounds the logits slab of prefill_indexer, as it
# bounds sglang's prefill indexer (reference prefill/p_opt.sh:58); slabs hold at most 4096 rows.
_PREFILL_BUDGET = int(float(os.environ.get("SGLANG_NSA_MQA_LOGITS_MEMORY_BUDGET_GB", "2")) * (1 << 30))
_PREFILL_MAX_SLAB_ROWS = 4096
_HEADS = (32, 64)


def sparse_mask_topk_transform(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk=2048):
    """Drop-in for lightop.attention.fast_topk_transform_sparse_mask_fused (reference
    hcu_ops/hcu_ops/__init__.py:15-32): int32 [rows, 2048] page-table entries of the top-2048
    tokens of every row (ties to the lower token), -1 padded for rows shorter than 2048."""
    global _MQA_HIST
    st = _MQA_HIST
    if st is not None:
        _MQA_HIST = None
        if st[0] is score and st[1].data_ptr() == lengths.data_ptr() and st[1].shape == lengths.shape:
            # the pass-1 workspace came from mqa_logits(..., hist_lens=lengths)
            return _C.sparse_mask_topk_transform_split_pre(score, nonzero_mask, lengths, page_table_size_1,
                                                           cu_seqlens_q, topk, _TOPK_SPLITS, st[2], st[3])
    if _TOPK_IMPL == "single":
        return _C.sparse_mask_topk_transform(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk)
    return _C.sparse_mask_topk_transform_split(score, nonzero_mask, lengths, page_table_size_1, cu_seqlens_q, topk,
                                               _TOPK_SPLITS)


def sparse_mask_topk_transform_blocks(score, nonzero_mask, lengths, block_table, cu_seqlens_q, topk=2048):
    """sparse_mask_topk_transform with the 64-token-page block table that page_table_size_1 expands
    (this build's addition; the reference gathers page_table_size_1[row][t]): token t maps to
    block_table[row][t // 64] * 64 + t % 64, so the transform reads 4 B per 64 tokens instead of
    4 B per token.  Pairs with a preceding mqa_logits(..., hist_lens=lengths) like the reference
    form."""
    global _MQA_HIST
    st = _MQA_HIST
    zws, done = None, False
    if st is not None:
        _MQA_HIST = None
        if st[0] is score and st[1].data_ptr() == lengths.data_ptr() and st[1].shape == lengths.shape:
            zws, done = st[2], st[3]
    splits = 1 if _TOPK_IMPL == "single" and zws is None else _TOPK_SPLITS
    return _C.sparse_mask_topk_transform_blocks(score, nonzero_mask, lengths, block_table, cu_seqlens_q, topk, splits,
                                                zws, done)


def mqa_logits_supported(q, kv_cache, weights, group_size, context_lens=None, block_table=None,
                         max_context_len=None):
    """Whether mqa_logits takes these operands (else the caller keeps its fallback)."""
    b = q.shape[0] if q.dim() == 4 else 0
    h = q.shape[2] if q.dim() == 4 else 0
    rpc = 1 if group_size == 1 else _MQA_RPC
    ok = (q.dtype == torch.float8_e4m3fn and q.dim() == 4 and q.shape[1] == 1 and h in _HEADS and q.shape[3] == 128
          and b > 0 and q.is_contiguous() and weights.dtype == torch.float32
          and tuple(weights.shape) == (b, h) and weights.is_contiguous()
          and kv_cache.dtype == torch.uint8 and kv_cache.dim() == 4
          and tuple(kv_cache.shape[1:]) == (64, 1, 132) and kv_cache.stride(1) == 132
          and kv_cache.stride(3) == 1 and kv_cache.stride(0) % 16 == 0
          and group_size >= 1 and b % group_size == 0 and rpc in (1, 2, 3, 4) and group_size % rpc == 0)
    if ok and context_lens is not None:
        ok = context_lens.dtype == torch.int32 and context_lens.numel() == b and context_lens.is_contiguous()
    if ok and block_table is not None:
        ok = (block_table.dtype == torch.int32 and block_table.dim() == 2 and block_table.shape[0] == b
              and block_table.stride(1) == 1
              and (max_context_len is None or max_context_len == block_table.shape[1] * 64))
    return ok


def _topk_splits(rows, width):
    """CTAs per row the paired split top-k will use for [rows, width] scores (reference
    hcu_ops/hcu_ops/__init__.py:61-66, with this build's split policy)."""
    global _N_CU
    if _N_CU is None:
        _N_CU = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    return _C.topk_splits(rows, width, _TOPK_SPLITS, _N_CU)


def mqa_logits(q, kv_cache, weights, context_lens, block_table, max_context_len, group_size, hist_lens=None,
               persistent_ctas=None, rows_per_cta=None):
    """(logits f32 [B, max_context_len], mask i16 [B, max_context_len/16]) of the paged indexer
    (reference hcu_ops/hcu_ops/__init__.py:82-105).

    hist_lens: lengths of the paired sparse_mask_topk_transform; when that call will split rows,
    its workspace is prepared here (pass 1 built, or its counters zeroed; see the knobs above)."""
    global _MQA_HIST
    rows = q.shape[0]
    if persistent_ctas is None:
        persistent_ctas = _MQA_PCTAS_G1 if group_size == 1 else _MQA_PCTAS
    if rows_per_cta is None:
        rows_per_cta = 1 if group_size == 1 else _MQA_RPC
    hist_max_rows = _MQA_HIST_MAX_ROWS if group_size == 1 else _MQA_HIST_MAX_ROWS_G6
    use_hist = (hist_lens is not None and _TOPK_IMPL == "split"
                and rows <= max(hist_max_rows, _MQA_PAIR_MAX_ROWS)
                and hist_lens.dtype == torch.int32 and hist_lens.dim() == 1
                and hist_lens.shape[0] == rows and hist_lens.is_contiguous()
                and _topk_splits(rows, max_context_len) > 1)
    fused = use_hist and rows <= hist_max_rows and rows_per_cta <= 3
    logits, mask, zws = _C.mqa_logits_hist(q, kv_cache, weights, context_lens.view(-1), block_table,
                                           max_context_len, group_size, persistent_ctas, rows_per_cta,
                                           hist_lens if use_hist else None, fused)
    _MQA_HIST = (logits, hist_lens, zws, fused) if use_hist else None
    return logits, mask


def dequantize_k_cache_paged(quant_k_cache, page_table_1_flattened, group_size=128):
    """sglang dequantize_k_cache_paged for the 656-B MLA slot (reference
    prefill/patches/dequant_k_cache.py.diff:51-69): bf16 [n, 1, 576]."""
    return _C.dequantize_k_cache_paged(quant_k_cache, page_table_1_flattened, group_size)


def dequant_k_paged(kv_cache, slots):
    """Indexer 132-B paged fp8 K at token slots -> bf16 [n, 128] (fp32 product, one RNE)."""
    return _C.dequant_k_paged(kv_cache, slots)


def gather_k_paged(kv_cache, slots):
    """Indexer 132-B paged fp8 K at token slots -> (fp8 [n, 128], f32 scale [n])."""
    return _C.gather_k_paged(kv_cache, slots)


def quant_q_fp8(q, weights):
    """bf16 q [..., H, 128] -> (fp8 q8, weights * per-(row, head) scale)."""
    return _C.quant_q_fp8(q, weights)


def store_k_cache(k, slots, kv_cache):
    """Quantises bf16 k [n, 128] per token and stores it at `slots` of the 132-B paged cache
    (a negative slot, a padded entry, stores nothing)."""
    _C.store_k_cache(k, slots, kv_cache)


def mqa_logits_prefill(q, weights, kv_cache, block_table, lens, width):
    """Prefill indexer logits f32 [rows, width] of one request (key t < lens[r] of row r)."""
    return _C.mqa_logits_prefill(q, weights, kv_cache, block_table, lens, width)


def topk_transform(score, lengths, page_table_size_1, cu_seqlens_q, topk=2048, max_splits=None, out=None):
    """Top-2048 + page-table transform over dense scores (every score below the length valid);
    cu_seqlens_q [requests + 1] maps rows to their request's page-table row (varlen layout).
    out: an int32 [rows, 2048] contiguous tensor to write (and return) instead of a new one."""
    if max_splits is None:
        max_splits = _TOPK_SPLITS if _TOPK_IMPL == "split" else 1
    return _C.topk_transform(score, lengths, page_table_size_1, cu_seqlens_q, topk, max_splits, out)


def prefill_indexer(q, weights, kv_cache, block_table, lens, width, page_table_1=None, memory_budget_bytes=None,
                    max_slab_rows=None, out=None):
    """Top-2048 slots of every query row of one prefill request: int32 [rows, 2048].

    q fp8 [rows, H, 128] and weights f32 [rows, H] (quant_q_fp8's outputs), the request's paged
    K (block_table int32 [pages]), lens int32 [rows] (causal: prefix + i + 1), width = keys of the
    request.  The logits are scored in row slabs of at most memory_budget_bytes (default
    SGLANG_NSA_MQA_LOGITS_MEMORY_BUDGET_GB) and max_slab_rows (default 4096) rows, each slab's
    top-2048 selected right behind it, so at most one slab of logits exists.  page_table_1:
    int32 [>= width] token -> slot (default: the block table's slots, bt[t / 64] * 64 + t % 64).
    out: an int32 [rows, 2048] contiguous tensor to fill instead of a new one."""
    if page_table_1 is None:
        t = torch.arange(width, dtype=torch.int64, device=block_table.device)
        page_table_1 = (block_table.long()[t // 64] * 64 + t % 64).to(torch.int32)
    budget = _PREFILL_BUDGET if memory_budget_bytes is None else int(memory_budget_bytes)
    cap = _PREFILL_MAX_SLAB_ROWS if max_slab_rows is None else int(max_slab_rows)
    splits = _TOPK_SPLITS if _TOPK_IMPL == "split" else 1
    return _C.prefill_indexer(q, weights, kv_cache, block_table, lens, width, page_table_1, budget, cap, splits, out)
