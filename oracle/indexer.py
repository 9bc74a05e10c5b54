"""CPU restatement of the DSA indexer path (numpy; torch CPU only for the CPU-baseline pipeline).

Test infrastructure: see oracle/__init__.py for who may import this and how it is pinned.
"""
import numpy as np

from .fp8 import bf16_rne, float_key, fp8_decode, fp8_encode

PAGE = 64
HEAD_DIM = 128
TOK_BYTES = HEAD_DIM + 4
PAGE_FP8 = PAGE * HEAD_DIM
TOPK = 2048
ZERO_KEY = np.uint32(0x80000000)


# --------------------------------------------------------------------------------------------
# K-cache layout: page p = [64 x 128 fp8][64 x f32 scale] (hcu_ops/csrc/mqa_hist.cu:79-91,
# hcu_ops/tests/test_mqa_hist.py:31-38).  `kv` is uint8 [n_pages, page_stride].

def kv_token(kv, slot):
    """(fp8 codes [128], scale f32) of token slot = page * 64 + offset."""
    page, off = divmod(int(slot), PAGE)
    codes = kv[page, off * HEAD_DIM:(off + 1) * HEAD_DIM]
    scale = kv[page, PAGE_FP8 + off * 4:PAGE_FP8 + off * 4 + 4].view(np.float32)[0]
    return codes, scale


def kv_tokens(kv, slots):
    """Vectorised kv_token: (codes uint8 [n, 128], scale f32 [n])."""
    slots = np.asarray(slots, dtype=np.int64)
    page, off = slots // PAGE, slots % PAGE
    cols = off[:, None] * HEAD_DIM + np.arange(HEAD_DIM)[None, :]
    codes = kv[page[:, None], cols]
    sc_bytes = kv[page[:, None], PAGE_FP8 + off[:, None] * 4 + np.arange(4)[None, :]]
    scale = np.ascontiguousarray(sc_bytes).view(np.float32).reshape(-1)
    return codes, scale


def slots_of(block_table_row, n_tokens):
    """Token slots of the first n_tokens of a request: bt[t / 64] * 64 + t % 64."""
    t = np.arange(n_tokens, dtype=np.int64)
    return np.asarray(block_table_row, dtype=np.int64)[t // PAGE] * PAGE + t % PAGE


def dequant_k_paged(kv, slots):
    """bf16 bits [n, 128]: bf16_rne(f32(fp8) * scale) -- the closed form of the reference's paged
    dequant (prefill/patches/dequant_k_cache.py.diff:30-36) on the indexer's 132-B layout."""
    codes, scale = kv_tokens(kv, slots)
    vals = fp8_decode(codes) * scale[:, None]  # float32 * float32 -> float32 (one rounding)
    out = bf16_rne(vals.astype(np.float32))
    out[np.asarray(slots) < 0] = 0
    return out


def dequant_mla(cache, slots):
    """bf16 bits [n, 576] of the 656-B MLA slot (dequant_k_cache.py.diff:16-42,56-62):
    [0:512] = bf16_rne(f32(fp8[j]) * scale[j // 128]), [512:576] = the bf16 rope copy.  A
    negative slot (a padded entry, which the reference's kernel would read out of bounds) gives
    a zero row, as in dequant_k_paged."""
    slots = np.asarray(slots, dtype=np.int64)
    rows = cache[np.maximum(slots, 0)]
    codes = rows[:, :512]
    scale = np.ascontiguousarray(rows[:, 512:528]).view(np.float32).reshape(-1, 4)
    vals = fp8_decode(codes).reshape(-1, 4, 128) * scale[:, :, None]
    nope = bf16_rne(vals.reshape(-1, 512).astype(np.float32))
    rope = np.ascontiguousarray(rows[:, 528:656]).view(np.uint16).reshape(-1, 64)
    out = np.concatenate([nope, rope], axis=1)
    out[slots < 0] = 0
    return out


def cpu_dequant_torch(src, slots, mla):
    """torch-CPU restatement of dequant_k_paged (mla=False: src u8 [pages, 8448] of the 132-B
    layout) and dequant_mla (mla=True: src u8 [pool, 656]) for valid slots, on torch's intra-op
    threads (the multi-thread CPU baseline): bf16 [n, 128] / [n, 576].  fp8 -> f32 is exact, the
    product one f32 rounding, .to(bfloat16) round-to-nearest-even, as in the numpy forms above."""
    import torch
    slots = slots.long()
    if mla:
        rows = src[slots]
        n = rows.shape[0]
        vals = rows[:, :512].contiguous().view(torch.float8_e4m3fn).float().view(n, 4, 128)
        scale = rows[:, 512:528].contiguous().view(torch.float32).view(n, 4, 1)
        nope = (vals * scale).view(n, 512).to(torch.bfloat16)
        rope = rows[:, 528:656].contiguous().view(torch.bfloat16)
        return torch.cat([nope, rope], 1)
    page, off = slots // PAGE, slots % PAGE
    cols = off[:, None] * HEAD_DIM + torch.arange(HEAD_DIM)[None, :]
    codes = src[page[:, None], cols]
    sc = src[page[:, None], PAGE_FP8 + off[:, None] * 4 + torch.arange(4)[None, :]].contiguous().view(torch.float32)
    return (codes.view(torch.float8_e4m3fn).float() * sc).to(torch.bfloat16)


# --------------------------------------------------------------------------------------------
# Per-vector fp8 quantisation (hcu_ops/csrc/norm_quant.cu:13-14: amax = max|x| taken with fmaxf
# from 0, so NaN elements do not count, scale = amax / 448, q = fp8(x * (448 / amax)),
# amax == 0 -> 0), all in float32.

def quant_vectors(x):
    """x float32 [..., 128] -> (codes uint8 [..., 128], scale float32 [...])."""
    x = np.asarray(x, dtype=np.float32)
    amax = np.fmax.reduce(np.abs(x), axis=-1, initial=np.float32(0.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(amax == 0, np.float32(0), np.float32(448.0) / amax).astype(np.float32)
    scale = (amax / np.float32(448.0)).astype(np.float32)
    codes = fp8_encode((x * inv[..., None]).astype(np.float32))
    return codes, scale


def quant_q(q_bf16_bits, w):
    """bf16 q [rows, H, 128] (bit patterns) and w [rows, H] -> (q8 codes, w * scale)."""
    q = (np.asarray(q_bf16_bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)
    codes, scale = quant_vectors(q)
    return codes, (np.asarray(w, dtype=np.float32) * scale).astype(np.float32)


def build_kv_cache(k_f32, slots, n_pages, page_stride=PAGE * TOK_BYTES):
    """Quantises k float32 [n, 128] per token into a fresh 132-B paged cache at `slots`."""
    kv = np.zeros((n_pages, page_stride), dtype=np.uint8)
    codes, scale = quant_vectors(k_f32)
    slots = np.asarray(slots, dtype=np.int64)
    page, off = slots // PAGE, slots % PAGE
    kv[page[:, None], off[:, None] * HEAD_DIM + np.arange(HEAD_DIM)[None, :]] = codes
    sb = scale.astype(np.float32).view(np.uint8).reshape(-1, 4)
    kv[page[:, None], PAGE_FP8 + off[:, None] * 4 + np.arange(4)[None, :]] = sb
    return kv


# --------------------------------------------------------------------------------------------
# MQA logits (hcu_ops/csrc/mqa_hist.cu:96-273): rows of a group share the first row's block
# table; logit = scale_t * sum_h w_h * relu(q8_h . k8_t); mask bit = t < len && logit != 0.

def head_scores(q8_codes_row, k8_codes):
    """Exact q8_h . k8_t for every head h and key t (float64 [H, n]); the fp8 products and
    their 128-term sums are exact in float64."""
    q = fp8_decode(q8_codes_row).astype(np.float64)
    k = fp8_decode(k8_codes).astype(np.float64)
    return q @ k.T


def logits_row(q8_codes_row, w_row, k8_codes, k_scale):
    """(logit, magnitude, dot magnitude), float64 [n] each, of one query row over keys.
    The magnitude A_t = scale_t * sum_h |w_h| relu(acc_h) bounds |logit| and sets the scale of
    the fp32 rounding error (it equals |logit| when all weights share a sign).  The dot magnitude
    M_t = scale_t * sum_h |w_h| sum_d |q8_hd k8_td| (every head, every product) sets the scale of
    a matrix instruction's accumulation error, which is relative to the products it sums."""
    acc = head_scores(q8_codes_row, k8_codes)
    r = np.maximum(acc, 0.0)
    w = np.asarray(w_row, dtype=np.float64)
    s = np.asarray(k_scale, dtype=np.float64)
    q = np.abs(fp8_decode(q8_codes_row).astype(np.float64))
    k = np.abs(fp8_decode(k8_codes).astype(np.float64))
    return (w @ r) * s, (np.abs(w) @ r) * s, (np.abs(w) @ (q @ k.T)) * s


def mqa_logits_decode(q8, w, kv, context_lens, block_table, group, width):
    """Oracle of dsa_mqa_logits_decode: (logits float64 [B, width] with NaN where not
    written, magnitude and dot magnitude float64 [B, width] (logits_row), mask int16
    [B, width / 16])."""
    B = q8.shape[0]
    logits = np.full((B, width), np.nan)
    mag = np.zeros((B, width))
    dmag = np.zeros((B, width))
    bits = np.zeros((B, width), dtype=bool)
    lens = np.clip(np.asarray(context_lens, dtype=np.int64), 0, width)
    for g0 in range(0, B, group):
        n = int(lens[g0:g0 + group].max()) if B else 0
        if n == 0:
            continue
        # the group's keys are gathered once; every row of the group reads a prefix of them
        codes, scale = kv_tokens(kv, slots_of(block_table[g0], n))
        for r in range(g0, g0 + group):
            L = int(lens[r])
            if L == 0:
                continue
            lg, mg, dm = logits_row(q8[r], w[r], codes[:L], scale[:L])
            logits[r, :L] = lg
            mag[r, :L] = mg
            dmag[r, :L] = dm
            bits[r, :L] = lg != 0.0
    return logits, mag, dmag, pack_mask(bits)


def pack_mask(bits):
    """bool [rows, width] -> int16 [rows, ceil(width / 16)] (bit t % 16 of word t / 16)."""
    rows, width = bits.shape
    pad = (-width) % 16
    if pad:
        bits = np.concatenate([bits, np.zeros((rows, pad), dtype=bool)], axis=1)
    w16 = (1 << np.arange(16)).astype(np.int64)
    words = (bits.reshape(rows, -1, 16).astype(np.int64) * w16).sum(-1)
    return words.astype(np.uint16).view(np.int16)


def unpack_mask(mask, width):
    m = np.asarray(mask).view(np.uint16).astype(np.int64)
    bits = (m[:, :, None] >> np.arange(16)[None, None, :]) & 1
    return bits.reshape(m.shape[0], -1)[:, :width].astype(bool)


def mqa_logits_prefill(q8, w, kv, block_table, lens, width):
    """Oracle of dsa_mqa_logits_prefill: rows of one request, key t < lens[r]: (logits,
    magnitude, dot magnitude) as mqa_logits_decode."""
    rows = q8.shape[0]
    n = int(np.clip(np.max(lens), 0, width)) if rows else 0
    codes, scale = kv_tokens(kv, slots_of(block_table, n))
    logits = np.full((rows, width), np.nan)
    mag = np.zeros((rows, width))
    dmag = np.zeros((rows, width))
    for r in range(rows):
        L = int(np.clip(lens[r], 0, width))
        lg, mg, dm = logits_row(q8[r], w[r], codes[:L], scale[:L])
        logits[r, :L] = lg
        mag[r, :L] = mg
        dmag[r, :L] = dm
    return logits, mag, dmag


# --------------------------------------------------------------------------------------------
# Top-k (hcu_ops/csrc/sparse_mask_topk.cu:1-7,40-43,141-349).

def row_keys(score_row, mask_row, length):
    """uint32 keys of tokens [0, length): masked-out tokens are +0 (kZeroKey), never read."""
    s = np.asarray(score_row[:length], dtype=np.float32)
    k = float_key(s)
    if mask_row is not None:
        bits = unpack_mask(np.asarray(mask_row)[None, :], length)[0]
        k = np.where(bits, k, ZERO_KEY)
    return k.astype(np.uint32)


def topk_tokens(keys, k=TOPK):
    """Token indices of the k largest keys, ties to the lower index (stable sort)."""
    order = np.lexsort((np.arange(keys.shape[0]), -keys.astype(np.int64)))
    return np.sort(order[:k])


def topk_transform(score, mask, lengths, page_table, width, cu_seqlens_q=None):
    """Oracle of dsa_topk_transform: int32 [rows, 2048]; selected rows are returned as the
    page-table entries of the selected tokens in ascending token order (the contract is the
    set), short rows as page_table[:len] then -1.  Tokens past a page-table row's columns map
    to -1 (the reference requires >= len columns; this build defines the rest)."""
    rows = score.shape[0]
    out = np.full((rows, TOPK), -1, dtype=np.int32)

    def entries(pt, toks):
        v = np.full(len(toks), -1, dtype=np.int32)
        inside = toks < pt.shape[0]
        v[inside] = pt[toks[inside]]
        return v

    for r in range(rows):
        pr = r if cu_seqlens_q is None else int(np.searchsorted(cu_seqlens_q, r, side="right") - 1)
        L = int(np.clip(lengths[r], 0, width))
        pt = page_table[pr]
        if L <= TOPK:
            out[r, :L] = entries(pt, np.arange(L))
            continue
        keys = row_keys(score[r], None if mask is None else mask[r], L)
        out[r] = entries(pt, topk_tokens(keys))
    return out


def pass1_hist(score, mask, hist_lens, width):
    """Top-k pass-1 workspace [ghist1 rows*4096 | ghist2 rows*4096 | (pos, zeros) rows*2] for
    rows with min(hist_len, width) > 2048 (closed form of hcu_ops/tests/test_mqa_hist.py:109-124):
    ghist1 = 12-bit key[31:20] histogram of the set mask bits below the length plus the
    unset ones counted in the zero bin 0x800; pos = set bits with key > +0."""
    rows = score.shape[0]
    g1 = np.zeros((rows, 4096), dtype=np.int64)
    cnt = np.zeros((rows, 2), dtype=np.int64)
    for r in range(rows):
        h = min(int(hist_lens[r]), width)
        if h <= TOPK:
            continue
        keys = row_keys(score[r], None if mask is None else mask[r], h)
        g1[r] = np.bincount((keys >> 20).astype(np.int64), minlength=4096)
        cnt[r] = ((keys > ZERO_KEY).sum(), (keys == ZERO_KEY).sum())
    return np.concatenate([g1.reshape(-1), np.zeros(rows * 4096, dtype=np.int64), cnt.reshape(-1)]).astype(np.int32)


# --------------------------------------------------------------------------------------------
# torch-CPU indexer (the CPU baseline): dequant -> fp32 matmul -> relu * w -> sum_h -> * s ->
# top-2048 by kthvalue threshold with lower-index ties -> page-table gather.

def cpu_indexer_row_torch(q8_f32, w, k_f32, k_scale, page_slots):
    """One query row on torch CPU: q8_f32 [H, 128], w [H], k_f32 [L, 128] (dequantised fp8),
    k_scale [L], page_slots [L] int32 -> int32 [2048] selected slots (-1 padded)."""
    import torch
    acc = q8_f32 @ k_f32.T                                   # [H, L] fp32
    logit = (torch.relu(acc) * w[:, None]).sum(0) * k_scale  # [L]
    L = logit.shape[0]
    out = torch.full((TOPK,), -1, dtype=torch.int32)
    if L <= TOPK:
        out[:L] = page_slots[:L]
        return out
    b = logit.view(torch.int32).to(torch.int64) & 0xFFFFFFFF
    key = torch.where(b >= 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    thr = torch.kthvalue(key, L - TOPK + 1).values           # the 2048th largest key
    above = key > thr
    n_above = int(above.sum())
    ties = torch.nonzero(key == thr).flatten()[:TOPK - n_above]
    sel = torch.cat([torch.nonzero(above).flatten(), ties])
    out[:] = page_slots[sel]
    return out
