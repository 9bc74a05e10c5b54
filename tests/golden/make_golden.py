"""Writes the known-answer fixtures of this directory (run from the repository root:
`python tests/golden/make_golden.py`).  The reference ships no golden vectors for the indexer
path, so these are computed here, independently of `oracle/`: the fp8 and bf16 conversions by
torch's casts (the reference generates its fp8 operands with torch's float -> float8_e4m3fn cast,
hcu_ops/tests/test_mqa_hist.py:36,49), the dot products exactly in float64, and the top-k by a
brute-force sort on the reference's key order (sparse_mask_topk.cu:4-7,40-43,199-234,301-345).

topk_small.npz    seven rows of a 3072-wide score block (ties, exactly 2048 positives, masked zeros
                  filling the set, a short row, NaN / inf / -0.0, a threshold at -0.0 below +0) and
                  their expected rows.
indexer_small.npz one decode group of two rows, 32 heads, three 64-token pages: bf16 q, head
                  weights, the 132-B paged K cache and block table; expected q8 codes, effective
                  weights, exact logits with their magnitudes, the mask words and the dequantised
                  bf16 keys of the first row; and bf16 keys written by the K-cache writer into a
                  zeroed two-page cache (padded slots store nothing).
mla_small.npz     24 slots of the 656-B MLA layout (512 fp8, 4 fp32 group scales, 64 bf16 rope) and
                  the expected bf16 [n, 576] rows of a slot list (a padded slot gives zeros).
"""
import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
TOPK = 2048
ZERO_KEY = 0x80000000


# ------------------------------------------------------------------------------------------ top-k

def keys_of(x, keep):
    """Order-preserving uint32 keys of float32 scores (sparse_mask_topk.cu:40-43); a token whose
    mask bit is clear counts as +0."""
    b = x.view(np.uint32).astype(np.uint64)
    k = np.where(b & 0x80000000, (~b) & 0xFFFFFFFF, b | 0x80000000)
    return np.where(keep, k, ZERO_KEY).astype(np.uint64)


def expected_row(keys, pt_row, length):
    """The reference single kernel's row: the 2048 largest keys, ties to the lower token; keys
    above the threshold in ascending token order, then the ties taken; with exactly 2048
    positive keys the threshold is +0 (its sparse fast path) and they come out in one run."""
    if length <= TOPK:
        return np.array([pt_row[i] if i < length else -1 for i in range(TOPK)], dtype=np.int32)
    k = [int(v) for v in keys[:length]]
    order = sorted(range(length), key=lambda t: (-k[t], t))
    chosen = order[:TOPK]
    if sum(1 for v in k if v > ZERO_KEY) == TOPK:
        out = sorted(chosen)
    else:
        thr = k[order[TOPK - 1]]
        out = sorted(t for t in chosen if k[t] > thr) + sorted(t for t in chosen if k[t] == thr)
    return np.array([pt_row[t] for t in out], dtype=np.int32)


def topk_fixture():
    W, B = 3072, 7
    rng = np.random.default_rng(2048)
    x = rng.standard_normal((B, W)).astype(np.float32)
    keep = np.ones((B, W), dtype=bool)
    lengths = np.array([3072, 2500, 3000, 3072, 1500, 3072, 2600], dtype=np.int32)
    # 1: heavy ties -- four values only, the threshold value held by hundreds of tokens
    x[1] = rng.choice(np.array([1.0, 0.5, 0.25, -1.0], dtype=np.float32), W, p=[0.3, 0.3, 0.3, 0.1])
    # 2: exactly 2048 positive keys, the rest +0 or negative
    x[2] = -np.abs(x[2])
    x[2, rng.choice(3000, 2048, replace=False)] = np.abs(rng.standard_normal(2048)).astype(np.float32) + 0.01
    zero = np.flatnonzero(x[2, :3000] < 0)[::3]
    x[2, zero] = 0.0
    # 3: 1000 positives; 1400 masked-out tokens (+0 whatever their score, half of them 7.0) fill the
    # set; the rest negative
    x[3] = -np.abs(x[3]) - 0.01
    pos = rng.choice(W, 1000, replace=False)
    x[3, pos] = np.abs(x[3, pos])
    rest = np.setdiff1d(np.arange(W), pos)
    masked = rng.choice(rest, 1400, replace=False)
    keep[3, masked] = False
    x[3, masked[::2]] = 7.0  # masked-out tokens are +0 whatever their score
    # 5: specials among normal scores
    sp = rng.choice(W, 40, replace=False)
    x[5, sp[0:8]] = np.nan
    x[5, sp[8:16]] = np.inf
    x[5, sp[16:24]] = -np.inf
    x[5, sp[24:32]] = -0.0
    x[5, sp[32:40]] = 0.0
    # 6: 2000 positives, 30 x +0.0 and 40 x -0.0: the threshold is -0.0, just below +0
    x[6] = -np.abs(x[6]) - 0.01
    perm = rng.permutation(2600)
    x[6, perm[:2000]] = np.abs(x[6, perm[:2000]])
    x[6, perm[2000:2030]] = 0.0
    x[6, perm[2030:2070]] = -0.0
    words = keep.reshape(B, W // 16, 16).astype(np.int64) << np.arange(16)
    mask = words.sum(-1).astype(np.uint16).view(np.int16)
    pt = (np.arange(W, dtype=np.int32)[None, :] * 3 + 5 + 100000 * np.arange(B, dtype=np.int32)[:, None])
    out = np.stack([expected_row(keys_of(x[r], keep[r]), pt[r], int(lengths[r])) for r in range(B)])
    np.savez_compressed(os.path.join(HERE, "topk_small.npz"), score=x, mask=mask, lengths=lengths,
                        page_table=pt, width=np.int32(W), expected=out)


# ---------------------------------------------------------------------------------------- indexer

def fp8_values(codes):
    return torch.from_numpy(np.ascontiguousarray(codes)).view(torch.float8_e4m3fn).to(torch.float64).numpy()


def indexer_fixture():
    H, G, PAGES, W = 32, 2, 4, 192
    g = torch.Generator().manual_seed(132)
    rng = np.random.default_rng(132)
    q = torch.randn(G, H, 128, generator=g).to(torch.bfloat16)
    w = (torch.randn(G, H, generator=g) * 0.35).float()
    codes = rng.integers(0, 256, (PAGES, 64, 128)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN codes
    scales = (2.0 ** rng.uniform(-9, -3, (PAGES, 64))).astype(np.float32)
    kv = np.concatenate([codes.reshape(PAGES, 8192), scales.view(np.uint8).reshape(PAGES, 256)], axis=1)
    bt = np.array([[2, 0, 3], [2, 0, 3]], dtype=np.int32)  # page 1 is not referenced
    lens = np.array([130, 77], dtype=np.int32)

    # q quantisation (norm_quant.cu:13-14): amax = max|x|, q = fp8(x * (448 / amax)), w * amax / 448
    qf = q.float().numpy()
    amax = np.abs(qf).max(-1).astype(np.float32)
    y = (qf * (np.float32(448.0) / amax)[..., None]).astype(np.float32)
    q8 = torch.from_numpy(y).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    w_eff = (w.numpy() * (amax / np.float32(448.0))).astype(np.float32)

    # keys of the group (tokens 0 .. 129 through the first row's block table)
    slots = np.array([bt[0, t // 64] * 64 + t % 64 for t in range(int(lens.max()))], dtype=np.int64)
    kc = codes.reshape(-1, 128)[slots]
    ks = scales.reshape(-1)[slots].astype(np.float64)
    acc = np.einsum("rhd,td->rht", fp8_values(q8), fp8_values(kc))  # exact: fp8 products, 128 terms
    relu = np.maximum(acc, 0.0)
    we = w_eff.astype(np.float64)
    logits = np.full((G, W), np.nan)
    magnitude = np.zeros((G, W))
    bits = np.zeros((G, W), dtype=bool)
    for r in range(G):
        L = int(lens[r])
        logits[r, :L] = (we[r] @ relu[r, :, :L]) * ks[:L]
        magnitude[r, :L] = (np.abs(we[r]) @ relu[r, :, :L]) * ks[:L]
        bits[r, :L] = logits[r, :L] != 0.0
    mask = (bits.reshape(G, W // 16, 16).astype(np.int64) << np.arange(16)).sum(-1).astype(np.uint16).view(np.int16)

    # dequant of the first row's keys: bf16(f32(fp8) * f32(scale)), both roundings to nearest even
    prod = (fp8_values(kc).astype(np.float32) * scales.reshape(-1)[slots][:, None]).astype(np.float32)
    deq = torch.from_numpy(prod).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)

    # K-cache writer: per token the same quantisation, codes at page * 8448 + off * 128, the fp32
    # scale at page * 8448 + 8192 + off * 4; slot < 0 stores nothing
    k = (torch.randn(50, 128, generator=g) * 3).to(torch.bfloat16)
    kslots = rng.permutation(128)[:50].astype(np.int32)
    kslots[::9] = -1
    kf = k.float().numpy()
    kam = np.abs(kf).max(-1).astype(np.float32)
    kcodes = torch.from_numpy((kf * (np.float32(448.0) / kam)[:, None]).astype(np.float32)).to(
        torch.float8_e4m3fn).view(torch.uint8).numpy()
    kscale = (kam / np.float32(448.0)).astype(np.float32)
    written = np.zeros((2, 8448), dtype=np.uint8)
    for i, sl in enumerate(kslots):
        if sl < 0:
            continue
        pg, off = divmod(int(sl), 64)
        written[pg, off * 128:(off + 1) * 128] = kcodes[i]
        written[pg, 8192 + off * 4:8192 + off * 4 + 4] = kscale[i:i + 1].view(np.uint8)

    np.savez_compressed(os.path.join(HERE, "indexer_small.npz"), q_bf16=q.view(torch.int16).numpy().view(np.uint16),
                        w=w.numpy(), kv_cache=kv, block_table=bt, context_lens=lens, width=np.int32(W),
                        group=np.int32(G), q8=q8, w_eff=w_eff, logits=logits, magnitude=magnitude, mask=mask,
                        slots=slots.astype(np.int32), dequant_bf16=deq,
                        k_bf16=k.view(torch.int16).numpy().view(np.uint16), k_slots=kslots, k_cache_written=written)


def mla_fixture():
    pool, n = 24, 40
    g = torch.Generator().manual_seed(656)
    cache = np.zeros((pool, 656), dtype=np.uint8)
    cache[:, :512] = (torch.randn(pool, 512, generator=g) * 0.1).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    scales = (torch.rand(pool, 4, generator=g) * 0.02 + 1e-3).numpy().astype(np.float32)
    cache[:, 512:528] = scales.view(np.uint8)
    cache[:, 528:] = torch.randn(pool, 64, generator=g).to(torch.bfloat16).view(torch.uint8).numpy()
    slots = torch.randint(0, pool, (n,), generator=g, dtype=torch.int32).numpy()
    slots[5] = -1
    rows = cache[np.maximum(slots, 0)]
    vals = fp8_values(rows[:, :512]).astype(np.float32).reshape(n, 4, 128) * scales[np.maximum(slots, 0)][:, :, None]
    nope = torch.from_numpy(vals.astype(np.float32).reshape(n, 512)).to(torch.bfloat16).view(torch.int16).numpy()
    rope = np.ascontiguousarray(rows[:, 528:]).view(np.int16).reshape(n, 64)
    out = np.concatenate([nope, rope], axis=1).view(np.uint16)
    out[slots < 0] = 0
    np.savez_compressed(os.path.join(HERE, "mla_small.npz"), cache=cache, slots=slots, expected=out)


if __name__ == "__main__":
    topk_fixture()
    indexer_fixture()
    mla_fixture()
    for f in ("topk_small.npz", "indexer_small.npz", "mla_small.npz"):
        print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
