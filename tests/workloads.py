"""Seeded synthetic inputs of the indexer workloads (CPU torch tensors).

Every tensor is drawn from a CPU ``torch.Generator`` in the documented order, so the GPU run and
the CPU checker see identical bytes; fp8 is produced by torch's float -> float8_e4m3fn cast
(OCP e4m3fn, round to nearest even) on the CPU.

Workloads (indexer heads H x 128, page size 64, 132-B paged fp8 K cache with per-token scale):
  decode_1x4k        1 request, 1 row, 4096 tokens
  decode_32x16k      32 requests x 1 row, 16384 tokens each
  decode_mtp64       64 requests x 2 rows (MTP verify: lengths L and L + 1), L ~ U[2048, 65536]
  prefill_8k_64k     8192 query rows over a 65536-token cached prefix (73728 keys, causal)
  prefill_16k_128k   16384 query rows over a 131072-token prefix (147456 keys, causal),
                     K drawn from Student-t(4) before quantisation
  dequant_mla_393k   392832 tokens gathered at random from a 2^19-slot pool of 656-B MLA slots
                     (the shape of prefill/microbench/mb_dequant.py:87-113); dequant_mla_131k the
                     same with 131072 tokens
  dequant_k_74k      the 73728 keys of prefill_8k_64k, gathered from its 132-B paged cache
Draw order (decode): q ~ N(0,1) -> bf16; w ~ N(0, 1/8); page permutation; K ~ N(0,1) per pooled
token (decode_mtp64 draws its request lengths from a second generator seeded seed + 1000).
Prefill: q, w, page permutation, K.
The per-token K quantisation is amax / 448 with codes fp8(x * (448 / amax)) in float32
(hcu_ops/csrc/norm_quant.cu:13-14 convention).

topk_scores() restates the reference's ten top-k score distributions
(hcu_ops/tests/topk_lib.py:8-51), with masked-out positions poisoned with NaN.
"""
import math
from dataclasses import dataclass
import torch

PAGE = 64
HEAD_DIM = 128
TOK_BYTES = HEAD_DIM + 4


def quantize_tokens(x):
    """float32 [n, 128] -> (fp8 e4m3fn [n, 128], scale float32 [n]), amax / 448 per token."""
    x = x.float()
    amax = x.abs().amax(-1)
    inv = torch.where(amax == 0, torch.zeros_like(amax), torch.full_like(amax, 448.0) / amax)
    scale = amax / 448.0
    return (x * inv[:, None]).to(torch.float8_e4m3fn), scale


def pack_kv_pages(k8, scale, n_pages):
    """Token-major fp8 [n_pages * 64, 128] + scale -> uint8 [n_pages, 64, 1, 132] pages laid
    out as [64 x 128 fp8][64 x f32 scale] (hcu_ops/tests/test_mqa_hist.py:36-38)."""
    fp8 = k8.view(torch.uint8).reshape(n_pages, PAGE * HEAD_DIM)
    sc = scale.float().contiguous().view(torch.uint8).reshape(n_pages, PAGE * 4)
    return torch.cat([fp8, sc], 1).contiguous().view(n_pages, PAGE, 1, TOK_BYTES)


def _randn_tokens(g, n, dist):
    if dist == "normal":
        return torch.randn(n, HEAD_DIM, generator=g)
    if dist == "student_t4":  # z / sqrt(chi2_4 / 4)
        z = torch.randn(n, HEAD_DIM, generator=g)
        chi = torch.randn(n, HEAD_DIM, 4, generator=g).pow(2).sum(-1)
        return z / torch.sqrt(chi / 4.0)
    raise ValueError(dist)


def build_kv(g, n_pages, dist="normal", chunk_pages=4096):
    """Random K for every pooled token, quantised per token into the paged layout."""
    parts = []
    for p0 in range(0, n_pages, chunk_pages):
        np_ = min(chunk_pages, n_pages - p0)
        k8, sc = quantize_tokens(_randn_tokens(g, np_ * PAGE, dist))
        parts.append(pack_kv_pages(k8, sc, np_))
    return torch.cat(parts, 0) if len(parts) > 1 else parts[0]


@dataclass
class DecodeCase:
    name: str
    q: torch.Tensor            # bf16 [B, H, 128]
    w: torch.Tensor            # f32 [B, H]
    kv: torch.Tensor           # uint8 [n_pages, 64, 1, 132]
    context_lens: torch.Tensor  # int32 [B]
    block_table: torch.Tensor  # int32 [B, bt_pages] (rows of a group share their request's table)
    group: int

    @property
    def rows(self):
        return self.q.shape[0]

    @property
    def width(self):
        return self.block_table.shape[1] * PAGE

    def page_table_1(self):
        """int32 [B, width] token -> slot table (the page-table remap the top-k applies)."""
        t = torch.arange(self.width, dtype=torch.int64)
        return (self.block_table.long()[:, t // PAGE] * PAGE + t % PAGE).to(torch.int32)

    def tokens_scored(self):
        return int(self.context_lens.clamp(max=self.width).long().sum())


def decode_case(seed, req_lens, group=1, heads=64, bt_pages=None, name="decode", row_offsets=None):
    """Paged decode batch: request i holds req_lens[i] + group - 1 tokens; its rows see
    req_lens[i] + row_offsets[j] tokens (default 0, 1, ..., group - 1)."""
    g = torch.Generator().manual_seed(seed)
    n_req = len(req_lens)
    B = n_req * group
    q = torch.randn(B, heads, HEAD_DIM, generator=g).to(torch.bfloat16)
    w = torch.randn(B, heads, generator=g) * math.sqrt(1.0 / 8.0)
    offs = list(range(group)) if row_offsets is None else list(row_offsets)
    req_tokens = [int(L) + max(offs) for L in req_lens]
    req_pages = [(t + PAGE - 1) // PAGE for t in req_tokens]
    n_pages = sum(req_pages)
    cap = max(req_pages) if bt_pages is None else bt_pages
    assert cap >= max(req_pages)
    perm = torch.randperm(n_pages, generator=g).to(torch.int32)
    bt = torch.zeros(B, cap, dtype=torch.int32)
    lens = torch.empty(B, dtype=torch.int32)
    p0 = 0
    for i in range(n_req):
        pages = perm[p0:p0 + req_pages[i]]
        p0 += req_pages[i]
        for j in range(group):
            bt[i * group + j, :req_pages[i]] = pages
            lens[i * group + j] = int(req_lens[i]) + offs[j]
    kv = build_kv(g, n_pages)
    return DecodeCase(name, q, w.float(), kv, lens, bt, group)


@dataclass
class PrefillCase:
    name: str
    q: torch.Tensor           # bf16 [rows, H, 128]
    w: torch.Tensor           # f32 [rows, H]
    kv: torch.Tensor          # uint8 [n_pages, 64, 1, 132]
    block_table: torch.Tensor  # int32 [n_pages]
    lens: torch.Tensor        # int32 [rows], causal: prefix + i + 1
    n_keys: int

    @property
    def rows(self):
        return self.q.shape[0]

    def slots(self):
        t = torch.arange(self.n_keys, dtype=torch.int64)
        return (self.block_table.long()[t // PAGE] * PAGE + t % PAGE).to(torch.int32)

    def tokens_scored(self):
        return int(self.lens.long().sum())


def prefill_case(seed, n_q, prefix, heads=64, dist="normal", name="prefill"):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n_q, heads, HEAD_DIM, generator=g).to(torch.bfloat16)
    w = torch.randn(n_q, heads, generator=g) * math.sqrt(1.0 / 8.0)
    n_keys = prefix + n_q
    n_pages = (n_keys + PAGE - 1) // PAGE
    bt = torch.randperm(n_pages, generator=g).to(torch.int32)
    kv = build_kv(g, n_pages, dist)
    lens = (prefix + 1 + torch.arange(n_q)).to(torch.int32)
    return PrefillCase(name, q, w.float(), kv, bt, lens, n_keys)


# ---------------------------------------------------------------------------------------------
# The workloads at full size.

def decode_1x4k():
    return decode_case(1, [4096], group=1, name="decode_1x4k")


def decode_32x16k():
    return decode_case(2, [16384] * 32, group=1, name="decode_32x16k")


def decode_mtp64(n_req=64, lo=2048, hi=65536, seed=3):
    g = torch.Generator().manual_seed(seed + 1000)
    L = torch.randint(lo, hi + 1, (n_req,), generator=g).tolist()
    cap = (hi + 1 + PAGE - 1) // PAGE
    return decode_case(seed, L, group=2, bt_pages=cap, name="decode_mtp64")


def prefill_8k_64k():
    return prefill_case(4, 8192, 65536, name="prefill_8k_64k")


def prefill_16k_128k():
    return prefill_case(5, 16384, 131072, dist="student_t4", name="prefill_16k_128k")


@dataclass
class MlaDequantCase:
    name: str
    cache: torch.Tensor  # uint8 [pool, 1, 656]: [512 fp8 | 4 x f32 scale | 64 x bf16 rope]
    slots: torch.Tensor  # int32 [n]

    @property
    def tokens(self):
        return self.slots.shape[0]


def mla_dequant_case(seed, n_tok, pool=1 << 19, name="dequant_mla"):
    """A pool of MLA slots: fp8 codes drawn uniformly over the non-NaN codes, per-group scales in
    [1e-3, 1.1e-2), bf16 rope ~ N(0,1); n_tok slots drawn uniformly from the pool (repeats
    allowed, as the reference's microbenchmark draws them)."""
    g = torch.Generator().manual_seed(seed)
    codes = torch.randint(0, 254, (pool, 512), generator=g, dtype=torch.int32)
    codes = (codes + (codes >= 0x7F).int()).to(torch.uint8)  # skip 0x7F; 0xFF is never drawn
    scale = torch.rand(pool, 4, generator=g) * 0.01 + 1e-3
    rope = torch.randn(pool, 64, generator=g).to(torch.bfloat16)
    cache = torch.cat([codes, scale.view(torch.uint8).view(pool, 16), rope.view(torch.uint8).view(pool, 128)], 1)
    slots = torch.randint(0, pool, (n_tok,), generator=g, dtype=torch.int32)
    return MlaDequantCase(name, cache.contiguous().view(pool, 1, 656), slots)


@dataclass
class KDequantCase:
    name: str
    kv: torch.Tensor     # uint8 [n_pages, 64, 1, 132]
    slots: torch.Tensor  # int32 [n]

    @property
    def tokens(self):
        return self.slots.shape[0]


def dequant_mla_393k():
    return mla_dequant_case(6, 392832, name="dequant_mla_393k")


def dequant_mla_131k():
    return mla_dequant_case(6, 131072, name="dequant_mla_131k")


def dequant_k_74k():
    c = prefill_8k_64k()
    return KDequantCase("dequant_k_74k", c.kv, c.slots())


# ---------------------------------------------------------------------------------------------
# Top-k score distributions (hcu_ops/tests/topk_lib.py:8-51).

TOPK_DISTS = ("pos", "sparse30", "sparse2", "relu_sum", "mixed", "ties", "zeros", "neg", "narrow", "const")


def topk_scores(B, L, dist, W=None, ragged=False, seed=0):
    """(score f32 [B, W] with NaN at masked-out slots, mask int16 [B, ceil(W/16)],
    lengths int32 [B], page_table int32 [B, W] = arange + 7 + 1e6 * row)."""
    g = torch.Generator().manual_seed(seed)
    W = W or L
    r = lambda *s: torch.rand(*s, generator=g)
    if dist == "pos":
        x = r(B, W) * 10
    elif dist == "sparse30":
        x = r(B, W) * 10
        x[r(B, W) > 0.3] = 0
    elif dist == "sparse2":  # fast-path regime: positives < 2048 < positives + zeros
        x = r(B, W) * 10
        x[r(B, W) > 1500.0 / W] = 0
    elif dist == "relu_sum":
        n = torch.randn(B, W, 8, generator=g)
        x = (torch.relu(n) * (r(8) - 0.3)).sum(-1)
    elif dist == "mixed":
        x = torch.randn(B, W, generator=g)
    elif dist == "ties":
        x = torch.randint(0, 50, (B, W), generator=g).float() / 4
    elif dist == "zeros":
        x = torch.zeros(B, W)
    elif dist == "neg":
        x = -r(B, W)
        x[r(B, W) > 0.5] = 0
    elif dist == "narrow":  # one 12-bit key bin: the candidate lists overflow
        x = 1.0 + r(B, W) * 1e-3
    elif dist == "const":
        x = torch.full((B, W), 0.5)
    else:
        raise ValueError(dist)
    x = x.float().contiguous()
    nz = x != 0
    pad = (-W) % 16
    if pad:
        nz = torch.cat([nz, torch.zeros(B, pad, dtype=torch.bool)], 1)
    w16 = torch.tensor([1 << i for i in range(16)], dtype=torch.int32)
    bits = (nz.view(B, -1, 16).to(torch.int32) * w16).sum(-1, dtype=torch.int32)
    mask = torch.where(bits > 32767, bits - 65536, bits).to(torch.int16).contiguous()
    x = torch.where(x == 0, torch.full_like(x, float("nan")), x)
    if ragged:
        lengths = (L - torch.arange(B) * 37 - 3).clamp(min=1).to(torch.int32)
    else:
        lengths = torch.full((B,), L, dtype=torch.int32)
    pt = (torch.arange(W, dtype=torch.int32).unsqueeze(0).repeat(B, 1)
          + 7 + 1000000 * torch.arange(B, dtype=torch.int32).unsqueeze(1)).contiguous()
    return x, mask, lengths, pt
