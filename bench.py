"""Benchmark of the MI355X DSA indexer path (one GPU).

A step is one pass of the indexer over one batch with every input resident in HBM:
  decode   bf16 q -> fp8 quant -> paged fp8 MQA logits (+ the paired top-k's workspace) -> top-2048 +
           page-table remap
  prefill  bf16 q -> fp8 quant -> causal fp8 MQA logits over the paged K in 4096-row slabs, each
           slab's top-2048 + remap behind it (hcu_ops.prefill_indexer)
Steps are captured in a hipGraph (--steps-per-graph of them per graph, as a serving loop
captures the indexer inside its model step) and replayed.  The step graph first runs untimed
for --settle-ms (the GPU raises its clocks only after some milliseconds of load; a serving loop
runs continuously), then W more steps warm up, then exactly K steps are timed between two
synchronisations.  value = indexer K-tokens scored per second (tokens scored =
sum over query rows of the keys that row scores).

The JSON line also carries
  roofline      the dominant kernel (the logits kernel) timed live with HIP events on its launch
                stream over graph replays of that kernel alone, against its algorithmic bytes
                (decode: HBM) or flops (prefill: fp8 MFMA);
  path_roofline the whole step's algorithmic bytes / flops against the same peak;
  cpu_baseline  the oracle's torch-CPU restatement (dequant -> fp32 matmul -> relu*w -> sum ->
                *scale -> kthvalue top-2048 -> gather) timed on a bounded sample of the same
                workload on this host's cores.

The default line (decode_mtp64, the quoted decode configuration, as `value`) also holds one object
per other configuration -- prefill_8k_64k (the prefill headline), prefill_16k_128k, decode_32x16k,
decode_1x4k -- and one each for dequant_k_74k (the 132-B indexer K dequant) and dequant_mla_393k
(the 656-B MLA dequant), each with its own step time, roofline and CPU baseline.  Every workload
also reports the median / min / max of 20 individually timed graph replays; a prefill step's
time is that median (its roofline is taken over every slab's logits launch).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload decode_mtp64]
"""
import argparse
import json
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sglang0.5.18-opt_amd"))
sys.path.insert(0, ROOT)
sys.path.insert(0, os.path.join(ROOT, "tests"))  # the seeded workload generators

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP8_PEAK_TFLOPS = 5000.0     # MI355X dense fp8 MFMA
METRIC = "indexer K-tokens scored/sec (logits+top2048) at 64K ctx"

WORKLOADS = {
    "decode_1x4k": "decode, 1 request x 1 row, 4096-token paged fp8 K, 64 heads x 128",
    "decode_32x16k": "decode, 32 requests x 1 row, 16384 tokens each, 64 heads x 128, fp8 paged K (page 64)",
    "decode_mtp64": "decode MTP verify, 64 requests x 2 rows, ctx U[2048, 65536], 64 heads x 128, "
                    "fp8 paged K (page 64), shuffled pages",
    "prefill_8k_64k": "chunked prefill, 8192 query rows over a 65536-token cached prefix (73728 keys, causal), "
                      "64 heads x 128",
    "prefill_16k_128k": "long prefill, 16384 query rows over 147456 keys (causal) in 4096-row slabs, "
                        "Student-t(4) K, 64 heads x 128",
    "dequant_mla_393k": "MLA K-cache dequant, 392832 tokens gathered at random from 2^19 656-B slots -> bf16 [n, 576]",
    "dequant_mla_131k": "MLA K-cache dequant, 131072 tokens gathered at random from 2^19 656-B slots -> bf16 [n, 576]",
    "dequant_k_74k": "indexer K dequant, the 73728 keys of prefill_8k_64k from the 132-B paged cache -> bf16 [n, 128]",
    "reference_shapes": "per-call times at the shapes the reference publishes numbers for (BW1100, 32 heads): "
                        "logits G=6 / G=1 at 16K-128K, split top-2048 of 6-192 relu_sum rows in a 1M-wide block",
}
DEQUANT_METRIC = "paged K-cache dequant, algorithmic GB/s (slot index + slot bytes read, bf16 written)"


def profiled_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` from its committed rocprofv3 PMC summary
    (FETCH_SIZE + WRITE_SIZE, each scaled by the counter's reading for a copy of known size),
    or None when no summary exists."""
    path = os.path.join(ROOT, "profiles", f"{kernel}.{workload}.md")
    try:
        for line in open(path):
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1]), os.path.relpath(path, ROOT)
    except OSError:
        pass
    return None, None


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or "unknown"


# ---------------------------------------------------------------------------------------------
# Decode

class DecodeStep:
    def __init__(self, case, dev, blocks=False):
        """blocks: the top-k transform reads the block table (sparse_mask_topk_transform_blocks)
        instead of its page_table_size_1 expansion (the reference's caller form, the default)."""
        import torch
        import hcu_ops
        self.h = hcu_ops
        self.case = case
        self.blocks = blocks
        g = lambda t: t.to(dev)
        self.q, self.w, self.kv = g(case.q), g(case.w), g(case.kv)
        self.lens, self.bt = g(case.context_lens), g(case.block_table)
        self.pt = g(case.page_table_1())
        self.cu = torch.arange(case.rows + 1, dtype=torch.int32, device=dev)
        self.out = None

    def __call__(self):
        h, c = self.h, self.case
        q8, w = h.quant_q_fp8(self.q, self.w)
        logits, mask = h.mqa_logits(q8.unsqueeze(1), self.kv, w, self.lens, self.bt, c.width, c.group,
                                    hist_lens=self.lens)
        if self.blocks:
            self.out = h.sparse_mask_topk_transform_blocks(logits, mask, self.lens, self.bt, self.cu)
        else:
            self.out = h.sparse_mask_topk_transform(logits, mask, self.lens, self.pt, self.cu)
        return self.out

    def logits_only(self, hist=False):
        """The dominant kernel alone (the step's launch shape, q already quantised); hist=True also
        prepares the paired top-k's workspace as inside the step."""
        if not hasattr(self, "_q8"):
            self._q8, self._w8 = self.h.quant_q_fp8(self.q, self.w)
        c = self.case
        return self.h.mqa_logits(self._q8.unsqueeze(1), self.kv, self._w8, self.lens, self.bt, c.width, c.group,
                                 hist_lens=self.lens if hist else None)

    def tokens(self):
        return self.case.tokens_scored()

    def logits_bytes(self):
        """Algorithmic HBM bytes of one logits launch: each request's K tokens once (132 B),
        q8 + w per row, block table entries, logits written for t < len, mask words written."""
        c = self.case
        L = c.context_lens.clamp(max=c.width).long()
        req_tokens = L.view(-1, c.group).max(1).values
        H = c.q.shape[1]
        return int(req_tokens.sum() * 132 + c.rows * H * (128 + 4) + ((req_tokens + 63) // 64).sum() * 4
                   + L.sum() * 4 + c.rows * (c.width // 16) * 2)

    def path_bytes(self):
        """Algorithmic bytes of the step (the decode byte formula): K once per request, q bf16,
        w, block table, logits written and read, mask written and read, page-table gather + out."""
        c = self.case
        L = c.context_lens.clamp(max=c.width).long()
        req_tokens = L.view(-1, c.group).max(1).values
        H = c.q.shape[1]
        return int(req_tokens.sum() * 132 + c.rows * H * 128 * 2 + c.rows * H * 4 + ((req_tokens + 63) // 64).sum() * 4
                   + 2 * L.sum() * 4 + 2 * (L.sum() // 16) * 2 + c.rows * 2048 * 8)


def decode_cpu_baseline(case, budget_s):
    """Oracle's torch-CPU indexer on whole query rows, in row order, until budget_s of CPU time."""
    import numpy as np
    import torch
    from oracle import indexer as O
    from oracle.fp8 import fp8_decode
    q8, w = O.quant_q(case.q.view(torch.int16).numpy().view(np.uint16), case.w.numpy())
    kv = case.kv.view(case.kv.shape[0], -1).numpy()
    tokens = 0
    rows = 0
    lens = case.context_lens.clamp(max=case.width).numpy()
    t0 = time.perf_counter()
    for g0 in range(0, case.rows, case.group):
        # paged K gather + dequant once per request, shared by the request's rows
        n = int(lens[g0:g0 + case.group].max())
        slots = O.slots_of(case.block_table.numpy()[g0], n)
        codes, sc = O.kv_tokens(kv, slots)
        kf, st, sl = torch.from_numpy(fp8_decode(codes)), torch.from_numpy(sc), torch.from_numpy(slots.astype(np.int32))
        for r in range(g0, g0 + case.group):
            L = int(lens[r])
            O.cpu_indexer_row_torch(torch.from_numpy(fp8_decode(q8[r])), torch.from_numpy(w[r]), kf[:L], st[:L],
                                    sl[:L])
            tokens += L
            rows += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return tokens / 1e3 / dt, f"{rows} of {case.rows} query rows ({tokens} keys scored) in {dt:.1f} s"


# ---------------------------------------------------------------------------------------------
# Prefill

class PrefillStep:
    SLAB = 4096

    def __init__(self, case, dev):
        import torch
        import hcu_ops
        self.h = hcu_ops
        self.case = case
        g = lambda t: t.to(dev)
        self.q, self.w, self.kv, self.bt, self.lens = g(case.q), g(case.w), g(case.kv), g(case.block_table), \
            g(case.lens)
        self.pt = g(case.slots())
        self.width = case.n_keys
        self.out = torch.empty(case.rows, 2048, dtype=torch.int32, device=dev)
        self.slab = min(self.SLAB, case.rows)

    def __call__(self):
        # the logits kernel reads the paged fp8 K directly, so no dequantised copy of K is made;
        # logits in 4096-row slabs (the budget of 4096 rows of f32 logits), each slab's top-2048
        # right behind it
        h = self.h
        q8, w = h.quant_q_fp8(self.q, self.w)
        h.prefill_indexer(q8, w, self.kv, self.bt, self.lens, self.width, self.pt,
                          memory_budget_bytes=self.slab * self.width * 4, max_slab_rows=self.slab, out=self.out)
        return self.out

    def slabs(self):
        return [(r0, min(r0 + self.slab, self.case.rows)) for r0 in range(0, self.case.rows, self.slab)]

    def logits_only(self, slab=None):
        """The logits launches of every slab (slab=i: of slab i alone), q already quantised; each
        slab's logits buffer is dropped before the next is made, as in the step."""
        if not hasattr(self, "_q8"):
            self._q8, self._w8 = self.h.quant_q_fp8(self.q, self.w)
        for i, (r0, r1) in enumerate(self.slabs()):
            if slab is None or slab == i:
                self.h.mqa_logits_prefill(self._q8[r0:r1], self._w8[r0:r1], self.kv, self.bt, self.lens[r0:r1],
                                          self.width)

    def topk_us(self, torch):
        """Live duration of each slab's top-k launch (the step's: one CTA per row of the slab's
        logits, the request's page-table row shared), in graphs of 5 launches on logits made once
        beforehand; with the algorithmic bytes of each (scores read once, 2048 page-table entries
        gathered and written per row)."""
        if not hasattr(self, "_q8"):
            self._q8, self._w8 = self.h.quant_q_fp8(self.q, self.w)
        pt = self.pt.unsqueeze(0)
        res = []
        for r0, r1 in self.slabs():
            lg = self.h.mqa_logits_prefill(self._q8[r0:r1], self._w8[r0:r1], self.kv, self.bt, self.lens[r0:r1],
                                           self.width)
            lens = self.lens[r0:r1]
            cu = torch.tensor([0, r1 - r0], dtype=torch.int32, device=lg.device)
            out = torch.empty(r1 - r0, 2048, dtype=torch.int32, device=lg.device)
            ms = kernel_time_ms(lambda: self.h.topk_transform(lg, lens, pt, cu, out=out), torch, reps=5, rounds=3,
                                settle_ms=20.0)
            nbytes = int(self.case.lens[r0:r1].clamp(max=self.width).long().sum()) * 4 + (r1 - r0) * 2048 * 8
            res.append((ms * 1e3, nbytes))
            del lg, out
        return res

    def tokens(self):
        return self.case.tokens_scored()

    def logits_flops(self, slab=None):
        """fp8 MFMA flops of the logits launches (every slab, or slab i): 2 * H * 128 per (row, key)."""
        H = self.case.q.shape[1]
        rows = [(r0, r1) for i, (r0, r1) in enumerate(self.slabs()) if slab is None or slab == i]
        return 2 * H * 128 * sum(int(self.case.lens[r0:r1].long().sum()) for r0, r1 in rows)

    def path_flops(self):
        H = self.case.q.shape[1]
        return 2 * H * 128 * self.case.tokens_scored()


def prefill_cpu_baseline(case, budget_s):
    """Oracle's torch-CPU indexer on query rows spread over the causal range (every k-th row)
    until budget_s; extrapolated per scored key."""
    import numpy as np
    import torch
    from oracle import indexer as O
    from oracle.fp8 import fp8_decode
    kv = case.kv.view(case.kv.shape[0], -1).numpy()
    order = np.concatenate([np.arange(0, case.rows, 97), np.arange(48, case.rows, 97)])
    tokens = 0
    rows = 0
    t0 = time.perf_counter()
    slots = O.slots_of(case.block_table.numpy(), case.n_keys)  # paged K dequant, once per chunk
    codes, sc = O.kv_tokens(kv, slots)
    kf = torch.from_numpy(fp8_decode(codes))
    st = torch.from_numpy(sc)
    sl = torch.from_numpy(slots.astype(np.int32))
    for r in order:
        q8, w = O.quant_q(case.q[r:r + 1].view(torch.int16).numpy().view(np.uint16), case.w[r:r + 1].numpy())
        L = int(case.lens[r])
        O.cpu_indexer_row_torch(torch.from_numpy(fp8_decode(q8[0])), torch.from_numpy(w[0]), kf[:L], st[:L], sl[:L])
        tokens += L
        rows += 1
        if time.perf_counter() - t0 > budget_s:
            break
    dt = time.perf_counter() - t0
    return tokens / 1e3 / dt, (f"{rows} of {case.rows} query rows spread over the causal range ({tokens} keys "
                               f"scored) in {dt:.1f} s, extrapolated per scored key")


# ---------------------------------------------------------------------------------------------
# Dequant (the prefill path's gather of K to bf16, and the MLA cache's)

class DequantStep:
    def __init__(self, case, dev):
        import hcu_ops
        self.h = hcu_ops
        self.case = case
        self.mla = hasattr(case, "cache")
        self.src = (case.cache if self.mla else case.kv).to(dev)
        self.slots = case.slots.to(dev)
        self.kernel = "dequant_mla_kernel" if self.mla else "dequant_k_kernel"
        # per token: slot index + the slot's bytes read, bf16 row written
        self.tok_bytes = 4 + (656 + 576 * 2 if self.mla else 132 + 128 * 2)

    def __call__(self):
        if self.mla:
            return self.h.dequantize_k_cache_paged(self.src, self.slots)
        return self.h.dequant_k_paged(self.src, self.slots)

    def bytes(self):
        return self.case.tokens * self.tok_bytes


def dequant_cpu_baseline(case, budget_s, tok_bytes, torch):
    """The oracle's torch-CPU dequant (its numpy closed form restated on torch's intra-op threads)
    over consecutive chunks of the slot list, repeated until budget_s."""
    from oracle import indexer as O
    mla = hasattr(case, "cache")
    src = case.cache.view(case.cache.shape[0], -1) if mla else case.kv.view(case.kv.shape[0], -1)
    slots = case.slots
    threads, _ = cpu_threads(torch)
    done = 0
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and (done < slots.shape[0] or time.perf_counter() - t0 < 1.0):
        i = done % slots.shape[0]
        s = slots[i:i + 65536]
        O.cpu_dequant_torch(src, s, mla)
        done += s.shape[0]
    dt = time.perf_counter() - t0
    return (done * tok_bytes / dt / 1e9, threads,
            f"{done} tokens of the {slots.shape[0]}-slot list in {dt:.1f} s (torch CPU, {threads} threads)")


# ---------------------------------------------------------------------------------------------

def graph_of(fn, torch, n=1):
    """hipGraph of n back-to-back calls of fn (after two eager warm-up calls)."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(n):
            fn()
    torch.cuda.synchronize()
    return g


def settle(g, torch, ms):
    """Replays graph g untimed for about `ms` milliseconds of GPU time."""
    if ms <= 0:
        return
    t0 = time.perf_counter()
    while (time.perf_counter() - t0) * 1e3 < ms:
        for _ in range(4):
            g.replay()
        torch.cuda.synchronize()


def kernel_time_ms(fn, torch, reps=20, rounds=5, settle_ms=50.0):
    """Average duration of fn's launch: a graph of `reps` back-to-back launches, replayed untimed
    for settle_ms, then timed with HIP events on the current stream; median over rounds."""
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        fn()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for _ in range(reps):
            fn()
    for _ in range(3):  # first replays of a new graph run slow (fresh buffers)
        g.replay()
    torch.cuda.synchronize()
    settle(g, torch, settle_ms)
    times = []
    for _ in range(rounds):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) / reps)
    times.sort()
    return times[len(times) // 2]


def mfma_ceiling(torch, dev, ctas=2048, iters=2000, reps=5):
    """Measured fp8 MFMA ceilings of this chip (the library's MFMA probe on random non-NaN fp8
    codes, HIP events on the launch stream, median of `reps` launches after a warm-up one): MFMA
    alone, and MFMA with 4, 8 (the logits epilogue's count) and 16 VALU operations of the
    epilogue's kind per MFMA; plus the shader clock."""
    import hcu_ops
    g = torch.Generator().manual_seed(0)
    codes = torch.randint(0, 254, (4 * 16384,), generator=g, dtype=torch.int32)
    codes = (codes + (codes >= 0x7F).int()).to(torch.uint8)  # skips 0x7F; 0xFF is never drawn (NaNs)
    ops = codes.view(torch.int32).to(dev)
    flop = ctas * 4 * iters * 8 * 65536.0
    out = {"unit": "TFLOP/s", "probe": f"{ctas} CTAs x 4 waves x {iters} x 8 v_mfma_f32_16x16x128_f8f6f4, "
                                      "random fp8 operands"}
    for name, epi in (("mfma_only", 0), ("mfma_with_4_valu", 4), ("mfma_with_epilogue_valu", 8),
                      ("mfma_with_16_valu", 16)):
        times = []
        clocks = None
        for _ in range(reps + 1):
            a = torch.cuda.Event(enable_timing=True)
            b = torch.cuda.Event(enable_timing=True)
            a.record()
            _, clocks = hcu_ops._C.mfma_fp8_probe(ops, ctas, iters, epi)
            b.record()
            b.synchronize()
            times.append(a.elapsed_time(b))
        times = sorted(times[1:])
        ms = times[len(times) // 2]
        out[name] = round(flop / (ms / 1e3) / 1e12, 1)
        c = clocks.cpu().tolist()
        if c[1] > 0:
            out[f"{name}_shader_clock_ghz"] = round(c[0] / c[1] * 0.1, 3)
    return out


def cpu_threads(torch):
    """The CPU baseline's threads: torch.set_num_threads(os.cpu_count()), as specified for the
    baseline; the CPUs the process may run on are reported beside it."""
    n = os.cpu_count() or 1
    torch.set_num_threads(n)
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = n
    return torch.get_num_threads(), avail


def replay_stats(g, torch, per, n):
    """n replays of step graph g (per steps each), each timed alone with HIP events on the current
    stream: (median, min, max) ms per step."""
    times = []
    for _ in range(n):
        a = torch.cuda.Event(enable_timing=True)
        b = torch.cuda.Event(enable_timing=True)
        a.record()
        g.replay()
        b.record()
        b.synchronize()
        times.append(a.elapsed_time(b) / per)
    times.sort()
    return times[len(times) // 2], times[0], times[-1]


def timed_steps(step, args, torch):
    """ms per step: the step captured `steps_per_graph` to a hipGraph (as a serving loop captures the
    indexer inside its model step), replayed untimed for settle_ms, then W warm-up steps, then
    exactly K timed steps between two synchronisations (full graphs, then single-step graphs)."""
    per = max(1, min(args.steps_per_graph, args.steps))
    g = graph_of(step, torch, per)
    g1 = graph_of(step, torch, 1) if args.steps % per or args.warmup % per else None
    settle(g, torch, args.settle_ms)
    for _ in range(args.warmup // per):
        g.replay()
    for _ in range(args.warmup % per):
        g1.replay()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record()
    for _ in range(args.steps // per):
        g.replay()
    for _ in range(args.steps % per):
        g1.replay()
    end.record()
    torch.cuda.synchronize()
    med, lo, hi = replay_stats(g, torch, per, args.replays)
    stats = {"replays": args.replays, "steps_per_replay": per, "median_ms_per_step": round(med, 5),
             "min_ms_per_step": round(lo, 5), "max_ms_per_step": round(hi, 5)}
    return start.elapsed_time(end) / args.steps, per, stats


def run_indexer(name, args, torch, dev, steps=None):
    """One indexer workload: the timed step, its dominant kernel's roofline, the path roofline and
    the CPU baseline, as the fields of a JSON line."""
    import workloads as wl
    t0 = time.perf_counter()
    case = getattr(wl, name)()
    log(f"built {name} inputs on the CPU in {time.perf_counter() - t0:.1f} s")
    decode = name.startswith("decode")
    step = DecodeStep(case, dev) if decode else PrefillStep(case, dev)
    torch.cuda.synchronize()
    if steps is not None:
        args = argparse.Namespace(**{**vars(args), **steps})
    ms, per, stats = timed_steps(step, args, torch)
    timing = f"{args.steps} steps timed together between two synchronisations"
    if not decode:
        # a prefill step is milliseconds long: the median of the individually timed graph replays
        # (hipEvents around each), with their spread beside it
        ms = stats["median_ms_per_step"]
        timing = f"median of {args.replays} individually timed hipGraph replays (hipEvents)"
    tokens = step.tokens()
    value = tokens / 1e3 / (ms / 1e3)
    log(f"{name}: {timing}: {ms * 1e3:.1f} us/step, {value:.4g} K-tokens/s (replays {stats})")
    if decode:
        # the launch as the step makes it: logits + the paired top-k's workspace prepared
        k_ms = kernel_time_ms(lambda: step.logits_only(hist=True), torch)
        k0_ms = kernel_time_ms(step.logits_only, torch)
        kb = step.logits_bytes()
        achieved = kb / (k_ms / 1e3) / 1e9
        traffic, tsrc = profiled_traffic("mqa_logits_decode_kernel", name)
        roofline = {"bound": "hbm", "kernel": "mqa_logits_decode_kernel", "achieved": round(achieved, 1),
                    "peak": HBM_PEAK_GBS, "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4),
                    "traffic": traffic, "traffic_source": tsrc, "algorithmic_bytes": kb,
                    "kernel_us": round(k_ms * 1e3, 2), "without_topk_workspace_us": round(k0_ms * 1e3, 2)}
        pb = step.path_bytes()
        pa = pb / (ms / 1e3) / 1e9
        path = {"bound": "hbm", "achieved": round(pa, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(pa / HBM_PEAK_GBS, 4), "algorithmic_bytes": pb}
    else:
        # every slab's logits launch (graphs of 20 passes over all slabs): flops over all of them
        # against their summed duration, plus each slab alone
        k_ms = kernel_time_ms(step.logits_only, torch)
        kf = step.logits_flops()
        achieved = kf / (k_ms / 1e3) / 1e12
        per_slab = []
        for i in range(len(step.slabs())):
            s_ms = kernel_time_ms(lambda i=i: step.logits_only(slab=i), torch, rounds=3, settle_ms=20.0)
            per_slab.append({"kernel_us": round(s_ms * 1e3, 2),
                             "frac": round(step.logits_flops(i) / (s_ms / 1e3) / 1e12 / FP8_PEAK_TFLOPS, 4)})
        # prefill runs the paged logits kernel with 8 query rows per CTA
        traffic, tsrc = profiled_traffic("mqa_logits_decode_kernel", name)
        roofline = {"bound": "mfma", "kernel": "mqa_logits_decode_kernel", "achieved": round(achieved, 1),
                    "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s", "frac": round(achieved / FP8_PEAK_TFLOPS, 4),
                    "traffic": traffic, "traffic_source": tsrc, "algorithmic_flops": kf,
                    "launches": len(per_slab), "kernel_us": round(k_ms * 1e3, 2),
                    "kernel_us_per_launch": round(k_ms * 1e3 / len(per_slab), 2), "slabs": per_slab}
        measured = mfma_ceiling(torch, dev)
        measured["logits_frac_of_mfma_only"] = round(achieved / measured["mfma_only"], 4)
        measured["logits_frac_of_mfma_with_epilogue_valu"] = round(achieved / measured["mfma_with_epilogue_valu"], 4)
        roofline["measured_ceiling"] = measured
        tk = step.topk_us(torch)
        tk_us = sum(u for u, _ in tk)
        tk_b = sum(b for _, b in tk)
        roofline["slab_topk"] = {"kernel": "topk_row_sampled_kernel", "us_per_slab": [round(u, 1) for u, _ in tk],
                                 "achieved_gbs": round(tk_b / (tk_us / 1e6) / 1e9, 1),
                                 "frac_of_hbm": round(tk_b / (tk_us / 1e6) / 1e9 / HBM_PEAK_GBS, 4),
                                 "algorithmic_bytes": tk_b}
        log(f"{name}: slab top-k {[round(u, 1) for u, _ in tk]} us")
        log(f"{name}: measured fp8 MFMA ceiling {measured['mfma_only']} TFLOP/s alone, "
            f"{measured['mfma_with_epilogue_valu']} with the epilogue's VALU work")
        pf = step.path_flops()
        pa = pf / (ms / 1e3) / 1e12
        path = {"bound": "mfma", "achieved": round(pa, 1), "peak": FP8_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(pa / FP8_PEAK_TFLOPS, 4), "algorithmic_flops": pf}
    log(f"{name}: logits kernel {k_ms * 1e3:.1f} us -> {roofline['achieved']} {roofline['unit']} "
        f"({roofline['frac']:.1%})")
    cpu = None
    if not args.no_cpu_baseline:
        threads, avail = cpu_threads(torch)
        v, sample = (decode_cpu_baseline if decode else prefill_cpu_baseline)(case, args.cpu_budget)
        cpu = {"value": round(v, 2), "unit": "K-tokens/s", "cores": threads, "cpus_available": avail,
               "kind": "port", "sample": sample, "cpu": cpu_model()}
        log(f"{name}: cpu baseline {v:.4g} K-tokens/s on {threads} threads ({sample})")
    config = {"workload": f"{name}: {WORKLOADS[name]}", "query_rows": int(case.rows),
              "tokens_scored_per_step": int(tokens), "graph": f"hipGraph of {per} steps per replay",
              "timing": timing, "settle_ms": args.settle_ms}
    if not decode:
        config["dequant"] = ("none in the step: the logits kernel reads the paged fp8 K directly, so the bf16 "
                             "copy of K that the configuration names is never made (dequant_k_74k times that "
                             "dequant on its own)")
    res = {"value": round(value, 1), "ms_per_step": round(ms, 5), "steps": args.steps, "warmup": args.warmup,
           "replays": stats, "config": config, "roofline": roofline, "path_roofline": path, "cpu_baseline": cpu}
    if decode:
        # the same step with the top-k's page-table transform reading the block table the logits already
        # use (dsa_topk_transform_blocks) instead of its page_table_size_1 expansion: same output
        del step
        bstep = DecodeStep(case, dev, blocks=True)
        b_ms, _, b_stats = timed_steps(bstep, args, torch)
        res["block_table_topk"] = {
            "value": round(tokens / 1e3 / (b_ms / 1e3), 1), "unit": "K-tokens/s", "ms_per_step": round(b_ms, 5),
            "replays": b_stats, "path_roofline_frac": round(bstep.path_bytes() / (b_ms / 1e3) / 1e9 / HBM_PEAK_GBS, 4),
            "note": "the step with hcu_ops.sparse_mask_topk_transform_blocks (the top-k reads the block table, 4 B "
                    "per 64 tokens, instead of page_table_size_1, 4 B per token); same output; value and "
                    "ms_per_step above use the reference's page_table_size_1 form"}
        log(f"{name}: with the block-table top-k {b_ms * 1e3:.1f} us/step")
    return res


def main(argv=None):
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=20, help="untimed steps right before the timed ones")
    ap.add_argument("--settle-ms", type=float, default=200.0,
                    help="untimed replays of the step graph first, so that the GPU clocks have settled")
    ap.add_argument("--workload", default="decode_mtp64", choices=sorted(WORKLOADS))
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work per workload")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-prefill", action="store_true",
                    help="the default decode_mtp64 line only (no objects for the other workloads)")
    ap.add_argument("--no-reference-shapes", action="store_true",
                    help="no reference_shapes object (the reference's published shapes) in the default line")
    ap.add_argument("--no-dequant", action="store_true", help="no dequant objects (dequant_k_74k, dequant_mla_393k) in the default line")
    ap.add_argument("--steps-per-graph", type=int, default=10, help="steps captured in one hipGraph")
    ap.add_argument("--replays", type=int, default=20,
                    help="individually timed replays of the step graph (median / min / max reported)")
    ap.add_argument("--copy-calibration-mib", type=int, default=0,
                    help="first run a plain device copy of this many MiB three times (the known-size kernel that "
                         "scales FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args(argv)
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py runs the indexer on one GPU only: this build has no multi-GPU path "
              "(decode rows shard by request with no exchange between GPUs). Use --gpus 1.", file=sys.stderr)
        return 2

    import torch
    import workloads as wl

    dev = torch.device("cuda:0")
    if args.copy_calibration_mib > 0:
        n = args.copy_calibration_mib << 18
        src = torch.ones(n, dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)  # one elementwise kernel: reads and writes n * 4 bytes
        torch.cuda.synchronize()
        log(f"copy calibration: 3 copies of {args.copy_calibration_mib} MiB")
        del src, dst
    if args.workload == "reference_shapes":
        print(json.dumps({"metric": "per-call time at the reference's published shapes", "unit": "us",
                          "higher_is_better": False, "n_gpus": 1, "data": "synthetic (seeded)",
                          **run_reference_shapes(torch, dev)}), flush=True)
        return 0
    if args.workload.startswith("dequant"):
        d = run_dequant(args.workload, args, torch, dev)
        line = {"metric": DEQUANT_METRIC, "value": d["value"], "unit": "GB/s", "n_gpus": 1, "steps": d["steps"],
                "warmup": d["warmup"], "ms_per_step": d["ms_per_step"], "higher_is_better": True, "scaling": "weak",
                "vs_baseline": None, "dtype": "fp8e4m3 -> bf16", "data": "synthetic (seeded, see tests/workloads.py)",
                "replays": d["replays"], "config": d["config"], "roofline": d["roofline"],
                "cpu_baseline": d["cpu_baseline"]}
        print(json.dumps(line), flush=True)
        return 0

    head = run_indexer(args.workload, args, torch, dev)
    line = {"metric": METRIC, "value": head["value"], "unit": "K-tokens/s", "n_gpus": 1, "steps": head["steps"],
            "warmup": head["warmup"], "ms_per_step": head["ms_per_step"], "higher_is_better": True,
            "scaling": "weak", "vs_baseline": None, "dtype": "fp8e4m3 (fp32 accumulate)",
            "data": "synthetic (seeded, see tests/workloads.py)", "config": head["config"],
            "replays": head["replays"], "roofline": head["roofline"], "path_roofline": head["path_roofline"],
            "cpu_baseline": head["cpu_baseline"]}
    if "block_table_topk" in head:
        line["block_table_topk"] = head["block_table_topk"]
    if args.workload == "decode_mtp64" and not args.no_prefill:
        # the second headline workload (the 64K-prefix chunked prefill) and the other configurations
        # in the same line, each with its own roofline and CPU baseline; prefill step counts sized
        # to about the same wall time
        few = {"steps": max(2, args.steps // 10), "warmup": max(1, args.warmup // 10), "steps_per_graph": 1,
               "replays": max(20, args.replays)}
        for name, steps in (("prefill_8k_64k", few), ("prefill_16k_128k", few), ("decode_32x16k", None),
                            ("decode_1x4k", None)):
            line[name] = {"metric": METRIC, "unit": "K-tokens/s", **run_indexer(name, args, torch, dev, steps=steps)}
        if not args.no_dequant:
            for name in ("dequant_k_74k", "dequant_mla_393k"):
                line[name] = {"metric": DEQUANT_METRIC, "unit": "GB/s", **run_dequant(name, args, torch, dev)}
        if not args.no_reference_shapes:
            line["reference_shapes"] = run_reference_shapes(torch, dev)
    print(json.dumps(line), flush=True)
    return 0


# The reference's published per-call times (Hygon BW1100, 32 indexer heads, graph replays):
# docs/GLM5.3_DCU_优化报告_20261023.md:395-403 (logits), docs/GLM5.3_opt2_README_20261023.md:158-162 (top-k).
REF_LOGITS = [  # (group, requests, context, BW1100 us)
    (6, 1, 16384, 21.6), (6, 4, 16384, 46.0), (6, 8, 16384, 73.8), (6, 1, 65536, 43.3), (6, 2, 65536, 71.5), (6, 4, 65536, 121.1), (6, 8, 65536, 210.9),
    (6, 1, 131072, 72.5), (6, 2, 131072, 121.0),
    (1, 1, 65536, 20.3), (1, 2, 65536, 21.8), (1, 4, 65536, 39.0), (1, 8, 65536, 73.0),
]
REF_TOPK = [  # (rows, context, BW1100 us), relu_sum rows in a 2^20-wide block
    (6, 16384, 48.0), (6, 65536, 49.0), (6, 131072, 61.0), (12, 65536, 61.0), (24, 65536, 88.0),
    (48, 65536, 116.0), (48, 131072, 211.0), (192, 16384, 127.0), (192, 65536, 341.0), (192, 131072, 626.0),
]


def run_reference_shapes(torch, dev):
    """MI355X per-call times at the reference's published shapes, beside its BW1100 numbers:
    the decode logits launch (32 heads, MTP groups of 6 rows with context L + j for row j, or single
    rows; paired with the top-k's workspace as in a step) and the split top-2048 + page-table
    transform of relu_sum rows (8 ReLU'd normals with one weight vector, the reference's test
    distribution) of ragged lengths L - 37 i - 3 in a 2^20-wide block.  Context only: the
    reference's hardware and head count differ."""
    import hcu_ops as h
    import workloads as wl
    logits = []
    for group, n_req, L, ref_us in REF_LOGITS:
        case = wl.decode_case(900 + group * 10 + n_req, [L] * n_req, group=group, heads=32)
        g = lambda t: t.to(dev)
        q8, w = h.quant_q_fp8(g(case.q), g(case.w))
        kv, lens, bt = g(case.kv), g(case.context_lens), g(case.block_table)
        ms = kernel_time_ms(lambda: h.mqa_logits(q8.unsqueeze(1), kv, w, lens, bt, case.width, group, hist_lens=lens),
                            torch, reps=10, rounds=5, settle_ms=20.0)
        logits.append({"group": group, "requests": n_req, "context": L, "mi355x_us": round(ms * 1e3, 1),
                       "bw1100_us": ref_us})
        del case, q8, w, kv, lens, bt
    topk = []
    W = 1 << 20
    gen = torch.Generator(device=dev)
    for rows, L, ref_us in REF_TOPK:
        gen.manual_seed(rows * 7 + L)
        c = torch.rand(8, generator=gen, device=dev) - 0.3
        x = torch.full((rows, W), float("nan"), device=dev)
        for r in range(rows):
            x[r, :L] = (torch.relu(torch.randn(L, 8, generator=gen, device=dev)) * c).sum(-1)
        nz = ~torch.isnan(x) & (x != 0)
        x = torch.where(nz, x, torch.full_like(x, float("nan")))
        w16 = (1 << torch.arange(16, device=dev, dtype=torch.int32))
        bits = (nz.view(rows, -1, 16).to(torch.int32) * w16).sum(-1, dtype=torch.int32)
        mask = torch.where(bits > 32767, bits - 65536, bits).to(torch.int16).contiguous()
        del nz, bits
        lengths = (L - torch.arange(rows, device=dev) * 37 - 3).clamp(min=1).to(torch.int32)
        pt = (torch.arange(W, dtype=torch.int32, device=dev).unsqueeze(0) + 7
              + 1000000 * torch.arange(rows, dtype=torch.int32, device=dev).unsqueeze(1)).contiguous()
        cu = torch.arange(rows + 1, dtype=torch.int32, device=dev)
        ms = kernel_time_ms(lambda: h.sparse_mask_topk_transform(x, mask, lengths, pt, cu), torch, reps=10, rounds=5,
                            settle_ms=20.0)
        topk.append({"rows": rows, "context": L, "width": W, "mi355x_us": round(ms * 1e3, 1), "bw1100_us": ref_us})
        del x, mask, pt
        torch.cuda.empty_cache()
    log(f"reference shapes: logits {[(d['group'], d['requests'], d['context'], d['mi355x_us']) for d in logits]}")
    log(f"reference shapes: top-k {[(d['rows'], d['context'], d['mi355x_us']) for d in topk]}")
    return {"logits_32_heads": logits, "topk_2048_relu_sum_1m_wide": topk,
            "note": "per call, graphs of 10 launches, median of 5; MI355X with this build beside the reference's "
                    "published BW1100 (gfx938, 64 CUs) numbers for its hcu kernels; context, not a target"}


def run_dequant(name, args, torch, dev):
    """One dequant workload (a step is one dequant launch) as the fields of a JSON line."""
    import workloads as wl
    t0 = time.perf_counter()
    case = getattr(wl, name)()
    log(f"built {name} inputs on the CPU in {time.perf_counter() - t0:.1f} s")
    step = DequantStep(case, dev)
    torch.cuda.synchronize()
    ms, per, stats = timed_steps(step, args, torch)
    nb = step.bytes()
    value = nb / (ms / 1e3) / 1e9
    k_ms = kernel_time_ms(step, torch)
    achieved = nb / (k_ms / 1e3) / 1e9
    log(f"timed {args.steps} launches: {ms * 1e3:.1f} us each, {value:.1f} GB/s; graph of 20 alone {k_ms * 1e3:.1f} us")
    traffic, tsrc = profiled_traffic(step.kernel, name)
    roofline = {"bound": "hbm", "kernel": step.kernel, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic, "traffic_source": tsrc,
                "algorithmic_bytes": nb, "kernel_us": round(k_ms * 1e3, 2)}
    cpu = None
    if not args.no_cpu_baseline:
        v, threads, sample = dequant_cpu_baseline(case, min(args.cpu_budget, 5.0), step.tok_bytes, torch)
        cpu = {"value": round(v, 3), "unit": "GB/s", "cores": threads, "kind": "port", "sample": sample,
               "cpu": cpu_model()}
        log(f"cpu baseline {v:.3g} GB/s ({sample})")
    return {"value": round(value, 1), "ms_per_step": round(ms, 5), "steps": args.steps, "warmup": args.warmup,
            "replays": stats,
            "config": {"workload": f"{name}: {WORKLOADS[name]}", "tokens": int(case.tokens),
                       "bytes_per_token": step.tok_bytes, "graph": f"hipGraph of {per} launches per replay",
                       "settle_ms": args.settle_ms},
            "roofline": roofline, "cpu_baseline": cpu}


if __name__ == "__main__":
    sys.exit(main())
