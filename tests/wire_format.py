"""The top-k's output as a sparse-MLA consumer reads it, and a small consumer of it (test helpers).

Wire format (reference hcu_ops/csrc/sparse_mask_topk.cu:1-22,166-169,301-348; the caller returns the
tensor to the sparse attention as is, diffs/round2/layers_attention_dsa_dsa_indexer_metadata.py.diff:27-32): int32
[rows, 2048], row-contiguous.  Row r holds min(len_r, 2048) slot ids followed by -1 pads.  A slot
id is the page-table entry of the selected token, for the paged K cache slot = bt[t / 64] * 64 +
t % 64 (sparse_mask_topk.cu:348; the block-table form of page_table_size_1).  A row of at most
2048 tokens is its first len_r slots in token order; a longer row lists the tokens whose key is
above the threshold in ascending token order, then the ties at the threshold in ascending token
order, so its token sequence is at most two ascending runs.

The consumer is the sparse decode attention of MLA over those ids (flash_mla's sparse kernels:
q [H, 576] against the 576-dim bf16 K of each listed slot, softmax over the listed slots, output
the probability-weighted first 512 dims; ids of -1 take no part).  flash_mla is not available
here, so the consumer is this restatement, which the CPU tests pin against a dense masked
attention."""
import numpy as np

TOPK = 2048
PAGE = 64


def slot_table(block_table_row, width):
    """int64 [width]: token t -> slot bt[t / 64] * 64 + t % 64."""
    t = np.arange(width, dtype=np.int64)
    return np.asarray(block_table_row, dtype=np.int64)[t // PAGE] * PAGE + t % PAGE


def wire_format_problems(out, lens, slots_of_row):
    """Every way the rows of `out` break the wire format, as strings (empty when they keep it).

    out: int32 [rows, 2048]; lens: int [rows]; slots_of_row(r) -> int64 [>= len_r], token -> slot
    for row r (the page table the top-k was given).  The token order inside a row is checked up to
    what the format fixes (short rows: token order; long rows: at most two ascending runs); the
    exact split into runs depends on the scores and is checked against the oracle elsewhere."""
    out = np.asarray(out)
    problems = []
    if out.dtype != np.int32:
        problems.append(f"dtype {out.dtype}, not int32")
    if out.ndim != 2 or out.shape[1] != TOPK:
        return problems + [f"shape {out.shape}, not [rows, {TOPK}]"]
    for r in range(out.shape[0]):
        L = max(int(lens[r]), 0)
        n = min(L, TOPK)
        row = out[r].astype(np.int64)
        if not (row[n:] == -1).all():
            problems.append(f"row {r}: entries past {n} are not all -1")
        head = row[:n]
        if n == 0:
            continue
        if (head < 0).any():
            problems.append(f"row {r}: a pad among the first {n} entries")
            continue
        slots = np.asarray(slots_of_row(r), dtype=np.int64)[:L]
        order = np.argsort(slots, kind="stable")
        pos = np.searchsorted(slots[order], head)
        pos = np.minimum(pos, L - 1)
        if not (slots[order][pos] == head).all():
            problems.append(f"row {r}: a slot id that no token below the length maps to")
            continue
        tok = order[pos]
        if np.unique(tok).size != n:
            problems.append(f"row {r}: a token listed twice")
        descents = int((np.diff(tok) < 0).sum())
        if L <= TOPK and not np.array_equal(tok, np.arange(n)):
            problems.append(f"row {r}: a row of {L} <= {TOPK} tokens not copied in token order")
        elif descents > 1:
            problems.append(f"row {r}: {descents + 1} ascending runs, at most 2 allowed")
    return problems


def sparse_mla_decode(q, kv_rows, sm_scale):
    """Sparse MLA decode of one query row.  q float [H, 576]; kv_rows float [n, 576] (the listed
    slots' dequantised K in list order, pads removed).  Returns (o [H, 512], lse [H]) in float64,
    the softmax and the weighted sum taken in list order."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(kv_rows, dtype=np.float64)
    if k.shape[0] == 0:
        return np.zeros((q.shape[0], 512)), np.full(q.shape[0], -np.inf)
    s = (q @ k.T) * sm_scale
    m = s.max(axis=1, keepdims=True)
    e = np.exp(s - m)
    z = e.sum(axis=1, keepdims=True)
    return (e / z) @ k[:, :512], (np.log(z) + m)[:, 0]


def bf16_bits_to_f32(bits):
    """uint16 bf16 bits -> float32."""
    return (np.asarray(bits, dtype=np.uint32) << 16).view(np.float32)
