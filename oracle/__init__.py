"""CPU oracle of the DSA indexer path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this package,
and only as the checker (or, for the CPU baseline, as the timed CPU restatement).  The product
path (the hcu_ops package over libdsa_indexer.so) never imports it.

Contents (each function cites the reference file:line it restates):
  fp8.py        OCP fp8 e4m3fn decode / encode and fp32 -> bf16 RNE, from the format definitions
  indexer.py    paged dequant (132-B and 656-B layouts), per-vector fp8 quant, MQA logits + mask,
                top-k pass-1 histogram, brute-force top-2048 with the lower-index tie rule,
                page-table remap, and the torch-CPU indexer used as the CPU baseline
  topk_radix.c  sequential restatement of the reference's single-CTA radix select
                (12/12/8-bit digits, sparse fast path, ascending-token emission order),
                loaded through topk_c.py

How each part is pinned (checked by tests/test_oracle_*.py):
  fp8 decode    all 256 codes vs torch's float8_e4m3fn and the closed-form values of the format
  fp8 encode    vs torch's float -> float8_e4m3fn cast (RNE, non-saturating) on midpoints,
                subnormals, the 448 / 464 boundary and random values
  bf16 RNE      vs torch's float -> bfloat16 cast, incl. NaN / inf / ties
  dequant       vs torch-CPU (fp8.float() * scale).to(bfloat16), the reference's closed form
  logits        fp64 oracle vs an independent torch fp32 einsum and pure-Python loops on tiny
                shapes; linearity in w and in the K scale; all-negative rows give mask 0
  top-k         brute force (stable sort) vs the C radix restatement vs pure-Python selection on
                tiny rows, on the reference's ten score distributions (topk_lib.py:8-51), plus
                the invariants of topk_lib.py:70-89
  histogram     vs the closed form of test_mqa_hist.py:109-124
"""
