"""Register and scratch use of every kernel of the built library, from the compiler's
resource-usage remarks that build.py records: no kernel may spill to scratch memory (a spill in
the hot kernels costs microseconds a launch and has appeared from small source edits), and the
occupancy each launch shape is sized for must hold."""
import json
import os

import pytest

RES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sglang0.5.18-opt_amd", "_build",
                   "kernel_resources.json")


@pytest.fixture(scope="module")
def usage():
    if not os.path.exists(RES):
        pytest.skip("library not built here (sglang0.5.18-opt_amd/build.py writes the resource record)")
    with open(RES) as f:
        return json.load(f)


def test_no_kernel_spills(usage):
    assert usage, "no kernels recorded"
    spills = {k: v["scratch"] for k, v in usage.items() if v.get("scratch", 0)}
    assert not spills, f"kernels using scratch memory: {spills}"


def test_hot_kernels_keep_their_occupancy(usage):
    """The decode logits shapes run 4 waves a SIMD (two-row CTAs, 8 a CU) or 2 (one-row CTAs, two
    streams); the top-k's 512-thread CTAs run two a CU."""
    def occ(prefix):
        return {k: v["occupancy"] for k, v in usage.items() if prefix in k}
    decode_r2 = occ("mqa_logits_decode_kernelILi64ELi2ELb0ELb1E")
    assert decode_r2 and all(o >= 4 for o in decode_r2.values()), decode_r2
    topk = occ("topk_split_sampled_kernel")
    topk.update(occ("topk_row_sampled_kernel"))
    assert topk and all(o >= 4 for o in topk.values()), topk
