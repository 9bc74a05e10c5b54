"""GPU parity: paged K dequant / gather (132-B and 656-B layouts), q quantisation and the K-cache
writer against the oracle -- all bit-exact."""
import numpy as np
import pytest
import torch

import hcu_ops
import workloads as wl
from oracle import indexer as O

from gpu_util import kv_np, q_bits

pytestmark = pytest.mark.gpu


def _edge_cache():
    """8 pages, one scale per page (incl. 0, tiny and huge), even tokens hold codes 0..127 and
    odd tokens 128..255, so every fp8 code meets every scale."""
    scales = np.array([1.0, 2.0 ** -20, 3.0e-3, 1.7e5, 2.0 ** -126, 6.1e-5, 0.0, 448.0], dtype=np.float32)
    kv = np.zeros((len(scales), 64 * 132), dtype=np.uint8)
    for p, s in enumerate(scales):
        for t in range(64):
            kv[p, t * 128:(t + 1) * 128] = (np.arange(128) + 128 * (t % 2)).astype(np.uint8)
            kv[p, 8192 + t * 4:8192 + t * 4 + 4] = np.array([s], dtype=np.float32).view(np.uint8)
    return kv


def test_dequant_all_codes_all_scales(gpu):
    kv = _edge_cache()
    slots = np.random.default_rng(0).permutation(kv.shape[0] * 64).astype(np.int32)
    slots[::97] = -1  # padded entries dequantise to zeros
    kv_t = torch.from_numpy(kv).view(-1, 64, 1, 132).to(gpu)
    got = hcu_ops.dequant_k_paged(kv_t, torch.from_numpy(slots).to(gpu))
    ref = O.dequant_k_paged(kv, slots)
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), ref)


def test_dequant_and_gather_random_cache(gpu):
    case = wl.prefill_case(7, 64, 9000, heads=32)
    kv = kv_np(case.kv)
    slots = case.slots().numpy()
    kv_t = case.kv.to(gpu)
    s_t = torch.from_numpy(slots).to(gpu)
    got = hcu_ops.dequant_k_paged(kv_t, s_t)
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), O.dequant_k_paged(kv, slots))
    k8, sc = hcu_ops.gather_k_paged(kv_t, s_t)
    codes, scale = O.kv_tokens(kv, slots)
    assert np.array_equal(k8.view(torch.uint8).cpu().numpy(), codes)
    assert np.array_equal(sc.cpu().numpy().view(np.uint32), scale.view(np.uint32))


def test_dequant_k_large_output(gpu):
    """2^20 + 1 tokens: a 268 MB output, past the 256 MB at which the rows are stored
    nontemporally; padded (-1) slots give zero rows."""
    g = torch.Generator().manual_seed(5)
    pages = 4096
    kv = torch.randint(0, 256, (pages, 64 * 132), generator=g, dtype=torch.uint8)
    kv[:, 8192:] = (torch.rand(pages, 64, generator=g) * 0.05 + 1e-3).view(torch.uint8)
    n = (1 << 20) + 1
    slots = torch.randint(0, pages * 64, (n,), generator=g, dtype=torch.int32)
    slots[::1001] = -1
    got = hcu_ops.dequant_k_paged(kv.view(pages, 64, 1, 132).to(gpu), slots.to(gpu))
    ref = O.dequant_k_paged(kv.numpy(), slots.numpy())
    assert np.array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), ref)


# 250000: a 288 MB output (nontemporal rows); negative slots are padded entries (zero rows)
@pytest.mark.parametrize("n", [1, 7, 3000, 250000])
def test_dequant_mla_656(gpu, n):
    g = torch.Generator().manual_seed(2)
    pool = 4096
    cache = (torch.randn(pool, 656, generator=g) * 0.1).to(torch.float8_e4m3fn).view(torch.uint8)
    cache[:, 512:528] = (torch.rand(pool, 4, generator=g) * 0.02 + 1e-3).view(torch.uint8)
    cache[:, 528:] = torch.randn(pool, 64, generator=g).to(torch.bfloat16).view(torch.uint8)
    slots = torch.randint(0, pool, (n,), generator=g, dtype=torch.int32)
    slots[3::53] = -1
    got = hcu_ops.dequantize_k_cache_paged(cache.view(torch.float8_e4m3fn).view(pool, 1, 656).to(gpu), slots.to(gpu))
    assert tuple(got.shape) == (n, 1, 576) and got.dtype == torch.bfloat16
    ref = O.dequant_mla(cache.numpy(), slots.numpy())
    assert np.array_equal(got.view(n, 576).view(torch.int16).cpu().numpy().view(np.uint16), ref)


def test_quant_q_bit_exact(gpu):
    g = torch.Generator().manual_seed(3)
    q = torch.randn(37, 64, 128, generator=g) * torch.rand(37, 64, 1, generator=g) * 50
    q[3, 5] = 0.0  # zero vector: codes 0, weight 0
    q[4, 6, 7] = 1e4  # one dominant element
    qb = q.to(torch.bfloat16)
    w = torch.randn(37, 64, generator=g)
    q8, weff = hcu_ops.quant_q_fp8(qb.to(gpu), w.to(gpu))
    rc, rw = O.quant_q(q_bits(qb), w.numpy())
    assert np.array_equal(q8.view(torch.uint8).cpu().numpy(), rc)
    assert np.array_equal(weff.cpu().numpy().view(np.uint32), rw.view(np.uint32))


def test_store_k_cache_bit_exact(gpu):
    g = torch.Generator().manual_seed(4)
    n_pages = 40
    k = (torch.randn(1000, 128, generator=g) * 3).to(torch.bfloat16)
    slots = torch.randperm(n_pages * 64, generator=g)[:1000].to(torch.int32)
    kv = torch.zeros(n_pages, 64, 1, 132, dtype=torch.uint8)
    kv_g = kv.to(gpu)
    hcu_ops.store_k_cache(k.to(gpu), slots.to(gpu), kv_g)
    kf = (k.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    ref = O.build_kv_cache(kf, slots.numpy(), n_pages)
    assert np.array_equal(kv_g.view(n_pages, -1).cpu().numpy(), ref)


def test_store_k_cache_skips_padded_slots(gpu):
    """Negative slots (padded entries) store nothing: the cache equals the oracle's cache of the
    other entries alone, zero everywhere else."""
    g = torch.Generator().manual_seed(5)
    n_pages = 24
    k = (torch.randn(1200, 128, generator=g) * 2).to(torch.bfloat16)
    slots = torch.randperm(n_pages * 64, generator=g)[:1200].to(torch.int32)
    slots[::7] = -1
    slots[-1] = -5
    kv_g = torch.zeros(n_pages, 64, 1, 132, dtype=torch.uint8, device=gpu)
    hcu_ops.store_k_cache(k.to(gpu), slots.to(gpu), kv_g)
    keep = (slots >= 0).numpy()
    kf = (k.view(torch.int16).numpy().view(np.uint16).astype(np.uint32) << 16).view(np.float32)
    ref = O.build_kv_cache(kf[keep], slots.numpy()[keep], n_pages)
    assert np.array_equal(kv_g.view(n_pages, -1).cpu().numpy(), ref)
