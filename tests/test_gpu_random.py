"""Randomised serving traffic on the GPU: the same seeded runs as
tests/test_host_random.py (admissions with prefix hits, ragged prefill, decode of
whole batches, subsets and mixed with prefill rows, partial pages shared by
reference, releases, evictions, OOM), through the real kernels: the host and
device planners, append, zero and copy pages, the decode (grouped when requests
share their first pages) and prefill kernels. fp16 pools, head_dim 64, 8 query /
2 KV heads. After every forward: outputs within 2e-3 abs + 1e-2 rel of the
oracle's fp32 SDPA on the same (fp16-rounded) inputs, positions, copy-on-writes,
free and cached pages, and every sequence's K/V read through its block table
bit-exact."""
import sys

import pytest
import torch

pytestmark = pytest.mark.gpu

GPU = dict(device="cuda:0", dtype=torch.float16, HQ=8, HKV=2, D=64, atol=2e-3, rtol=1e-2)


@pytest.mark.parametrize("seed,ps,pages", [(s, [1, 2, 3, 4, 8, 16][s % 6], [16, 20, 24, 30, 40, 64][(s // 6) % 6])
                                           for s in range(1, 21)])
def test_random_serving_traffic_on_gpu(seed, ps, pages):
    import test_host_random as R
    print(f"random traffic seed={seed} ps={ps} pages={pages}", flush=True)
    sys.stdout.flush()
    R.run_traffic(seed, ps, pages, GPU)


@pytest.mark.parametrize("seed,ps,pages,HQ,HKV,D,dtype", [
    (501, 16, 40, 32, 8, 128, torch.float16),   # the Llama-3 layer shape
    (502, 8, 60, 32, 8, 128, torch.bfloat16),
    (503, 32, 30, 16, 8, 128, torch.float16),   # G = 2
    (504, 4, 50, 8, 8, 64, torch.bfloat16),     # G = 1
    (505, 1, 70, 16, 2, 64, torch.float16),     # G = 8, one-token pages
    (506, 16, 24, 32, 8, 128, torch.bfloat16),
    (507, 16, 40, 12, 2, 256, torch.bfloat16),  # G = 6 at head_dim 256
    (508, 5, 60, 24, 8, 64, torch.float16),     # G = 3, pages of 5 tokens
    (509, 16, 40, 16, 1, 128, torch.float16),   # G = 16
])
def test_random_serving_traffic_shapes_on_gpu(seed, ps, pages, HQ, HKV, D, dtype):
    """The same traffic at other head shapes and in bf16, on the same bar."""
    import test_host_random as R
    print(f"random traffic seed={seed} ps={ps} pages={pages} {HQ}/{HKV}x{D} {dtype}", flush=True)
    sys.stdout.flush()
    env = dict(GPU, HQ=HQ, HKV=HKV, D=D, dtype=dtype)
    R.run_traffic(seed, ps, pages, env)


@pytest.mark.parametrize("native", [True, False])
@pytest.mark.parametrize("seed,ps,pages", [(21, 4, 48), (22, 1, 60), (23, 16, 12), (25, 3, 40), (26, 8, 40)])
def test_random_serving_traffic_device_planned_on_gpu(monkeypatch, seed, ps, pages, native):
    """The same traffic with every forward that is not a plain decode step planned on
    the device (nslg_block_table_csr, nslg_forward_plan), its host part from the
    native planner or from the numpy path."""
    import test_host_random as R
    from nanoslg_amd import kv_cache as KC
    print(f"device-planned traffic seed={seed} ps={ps} pages={pages} native={native}", flush=True)
    monkeypatch.setattr(KC.PagedCacheContext, "DEVICE_PLAN_TOKENS", 1)
    monkeypatch.setattr(KC.PagedKVCache, "NATIVE_PLAN", native)
    R.run_traffic(seed, ps, pages, GPU)


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_random_contiguous_traffic_on_gpu(seed):
    import test_host_random as R
    print(f"random contiguous traffic seed={seed}", flush=True)
    R.run_contiguous_traffic(seed, GPU)
