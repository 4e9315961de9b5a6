"""nslg_paged_decode_noalloc (the decode without a caller workspace: its split-K
partials live in the library's static per-GPU scratch) against nslg_paged_decode
with a workspace, through the C ABI: the same kernels, so the outputs must be
bit-identical. Two calls in a row, the second on a smaller batch (the scratch
keeps the first call's contents), per dtype; and the rejection of a batch whose
scratch need exceeds the static array."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _case(lens, ps, P, Hq, Hkv, D, dtype, seed):
    """A random paged batch on the device: pools, CSR block table, q."""
    rng = np.random.default_rng(seed)
    npg = [math.ceil(L / ps) if L > 0 else 0 for L in lens]
    assert sum(npg) <= P - 1
    perm = rng.permutation(np.arange(1, P))
    tables, off = [], 0
    for n in npg:
        tables.append(perm[off:off + n].tolist())
        off += n
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(len(lens), Hq, D, generator=g).to(dtype).to(DEV)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(DEV)  # noqa: E731
    if len(indices) == 0:
        indices = np.zeros(1, np.int32)
    return q, k, v, t(indptr), t(indices), t(lpl), int(indptr[-1])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_noalloc_decode_matches_workspace_entry_point(dtype):
    from nanoslg_amd import kernels
    Hq, Hkv, D, ps, P = 32, 8, 128, 16, 4096
    # first call: 24 sequences up to 3000 tokens (many chunks each); second: 5 shorter
    # ones, including an empty sequence, after the first call's partials
    rng = np.random.default_rng(7)
    big = [int(x) for x in rng.integers(1, 3001, size=24)]
    small = [300, 0, 17, 1024, 2]
    for i, lens in enumerate((big, small)):
        _log(f"noalloc decode dtype={dtype} call={i} B={len(lens)} sum={sum(lens)}")
        q, k, v, ip, ix, lp, tp = _case(lens, ps, P, Hq, Hkv, D, dtype, seed=100 + i)
        need = kernels.paged_decode_workspace_size(len(lens), Hq, Hkv, D, tp, ps, dtype)
        from nanoslg_amd import _lib
        assert need <= _lib.NSLG_NOALLOC_SCRATCH_BYTES
        out_na = torch.full((len(lens), Hq, D), float("nan"), dtype=dtype, device=DEV)
        kernels.paged_decode_noalloc(q, k, v, ip, ix, lp, tp, out=out_na)
        ws = kernels.Workspace(DEV)
        out_ws = kernels.paged_decode(q, k, v, ip, ix, lp, tp, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_ws), (dtype, i)
        # and the tolerance of the attention against the oracle's fp32 SDPA
        want = O.paged_attention_ref([q[b:b + 1].float().cpu() for b in range(len(lens))],
                                     k.float().cpu().reshape(-1, Hkv, D), v.float().cpu().reshape(-1, Hkv, D),
                                     ps, ip.tolist(), ix.tolist(), lp.tolist(), [1] * len(lens), None)
        for b, L in enumerate(lens):
            if L > 0:
                torch.testing.assert_close(out_na[b].float().cpu(), want[b][0], atol=2e-3, rtol=1e-2)
            else:
                assert not out_na[b].any()


def test_noalloc_decode_rejects_a_batch_beyond_its_scratch():
    """A call needing more than the static scratch fails with NSLG_EWORKSPACE on the
    host, before any launch (its inputs are in bounds anyway: every sequence empty)."""
    from nanoslg_amd import _lib, kernels
    Hq, Hkv, D, ps = 32, 8, 128, 16
    B, total_pages = 1000, 1 << 20
    need = kernels.paged_decode_workspace_size(B, Hq, Hkv, D, total_pages, ps, torch.float16)
    assert need > _lib.NSLG_NOALLOC_SCRATCH_BYTES
    k = torch.zeros(64, ps, Hkv, D, dtype=torch.float16, device=DEV)
    q = torch.zeros(B, Hq, D, dtype=torch.float16, device=DEV)
    ip = torch.zeros(B + 1, dtype=torch.int32, device=DEV)
    ix = torch.zeros(1, dtype=torch.int32, device=DEV)
    lp = torch.ones(B, dtype=torch.int32, device=DEV)
    out = torch.empty_like(q)
    with pytest.raises(_lib.KernelLibraryError, match="static scratch"):
        kernels.paged_decode_noalloc(q, k, k, ip, ix, lp, total_pages, out=out)
