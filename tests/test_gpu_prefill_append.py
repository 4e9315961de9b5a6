"""nslg_paged_prefill_append (the forward's K/V write and its causal attention in one
launch) against nslg_append_kv then nslg_paged_prefill / nslg_paged_prefill_grid on
copies of the same pool: the output and the whole pool bit-identical. Cached
prefixes that end inside a page and inside a key tile, fresh prompts, sequences
without new tokens, GQA groups that do not divide a row tile (tokens whose query
rows span two tiles), page sizes of 1, 5 and 16, padded grids with input offsets,
f16 and bf16 at head_dim 64, 128 and 256. The two launches are tied to the oracle
by the prefill and append tests."""
import sys

import numpy as np
import pytest
import torch

DEV = "cuda:0"


def _case(seed, B, Hq, Hkv, D, ps, grid):
    """Inputs of one call, built and bounds-checked on the host: per sequence a cached
    prefix (start) and new tokens (n), distinct pages per sequence (page 0 unused),
    the slot of every new token, and for a grid its rows and input offsets."""
    rng = np.random.default_rng(seed)
    start = [int(x) for x in rng.integers(0, 700, size=B)]
    news = [int(x) for x in rng.integers(1, 300, size=B)]
    start[0] = 0                      # a fresh prompt
    if B > 2:
        news[2] = 0                   # a sequence without new tokens
        start[1] = 64 * 3 + 17        # prefix ends inside a key tile
    lens = [s + n for s, n in zip(start, news)]
    npg = [(L + ps - 1) // ps for L in lens]
    P = sum(npg) + 3
    ids = rng.permutation(np.arange(1, P)).astype(np.int32)
    indptr = np.zeros(B + 1, np.int32)
    np.cumsum(npg, out=indptr[1:])
    indices = ids[:indptr[-1]]
    lpl = np.asarray([L - (m - 1) * ps if m else 0 for L, m in zip(lens, npg)], np.int32)
    qo = np.zeros(B + 1, np.int32)
    np.cumsum(news, out=qo[1:])
    T = int(qo[-1])
    offs = [int(x) for x in rng.integers(0, 5, size=B)] if grid else [0] * B
    W = max(o + n for o, n in zip(offs, news)) if grid else 0
    n_rows = B * W if grid else T
    rows = np.zeros(max(T, 1), np.int32)
    slots = np.full(n_rows, -1, np.int32)
    for b in range(B):
        for t in range(news[b]):
            r = b * W + offs[b] + t if grid else int(qo[b]) + t
            pos = start[b] + t
            slots[r] = int(indices[indptr[b] + pos // ps]) * ps + pos % ps
            rows[qo[b] + t] = r
    # host-side bounds: every page id and slot inside the pool, every row inside q
    assert indices.min() >= 1 and indices.max() < P and len(set(indices.tolist())) == len(indices)
    assert slots.max() < P * ps and (rows[:T] < n_rows).all()
    return dict(B=B, P=P, T=T, W=W, n_rows=n_rows, news=news, start=start, indptr=indptr, indices=indices,
                lpl=lpl, qo=qo, rows=rows, slots=slots, Hq=Hq, Hkv=Hkv, D=D, ps=ps, grid=grid, seed=seed)


SHAPES = [  # (B, Hq, Hkv, D, ps)
    (4, 32, 8, 128, 16),
    (5, 24, 8, 128, 5),    # G = 3: tokens whose rows span two row tiles; pages of 5
    (3, 16, 16, 64, 1),    # G = 1, one-token pages
    (4, 16, 1, 64, 16),    # G = 16
    (3, 12, 2, 256, 16),   # G = 6 at head_dim 256
    (2, 8, 8, 256, 5),
]


def test_case_builder_stays_in_bounds():
    """The host side of the GPU cases below (runs without a GPU)."""
    for i, (B, Hq, Hkv, D, ps) in enumerate(SHAPES):
        for grid in (False, True):
            c = _case(700 + i, B, Hq, Hkv, D, ps, grid)
            assert c["T"] == sum(c["news"]) and int(c["indptr"][-1]) == len(c["indices"])


@pytest.mark.gpu
@pytest.mark.parametrize("grid", [False, True])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape", range(len(SHAPES)))
def test_prefill_append_equals_append_then_prefill(shape, dtype, grid):
    from nanoslg_amd import kernels as K
    B, Hq, Hkv, D, ps = SHAPES[shape]
    c = _case(700 + shape, B, Hq, Hkv, D, ps, grid)
    print(f"prefill_append B={B} {Hq}/{Hkv}x{D} ps={ps} {dtype} grid={grid} T={c['T']}", flush=True)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(c["seed"])
    P, n_rows = c["P"], c["n_rows"]
    k_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    v_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(n_rows, Hq, D, generator=g).to(dtype).to(DEV)
    k_new = torch.randn(n_rows, Hkv, D, generator=g).to(dtype).to(DEV)
    v_new = torch.randn(n_rows, Hkv, D, generator=g).to(dtype).to(DEV)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(DEV)  # noqa: E731
    qo, ip, idx, lpl, slots = t(c["qo"]), t(c["indptr"]), t(c["indices"]), t(c["lpl"]), t(c["slots"])
    rows = t(c["rows"][:max(c["T"], 1)]) if grid else None
    W = c["W"] if grid else 0
    max_q = max(c["news"])
    kr, vr = k_pool.clone(), v_pool.clone()
    K.append_kv(k_new, v_new, slots, kr, vr)
    ref = K.paged_prefill(q, qo, c["T"], max_q, kr, vr, ip, idx, lpl, q_rows=rows, grid_width=W)
    kf, vf = k_pool.clone(), v_pool.clone()
    out = K.paged_prefill_append(q, qo, c["T"], max_q, k_new, v_new, kf, vf, ip, idx, lpl, q_rows=rows,
                                 grid_width=W)
    torch.cuda.synchronize()
    assert torch.equal(kf, kr) and torch.equal(vf, vr), "pool rows differ"
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16)), (out.float() - ref.float()).abs().max()


@pytest.mark.gpu
@pytest.mark.parametrize("grid", [False, True])
def test_prefill_append_strided_rows(grid):
    """k_new / v_new as the K and V halves of one [rows, 2, Hkv, D] projection output
    (row strides of 2 * Hkv * D elements, different base addresses), against append
    then prefill on the same rows."""
    from nanoslg_amd import kernels as K
    B, Hq, Hkv, D, ps = SHAPES[0]
    c = _case(720, B, Hq, Hkv, D, ps, grid)
    print(f"prefill_append strided grid={grid} T={c['T']}", flush=True)
    sys.stdout.flush()
    g = torch.Generator().manual_seed(720)
    P, n_rows = c["P"], c["n_rows"]
    k_pool = torch.randn(P, ps, Hkv, D, generator=g).half().to(DEV)
    v_pool = torch.randn(P, ps, Hkv, D, generator=g).half().to(DEV)
    q = torch.randn(n_rows, Hq, D, generator=g).half().to(DEV)
    kv = torch.randn(n_rows, 2, Hkv, D, generator=g).half().to(DEV)
    k_new, v_new = kv[:, 0], kv[:, 1]
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, np.int32)).to(DEV)  # noqa: E731
    qo, ip, idx, lpl, slots = t(c["qo"]), t(c["indptr"]), t(c["indices"]), t(c["lpl"]), t(c["slots"])
    rows = t(c["rows"][:max(c["T"], 1)]) if grid else None
    W = c["W"] if grid else 0
    kr, vr = k_pool.clone(), v_pool.clone()
    K.append_kv(k_new, v_new, slots, kr, vr)
    ref = K.paged_prefill(q, qo, c["T"], max(c["news"]), kr, vr, ip, idx, lpl, q_rows=rows, grid_width=W)
    kf, vf = k_pool.clone(), v_pool.clone()
    out = K.paged_prefill_append(q, qo, c["T"], max(c["news"]), k_new, v_new, kf, vf, ip, idx, lpl, q_rows=rows,
                                 grid_width=W)
    torch.cuda.synchronize()
    assert torch.equal(kf, kr) and torch.equal(vf, vr), "pool rows differ"
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
