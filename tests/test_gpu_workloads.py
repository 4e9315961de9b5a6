"""Parity at the workloads' full sizes, through the drop-in cache API.

Each test drives one of the measured workloads at its real shape (Llama-3.1-8B
layer: 32 query / 8 KV heads, head_dim 128, fp16, page 16) and checks every
attention output it checks against fp32 SDPA (the oracle's ``sdpa_gqa``, the
restatement of nanoslg/kv_cache.py:44-56) over the sequence's pages gathered
with plain torch indexing through the manager's block tables, run on the GPU
with torch's math backend in fp32 (the oracle's CPU loops would take minutes at
these sizes). Tolerance: 2e-3 abs + 1e-2 rel. Appended rows and copy-on-write
pages are compared bit for bit.

  small batch   4 sequences, contexts U[1024, 4096], 65,536-page pool, block
                tables a seeded permutation of the free pages, 128 decode steps,
                every step checked
  KV pressure   64 sequences, contexts log-uniform [2048, 32768], pool at 90 %
                occupancy with pages shuffled across sequences, 10 % of the pages
                released and re-admitted mid-run
  radix + CoW   16 requests on a released 2040-token prompt (its 127 full pages and
                its 8-token partial page matched through the radix tree),
                suffixes U[128, 1024] prefilled in one ragged forward (16 copies of
                the partial page), then 128 decode steps
  chunked prefill  8 prompts of 4096 tokens in 512-token chunks
  contiguous fp32  the reference's own CPU case on the GPU: one sequence, a
                512-token prompt, then 64 decode steps, fp32, against the oracle's
                restatement of the contiguous path (kv_cache.py:227-379)
"""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
HQ, HKV, D, PS = 32, 8, 128, 16
DEV = "cuda:0"


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _cache(pages, prefix=False):
    from nanoslg_amd.kv_cache import KVCacheConfig, PagedKVCache
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=PS,
                        max_pages=pages, dtype=torch.float16, device=torch.device(DEV),
                        enable_prefix_caching=prefix, backend="paged")
    return PagedKVCache(cfg)


def _shuffle_free(mgr, rng):
    free = np.array(mgr.pool._free, np.int64)
    rng.shuffle(free)
    mgr.pool._free = free.tolist()


def _admit_resident(mgr, sid, L):
    """A sequence of L tokens whose pages already hold the pool's (random) K/V."""
    mgr.allocate_sequence(sid, num_tokens=L)
    st = mgr.seqs[sid]
    st.num_tokens = L
    pages = st.bt[:st.n_pages].tolist()
    for i, p in enumerate(pages):
        mgr.pool.tokens_used[p] = PS if i < len(pages) - 1 else L - PS * (len(pages) - 1)


def _rows(mgr, sid, L):
    """Pool row ids (page * ps + slot) of the sequence's first L tokens, on the GPU."""
    st = mgr.seqs[sid]
    n = -(-L // PS)
    pages = torch.from_numpy(st.bt[:n].astype(np.int64)).to(DEV)
    return (pages[:, None] * PS + torch.arange(PS, device=DEV)[None, :]).reshape(-1)[:L]


def _reference(mgr, sid, q_rows):
    """fp32 SDPA over the sequence's gathered K/V; q_rows [n, Hq, D] are its last n
    tokens (bottom-right causal, the FlashInfer semantics of kv_cache.py:617-632)."""
    L = mgr.seqs[sid].num_tokens
    n = q_rows.shape[0]
    idx = _rows(mgr, sid, L)
    k = mgr.pool.k[0].reshape(-1, HKV, D)[idx].float().transpose(0, 1).unsqueeze(0).contiguous()
    v = mgr.pool.v[0].reshape(-1, HKV, D)[idx].float().transpose(0, 1).unsqueeze(0).contiguous()
    q = q_rows.float().transpose(0, 1).unsqueeze(0).contiguous()
    mask = None
    if n > 1:
        vis = torch.arange(L, device=DEV)[None, :] <= (L - n + torch.arange(n, device=DEV))[:, None]
        mask = torch.zeros(n, L, device=DEV).masked_fill(~vis, float("-inf"))[None, None]
    from torch.nn.attention import SDPBackend, sdpa_kernel
    with sdpa_kernel(SDPBackend.MATH):
        o = O.sdpa_gqa(q, k, v, attn_mask=mask)
    return o[0].transpose(0, 1)  # [n, Hq, D]


def _check_rows_written(mgr, sid, first, k_rows, v_rows):
    """The n new tokens of sid (positions first..first+n-1) hold exactly k_rows/v_rows."""
    n = k_rows.shape[0]
    idx = _rows(mgr, sid, first + n)[first:]
    got_k = mgr.pool.k[0].reshape(-1, HKV, D)[idx]
    got_v = mgr.pool.v[0].reshape(-1, HKV, D)[idx]
    assert torch.equal(got_k.view(torch.int16), k_rows.contiguous().view(torch.int16)), sid
    assert torch.equal(got_v.view(torch.int16), v_rows.contiguous().view(torch.int16)), sid


def _decode_and_check(mgr, ids, q, kn, vn, check=True):
    """One decode step of ids through begin_forward / attend / end_forward; q [B,1,Hq,D]."""
    starts = [mgr.seqs[s].num_tokens for s in ids]
    ctx = mgr.begin_forward(ids, [1] * len(ids))
    out = ctx.attend(0, q, kn, vn, HQ, HKV)
    mgr.end_forward(ctx)
    assert out.shape == (len(ids), 1, HQ * D) and out.dtype == torch.float16
    if not check:
        return
    for b, sid in enumerate(ids):
        assert mgr.seqs[sid].num_tokens == starts[b] + 1
        _check_rows_written(mgr, sid, starts[b], kn[b], vn[b])
        want = _reference(mgr, sid, q[b])
        torch.testing.assert_close(out[b].view(1, HQ, D).float(), want, atol=ATOL, rtol=RTOL,
                                   msg=lambda m, sid=sid: f"{sid}: {m}")


def test_small_batch_full_size():
    """4 sequences, contexts U[1024, 4096], 65,536-page pool, 128 steps, each checked."""
    _log("workload: small batch (B=4, 65536 pages, 128 steps)")
    rng = np.random.default_rng(2)
    lens = [int(x) for x in rng.integers(1024, 4097, size=4)]
    mgr = _cache(65536)
    _shuffle_free(mgr, rng)
    ids = [f"s{b}" for b in range(4)]
    for sid, L in zip(ids, lens):
        _admit_resident(mgr, sid, L)
    g = torch.Generator(device=DEV).manual_seed(2)
    mgr.pool.k.normal_(generator=g)
    mgr.pool.v.normal_(generator=g)
    for step in range(128):
        q = torch.randn(4, 1, HQ, D, generator=g, device=DEV, dtype=torch.float16)
        kn = torch.randn(4, 1, HKV, D, generator=g, device=DEV, dtype=torch.float16)
        vn = torch.randn(4, 1, HKV, D, generator=g, device=DEV, dtype=torch.float16)
        _decode_and_check(mgr, ids, q, kn, vn)
    assert [mgr.seqs[s].num_tokens for s in ids] == [L + 128 for L in lens]


def test_kv_pressure_full_size():
    """64 sequences, log-uniform [2048, 32768] contexts, 90 % occupancy, shuffled pages;
    10 % of the pages released and re-admitted between checked steps."""
    rng = np.random.default_rng(0)
    B = 64
    lens = [int(round(math.exp(x))) for x in rng.uniform(math.log(2048), math.log(32768), size=B)]
    pages = math.ceil(sum(math.ceil(L / PS) for L in lens) / 0.9) + 1
    _log(f"workload: KV pressure (B=64, sum L={sum(lens)}, {pages} pages)")
    mgr = _cache(pages)
    _shuffle_free(mgr, rng)
    ids = [f"s{b}" for b in range(B)]
    for sid, L in zip(ids, lens):
        _admit_resident(mgr, sid, L)
    g = torch.Generator(device=DEV).manual_seed(0)
    mgr.pool.k.normal_(generator=g)
    mgr.pool.v.normal_(generator=g)

    def inputs():
        return (torch.randn(B, 1, HQ, D, generator=g, device=DEV, dtype=torch.float16),
                torch.randn(B, 1, HKV, D, generator=g, device=DEV, dtype=torch.float16),
                torch.randn(B, 1, HKV, D, generator=g, device=DEV, dtype=torch.float16))

    # step 0 is planned on the host, the others on the device: steps 0-2 and every
    # 4th after them checked (a page opens every 16 steps of a sequence, at staggered
    # steps across the batch, so checked device-planned steps include page openings)
    for step in range(21):
        _decode_and_check(mgr, ids, *inputs(), check=step < 3 or step % 4 == 0)
    # churn: release whole sequences until 10 % of the used pages are free, re-admit them
    used = sum(mgr.seqs[s].n_pages for s in ids)
    freed, victims = 0, []
    for b in rng.permutation(B):
        if freed >= 0.1 * used:
            break
        sid = ids[b]
        victims.append((sid, mgr.seqs[sid].num_tokens))
        freed += mgr.seqs[sid].n_pages
        mgr.release_sequence(sid)
    _shuffle_free(mgr, rng)
    for sid, L in victims:
        _admit_resident(mgr, sid, L)
        rows = _rows(mgr, sid, -(-L // PS) * PS)
        mgr.pool.k[0].reshape(-1, HKV, D)[rows] = torch.randn(rows.numel(), HKV, D, generator=g, device=DEV,
                                                              dtype=torch.float16)
        mgr.pool.v[0].reshape(-1, HKV, D)[rows] = torch.randn(rows.numel(), HKV, D, generator=g, device=DEV,
                                                              dtype=torch.float16)
    _log(f"churn: {len(victims)} sequences, {freed} pages")
    # the first step after the churn is planned on the host from the device-resident
    # block tables (only the re-admitted sequences' tables are uploaded), the rest on
    # the device
    for step in range(9):
        _decode_and_check(mgr, ids, *inputs(), check=step < 3 or step % 4 == 0)
    assert mgr.pool.num_free + sum(mgr.seqs[s].n_pages for s in ids) == pages - 1


def test_radix_cow_full_size():
    """16 requests on one cached 2040-token prompt, through the cache API alone: the
    prompt's release caches its 127 full pages and its partial last page (8 tokens);
    each request's allocation matches all 2040 tokens (refcount of the partial page:
    the tree + 16); the ragged suffix prefill copies that page for every request
    (16 copy-on-writes; the tree keeps the original), then 128 decode steps; outputs
    against SDPA, the cached pages untouched, the copies exact."""
    _log("workload: radix prefix + copy-on-write (16 x 2040-token prefix, 128 decode steps)")
    B, PRE = 16, 2040
    full = PRE // PS
    rng = np.random.default_rng(4)
    suffix = [int(x) for x in rng.integers(128, 1025, size=B)]
    steps = 128
    pages = full + 1 + sum(math.ceil((PRE % PS + s + steps) / PS) + 1 for s in suffix) + 64
    mgr = _cache(pages, prefix=True)
    g = torch.Generator(device=DEV).manual_seed(4)
    randn = lambda *shape: torch.randn(*shape, generator=g, device=DEV, dtype=torch.float16)  # noqa: E731
    prompt = rng.integers(0, 128256, size=PRE).tolist()
    mgr.allocate_sequence("owner", token_ids=prompt)
    qp, kp, vp = randn(1, PRE, HQ, D), randn(1, PRE, HKV, D), randn(1, PRE, HKV, D)
    ctx = mgr.begin_forward(["owner"], [PRE])
    out = ctx.attend(0, qp, kp, vp, HQ, HKV)
    mgr.end_forward(ctx)
    torch.testing.assert_close(out[0].view(PRE, HQ, D).float(), _reference(mgr, "owner", qp[0]),
                               atol=ATOL, rtol=RTOL)
    owner_pages = mgr.seqs["owner"].bt[:full + 1].tolist()
    mgr.release_sequence("owner")
    assert mgr.tree.cached_pages == full + 1
    assert mgr.pool.tokens_used[owner_pages[full]] == PRE % PS
    ids = [f"r{b}" for b in range(B)]
    for sid, n in zip(ids, suffix):
        plen = mgr.allocate_sequence(sid, token_ids=prompt + rng.integers(0, 128256, size=n).tolist())
        assert plen == PRE
        st = mgr.seqs[sid]
        assert st.bt[:full + 1].tolist() == owner_pages and st.num_tokens == PRE
    assert mgr.pool.ref_count[owner_pages[full]] == B + 1
    shared_rows = _rows(mgr, ids[0], PRE)
    shared_k = mgr.pool.k[0].reshape(-1, HKV, D)[shared_rows].clone()
    S = max(suffix)
    q, k, v = randn(B, S, HQ, D), randn(B, S, HKV, D), randn(B, S, HKV, D)
    ctx = mgr.begin_forward(ids, suffix)
    out = ctx.attend(0, q, k, v, HQ, HKV)
    mgr.end_forward(ctx)
    assert sorted(s for s, _ in ctx.cow_pairs) == [owner_pages[full]] * B
    assert all(mgr.seqs[s].bt[full] != owner_pages[full] for s in ids)
    assert mgr.pool.ref_count[owner_pages[full]] == 1  # the tree's, for the next request
    for b, sid in enumerate(ids):
        n = suffix[b]
        _check_rows_written(mgr, sid, PRE, k[b, :n], v[b, :n])
        # the prefix as this request sees it (shared or copied page) is the prompt's K
        got = mgr.pool.k[0].reshape(-1, HKV, D)[_rows(mgr, sid, PRE)]
        assert torch.equal(got.view(torch.int16), shared_k.view(torch.int16)), sid
        torch.testing.assert_close(out[b, :n].view(n, HQ, D).float(), _reference(mgr, sid, q[b, :n]),
                                   atol=ATOL, rtol=RTOL, msg=lambda m, sid=sid: f"{sid}: {m}")
    for step in range(steps):
        _decode_and_check(mgr, ids, randn(B, 1, HQ, D), randn(B, 1, HKV, D), randn(B, 1, HKV, D),
                          check=step < 2 or step % 8 == 7 or step == steps - 1)
    # the cached prompt pages, the partial one included, were never written
    cached = torch.from_numpy(np.asarray(owner_pages, np.int64)).to(DEV)
    rows = (cached[:, None] * PS + torch.arange(PS, device=DEV)[None, :]).reshape(-1)[:PRE]
    assert torch.equal(mgr.pool.k[0].reshape(-1, HKV, D)[rows].view(torch.int16), shared_k.view(torch.int16))


def test_chunked_prefill_full_size():
    """8 prompts x 4096 tokens in 512-token chunks: every chunk's rows against SDPA
    with bottom-right causal masking over all earlier pages, its K/V rows exact."""
    _log("workload: chunked prefill (8 x 4096 in 512-token chunks)")
    B, L, CH = 8, 4096, 512
    mgr = _cache(B * L // PS + 64)
    _shuffle_free(mgr, np.random.default_rng(5))
    ids = [f"p{b}" for b in range(B)]
    for sid in ids:
        mgr.allocate_sequence(sid)
    g = torch.Generator(device=DEV).manual_seed(5)
    for c in range(L // CH):
        q = torch.randn(B, CH, HQ, D, generator=g, device=DEV, dtype=torch.float16)
        k = torch.randn(B, CH, HKV, D, generator=g, device=DEV, dtype=torch.float16)
        v = torch.randn(B, CH, HKV, D, generator=g, device=DEV, dtype=torch.float16)
        ctx = mgr.begin_forward(ids, [CH] * B)
        out = ctx.attend(0, q, k, v, HQ, HKV)
        mgr.end_forward(ctx)
        for b, sid in enumerate(ids):
            assert mgr.seqs[sid].num_tokens == (c + 1) * CH
            _check_rows_written(mgr, sid, c * CH, k[b], v[b])
            torch.testing.assert_close(out[b].view(CH, HQ, D).float(), _reference(mgr, sid, q[b]),
                                       atol=ATOL, rtol=RTOL, msg=lambda m, c=c, sid=sid: f"chunk {c} {sid}: {m}")


def test_contiguous_fp32_prompt_and_decode():
    """Contiguous backend in fp32: a 512-token prompt of N(0,1) K/V, then 64 decode
    steps (q ~ N(0,1) / sqrt(128)), each against the oracle's contiguous path run on
    the same inputs; pool bytes equal to the oracle's after every step."""
    _log("workload: contiguous fp32 (1 x 512 prompt + 64 decode steps)")
    from nanoslg_amd import kv_cache as KC
    Smax = 640
    cfg = KC.KVCacheConfig(num_layers=1, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, max_batch_size=1,
                           max_seq_len=Smax, dtype=torch.float32, device=DEV, backend="contiguous")
    mgr = KC.ContiguousKVCache(cfg)
    ref = O.ContiguousRef(1, 1, Smax, HKV, D)
    for m in (mgr, ref):
        m.allocate_sequence("s")
    g = torch.Generator().manual_seed(7)
    steps = [512] + [1] * 64
    for n in steps:
        q = torch.randn(1, n, HQ, D, generator=g) / math.sqrt(D)
        k = torch.randn(1, n, HKV, D, generator=g)
        v = torch.randn(1, n, HKV, D, generator=g)
        c1, c2 = mgr.begin_forward(["s"], [n]), ref.begin_forward(["s"], [n])
        o1 = c1.attend(0, q.to(DEV), k.to(DEV), v.to(DEV), HQ, HKV).cpu()
        o2 = c2.attend(0, q, k, v, HQ, HKV)
        assert o1.dtype == torch.float32
        torch.testing.assert_close(o1, o2, atol=2e-5, rtol=1e-4)
        mgr.end_forward(c1)
        ref.end_forward(c2)
    torch.cuda.synchronize()
    assert torch.equal(mgr.k.cpu(), ref.k) and torch.equal(mgr.v.cpu(), ref.v)
