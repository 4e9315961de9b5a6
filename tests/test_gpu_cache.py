"""The drop-in cache API on the GPU (real HIP kernels) against the CPU oracle on
identical call sequences: ragged prefill, decode, copy-on-write, radix prefix
sharing, the contiguous backend and the factory. Page contents are compared
bit-exactly through each sequence's block table; attention outputs within
2e-3 abs + 1e-2 rel of fp32 SDPA."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
DEV = torch.device("cuda:0")
L, HQ, HKV, D = 2, 32, 8, 128


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def make(ps=16, pages=256, prefix=True, dtype=torch.float16, partial=True):
    from nanoslg_amd import kv_cache as KC
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=ps,
                           max_pages=pages, dtype=dtype, device=DEV, enable_prefix_caching=prefix,
                           backend="paged", share_partial_pages=partial)
    return KC.PagedKVCache(cfg), O.PagedRef(L, pages, ps, HKV, D, torch.float32, enable_prefix_caching=prefix,
                                            share_partial_pages=partial)


def forward_both(mgr, ref, ids, ntok, offs, g, dtype=torch.float16):
    S = max(o + n for o, n in zip(offs, ntok))
    B = len(ids)
    q = torch.randn(B, S, HQ, D, generator=g).to(dtype)
    k = torch.randn(B, S, HKV, D, generator=g).to(dtype)
    v = torch.randn(B, S, HKV, D, generator=g).to(dtype)
    c1 = mgr.begin_forward(ids, ntok, offs)
    c2 = ref.begin_forward(ids, ntok, offs)
    assert torch.equal(c1.get_position_ids(S).cpu(), c2.get_position_ids(S))
    assert len(c1.cow_pairs) == len(c2.cow_events)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    for layer in range(L):
        o1 = c1.attend(layer, qd, kd, vd, HQ, HKV).float().cpu()
        o2 = c2.attend(layer, q.float(), k.float(), v.float(), HQ, HKV)
        assert o1.shape == (B, S, HQ * D)
        for b in range(B):
            rows = slice(offs[b], offs[b] + ntok[b])
            torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=ATOL, rtol=RTOL)
            pad = torch.ones(S, dtype=torch.bool)
            pad[rows] = False
            assert not o1[b, pad].any()
    mgr.end_forward(c1)
    ref.end_forward(c2)
    return c1, c2


def check_state(mgr, ref, ids):
    torch.cuda.synchronize()
    assert mgr.pool.num_free == ref.pool.num_free
    ps = mgr.cfg.page_size
    kpool, vpool = mgr.pool.k.cpu(), mgr.pool.v.cpu()
    for sid in ids:
        st = mgr.seqs[sid]
        assert st.num_tokens == ref.seqs[sid].num_tokens
        bt = st.block_table
        n = st.num_tokens
        for layer in range(L):
            k1 = torch.stack([kpool[layer, bt[t // ps], t % ps] for t in range(n)])
            v1 = torch.stack([vpool[layer, bt[t // ps], t % ps] for t in range(n)])
            k2, v2 = ref.logical_kv(sid, layer)
            assert torch.equal(k1.float(), k2) and torch.equal(v1.float(), v2)


def test_prefill_attend_checks_the_callers_tensors():
    """The cache's prefill calls take its own pool and plan as they are and check the
    caller's q, k_new and v_new as the public kernel calls do: a CPU tensor, another
    dtype, other head counts or too few rows raise before any launch, and the same
    forward then runs as usual (outputs and pool bytes against the oracle)."""
    _log("cache: prefill attend argument checks")
    mgr, ref = make(prefix=False)
    g = torch.Generator().manual_seed(11)
    for sid in ("a", "b"):
        mgr.allocate_sequence(sid)
        ref.allocate_sequence(sid)
    ids, ntok, S = ["a", "b"], [20, 20], 20
    q = torch.randn(2, S, HQ, D, generator=g).half()
    k = torch.randn(2, S, HKV, D, generator=g).half()
    v = torch.randn(2, S, HKV, D, generator=g).half()
    c1 = mgr.begin_forward(ids, ntok)
    c2 = ref.begin_forward(ids, ntok)
    qd, kd, vd = q.to(DEV), k.to(DEV), v.to(DEV)
    with pytest.raises(ValueError):
        c1.attend(0, qd, k, vd, HQ, HKV)  # k_new on the host
    with pytest.raises(TypeError):
        c1.attend(0, qd, kd.bfloat16(), vd, HQ, HKV)
    with pytest.raises(ValueError):
        c1.attend(0, qd, kd[:, :, :4], vd[:, :, :4], HQ, HKV)  # 4 KV heads for a pool of 8
    with pytest.raises(ValueError):
        c1.attend(0, qd, kd[:, :10], vd[:, :10], HQ, HKV)  # 20 rows of slots, 10 rows given
    with pytest.raises(ValueError):
        c1.attend(0, q, kd, vd, HQ, HKV)  # q on the host
    with pytest.raises(TypeError):
        c1.attend(0, qd.bfloat16(), kd, vd, HQ, HKV)
    for layer in range(L):
        o1 = c1.attend(layer, qd, kd, vd, HQ, HKV).float().cpu()
        o2 = c2.attend(layer, q.float(), k.float(), v.float(), HQ, HKV)
        torch.testing.assert_close(o1, o2, atol=ATOL, rtol=RTOL)
    mgr.end_forward(c1)
    ref.end_forward(c2)
    check_state(mgr, ref, ids)


def test_prefill_attend_takes_strided_kv_rows(monkeypatch):
    """K/V given as the strided halves of one [B, S, 2, Hkv, D] projection output go
    through the same one-launch write + prefill as contiguous rows, with the same
    output and pool bytes."""
    _log("cache: prefill attend with strided K/V rows")
    from nanoslg_amd import kernels as K
    taken = []
    orig = K._paged_prefill_append_layer

    def spy(*a, **k):
        r = orig(*a, **k)
        taken.append(r is not None)
        return r
    monkeypatch.setattr(K, "_paged_prefill_append_layer", spy)
    g = torch.Generator().manual_seed(12)
    S = 40
    q = torch.randn(2, S, HQ, D, generator=g).half().to(DEV)
    kv = torch.randn(2, S, 2, HKV, D, generator=g).half().to(DEV)
    res = []
    for strided in (False, True):
        mgr, _ = make(prefix=False)
        for sid in ("a", "b"):
            mgr.allocate_sequence(sid)
        k, v = kv[:, :, 0], kv[:, :, 1]
        if not strided:
            k, v = k.contiguous(), v.contiguous()
        c = mgr.begin_forward(["a", "b"], [S, S])
        o = c.attend(0, q, k, v, HQ, HKV)
        mgr.end_forward(c)
        torch.cuda.synchronize()
        res.append((o, mgr.pool.k.clone(), mgr.pool.v.clone()))
    assert taken == [True, True]
    assert all(torch.equal(x, y) for x, y in zip(*res))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_head_dim_256_prefill_then_decode(dtype):
    """A 16-bit cache at head_dim 256: a ragged prefill and a chunk over cached
    context (the VALU attention kernel), then decode steps (the MFMA decode), against
    the oracle: outputs within the tolerance, pad rows zero, pool bytes equal."""
    _log(f"cache: head_dim 256 {dtype}")
    from nanoslg_amd import kv_cache as KC
    Dh, Hq, Hkv, ps, pages = 256, 16, 4, 16, 64
    cfg = KC.KVCacheConfig(num_layers=1, num_kv_heads=Hkv, num_qo_heads=Hq, head_dim=Dh, page_size=ps,
                           max_pages=pages, dtype=dtype, device=DEV, enable_prefix_caching=False, backend="paged")
    mgr = KC.PagedKVCache(cfg)
    ref = O.PagedRef(1, pages, ps, Hkv, Dh, torch.float32, enable_prefix_caching=False)
    g = torch.Generator().manual_seed(256)
    ids = ["a", "b"]
    for sid in ids:
        mgr.allocate_sequence(sid)
        ref.allocate_sequence(sid)
    for ntok in ([37, 100], [20, 5], [1, 1], [1, 1], [1, 1]):
        S = max(ntok)
        q = torch.randn(2, S, Hq, Dh, generator=g).to(dtype)
        k = torch.randn(2, S, Hkv, Dh, generator=g).to(dtype)
        v = torch.randn(2, S, Hkv, Dh, generator=g).to(dtype)
        c1 = mgr.begin_forward(ids, ntok)
        c2 = ref.begin_forward(ids, ntok)
        o1 = c1.attend(0, q.to(DEV), k.to(DEV), v.to(DEV), Hq, Hkv).float().cpu()
        o2 = c2.attend(0, q.float(), k.float(), v.float(), Hq, Hkv)
        for b in range(2):
            torch.testing.assert_close(o1[b, :ntok[b]], o2[b, :ntok[b]], atol=ATOL, rtol=RTOL)
            assert not o1[b, ntok[b]:].any()
        mgr.end_forward(c1)
        ref.end_forward(c2)
    torch.cuda.synchronize()
    kpool, vpool = mgr.pool.k.cpu(), mgr.pool.v.cpu()
    for sid in ids:
        st = mgr.seqs[sid]
        bt, n = st.block_table, st.num_tokens
        k1 = torch.stack([kpool[0, bt[t // ps], t % ps] for t in range(n)])
        v1 = torch.stack([vpool[0, bt[t // ps], t % ps] for t in range(n)])
        k2, v2 = ref.logical_kv(sid, 0)
        assert torch.equal(k1.float(), k2) and torch.equal(v1.float(), v2)


def test_paged_prefill_then_decode():
    _log("cache: prefill + decode")
    g = torch.Generator().manual_seed(0)
    mgr, ref = make()
    ids = ["a", "b", "c"]
    lens = [50, 90, 17]
    for s, n in zip(ids, lens):
        assert mgr.allocate_sequence(s, num_tokens=n) == ref.allocate_sequence(s, num_tokens=n) == 0
    forward_both(mgr, ref, ids, lens, [max(lens) - n for n in lens], g)
    for _ in range(20):
        forward_both(mgr, ref, ids, [1, 1, 1], [0, 0, 0], g)
    forward_both(mgr, ref, ids, [33, 0, 5], [0, 33, 28], g)  # chunked prefill, one idle sequence
    check_state(mgr, ref, ids)
    for s in ids:
        mgr.release_sequence(s)
        ref.release_sequence(s)
    assert mgr.pool.num_free == ref.pool.num_free


def test_copy_on_write_shared_partial_page():
    """16 sequences share a 2040-token prefix (127 full pages + a page with 8 slots);
    the first append of each hits slot 8 of the shared page: 15 copies, the last
    sharer writes in place."""
    _log("cache: copy-on-write")
    g = torch.Generator().manual_seed(1)
    mgr, ref = make(pages=512, prefix=False)
    R = 16
    ids = [f"r{i}" for i in range(R)]
    prefix = 2040
    for impl in (mgr, ref):
        impl.allocate_sequence("p", num_tokens=prefix)
    forward_both(mgr, ref, ["p"], [prefix], [0], g)
    for impl in (mgr, ref):
        pages = impl.seqs["p"].block_table
        for sid in ids:
            impl.allocate_sequence(sid)
            for p in pages:
                impl.pool.add_ref(p)
            st = impl.seqs[sid]
            if hasattr(st, "bt"):
                st.extend(pages)
            else:
                st.block_table = list(pages)
            st.num_tokens = prefix
        # the prefix owner steps away: the sequences hold the only references
        st = impl.seqs.pop("p")
        for p in pages:
            impl.pool.release(p)
    shared_last = mgr.seqs[ids[0]].block_table[-1]
    assert mgr.pool.ref_count[shared_last] == R
    c1, c2 = forward_both(mgr, ref, ids, [1] * R, [0] * R, g)
    assert len(c1.cow_pairs) == R - 1 == len(c2.cow_events)
    assert mgr.seqs[ids[-1]].block_table[-1] == shared_last
    for _ in range(10):
        forward_both(mgr, ref, ids, [1] * R, [0] * R, g)
    check_state(mgr, ref, ids)


def test_radix_prefix_reuse():
    _log("cache: radix prefix reuse")
    g = torch.Generator().manual_seed(2)
    mgr, ref = make(pages=128, prefix=True)
    rng = np.random.default_rng(2)
    prompt = rng.integers(0, 128256, size=70).tolist()
    for impl in (mgr, ref):
        impl.allocate_sequence("a", token_ids=prompt)
    forward_both(mgr, ref, ["a"], [70], [0], g)
    mgr.release_sequence("a")
    ref.release_sequence("a")
    q2 = prompt[:64] + rng.integers(0, 128256, size=9).tolist()
    p1 = mgr.allocate_sequence("b", token_ids=q2)
    p2 = ref.allocate_sequence("b", token_ids=q2)
    assert p1 == p2 == 64
    check_state(mgr, ref, ["b"])
    forward_both(mgr, ref, ["b"], [9], [0], g)
    forward_both(mgr, ref, ["b"], [1], [0], g)
    check_state(mgr, ref, ["b"])


def test_contiguous_backend_on_gpu():
    _log("cache: contiguous backend")
    from nanoslg_amd import kv_cache as KC
    g = torch.Generator().manual_seed(3)
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, max_batch_size=3,
                           max_seq_len=256, dtype=torch.float16, device=DEV, backend="contiguous")
    mgr = KC.ContiguousKVCache(cfg)
    ref = O.ContiguousRef(L, 3, 256, HKV, D)
    ids = ["a", "b", "c"]
    for s in ids:
        mgr.allocate_sequence(s)
        ref.allocate_sequence(s)
    steps = [([40, 100, 7], [60, 0, 93])] + [([1, 1, 1], [0, 0, 0])] * 6 + [([20, 3, 1], [0, 17, 19])]
    for ntok, offs in steps:
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(3, S, HQ, D, generator=g).half()
        k = torch.randn(3, S, HKV, D, generator=g).half()
        v = torch.randn(3, S, HKV, D, generator=g).half()
        c1 = mgr.begin_forward(ids, ntok, offs)
        c2 = ref.begin_forward(ids, ntok, offs)
        assert torch.equal(c1.get_position_ids(S).cpu(), c2.get_position_ids(S))
        for layer in range(L):
            o1 = c1.attend(layer, q.to(DEV), k.to(DEV), v.to(DEV), HQ, HKV).float().cpu()
            o2 = c2.attend(layer, q.float(), k.float(), v.float(), HQ, HKV)
            for b in range(3):
                rows = slice(offs[b], offs[b] + ntok[b])
                torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=ATOL, rtol=RTOL)
        mgr.end_forward(c1)
        ref.end_forward(c2)
    torch.cuda.synchronize()
    assert torch.equal(mgr.k.cpu().float(), ref.k) and torch.equal(mgr.v.cpu().float(), ref.v)


def test_factory_on_gpu():
    _log("cache: factory")
    import types
    from nanoslg_amd import kv_cache as KC
    hf = types.SimpleNamespace(num_hidden_layers=2, num_key_value_heads=8, num_attention_heads=32,
                               hidden_size=4096)
    m = types.SimpleNamespace(kv_backend="auto", page_size=16, max_kv_pages=64)
    mgr = KC.create_cache_manager(hf, None, "cuda:0", torch.float16, m)
    assert isinstance(mgr, KC.PagedKVCache) and mgr.pool.k.is_cuda and mgr.cfg.max_pages == 64
    m = types.SimpleNamespace(kv_backend="auto", page_size=16)  # pages sized from free memory
    mgr = KC.create_cache_manager(hf, None, "cuda:0", torch.float16, m)
    assert 64 <= mgr.cfg.max_pages <= 65536


def test_forward_plan_on_device_equals_host_plan(monkeypatch):
    """Multi-token forwards (ragged, with input offsets, over shared prefixes) planned
    with the per-token arrays expanded on the device (the native host planner and
    nslg_forward_plan_csr) equal, entry for entry, the numpy path's host plan of the
    same forward; tokens_used, pool bytes and outputs are identical."""
    _log("forward plan device vs host")
    from nanoslg_amd import kv_cache as KC
    g = torch.Generator().manual_seed(17)
    mk = lambda: make(ps=16, pages=600, prefix=True)[0]  # noqa: E731
    host, dev = mk(), mk()
    prompt = list(range(3, 300))
    for m in (host, dev):
        m.allocate_sequence("p", token_ids=prompt)
    steps = [(["p"], [297], [0])]
    ids = ["a", "b", "c"]
    for ntok, offs in [([40, 400, 7], [3, 0, 20]), ([1, 1, 1], None), ([300, 2, 33], [0, 10, 0])]:
        steps.append((ids, ntok, offs))
    for sids, ntok, offs in steps:
        offs = offs or [0] * len(sids)
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(len(sids), S, HQ, D, generator=g).half().to(DEV)
        k = torch.randn(len(sids), S, HKV, D, generator=g).half().to(DEV)
        v = torch.randn(len(sids), S, HKV, D, generator=g).half().to(DEV)
        if sids == ids and "a" not in host.seqs:
            for m in (host, dev):
                m.release_sequence("p")
                for i, s in enumerate(ids):
                    m.allocate_sequence(s, token_ids=prompt[:200] + [900 + i] * (5 + i))
        outs, plans = [], []
        # host: the numpy path's host plan; dev: the native planner and the device launch
        for m, thr, native in ((host, 10 ** 9, False), (dev, 1, True)):
            monkeypatch.setattr(KC.PagedCacheContext, "DEVICE_PLAN_TOKENS", thr)
            m.NATIVE_PLAN = native
            c = m.begin_forward(sids, ntok, offs)
            outs.append([c.attend(layer, q, k, v, HQ, HKV) for layer in range(L)])
            plans.append(c.plan)
            m.end_forward(c)
        torch.cuda.synchronize()
        a, b = plans
        for name in ("slot", "pos_i32", "indptr", "indices", "lpl", "qo_indptr", "q_rows"):
            x, y = getattr(a, name).cpu().long(), getattr(b, name).cpu().long()
            if name == "indices":
                n = int(a.indptr[-1])
                x, y = x[:n], y[:n]
            assert torch.equal(x, y), name
        for oa, ob in zip(*outs):
            assert torch.equal(oa, ob)
        assert np.array_equal(host.pool.tokens_used, dev.pool.tokens_used)
    assert torch.equal(host.pool.k, dev.pool.k) and torch.equal(host.pool.v, dev.pool.v)


def test_native_plan_grows_the_upload_buffer():
    """A forward whose sequences' tables exceed the pinned upload buffer (two sequences
    of 40,000 pages, each table uploaded whole on its first forward): the native
    planner asks for a larger buffer, the staging ring grows it, and the CSR, the last
    page lengths and the decode step's slots and positions equal the block tables'
    closed form (kv_cache.py:598-615, 575-594)."""
    _log("native plan: upload buffer growth")
    from nanoslg_amd import kv_cache as KC
    ps, pages = 16, 80_100
    cfg = KC.KVCacheConfig(num_layers=1, num_kv_heads=1, num_qo_heads=1, head_dim=64, page_size=ps,
                           max_pages=pages, dtype=torch.float16, device=DEV, enable_prefix_caching=False,
                           backend="paged")
    mgr = KC.PagedKVCache(cfg)
    lens = [40_000 * ps - 5, 39_990 * ps]
    assert sum(-(-n // ps) for n in lens) > mgr.STAGING_INTS
    for i, n in enumerate(lens):
        mgr.allocate_sequence(f"s{i}", num_tokens=n)
        mgr.seqs[f"s{i}"].num_tokens = n
    ctx = mgr.begin_forward(["s0", "s1"], [1, 1])
    torch.cuda.synchronize()
    plan = ctx.plan
    tabs = [mgr.seqs[f"s{i}"].bt[:mgr.seqs[f"s{i}"].n_pages].astype(np.int64) for i in range(2)]
    new = [n + 1 for n in lens]
    npg = [-(-n // ps) for n in new]
    assert plan.indptr.cpu().tolist() == [0, npg[0], npg[0] + npg[1]]
    assert np.array_equal(plan.indices[:sum(npg)].cpu().numpy(), np.concatenate([t[:k] for t, k in zip(tabs, npg)]))
    assert plan.lpl.cpu().tolist() == [n - (k - 1) * ps for n, k in zip(new, npg)]
    assert plan.slot.cpu().tolist() == [int(t[n // ps]) * ps + n % ps for t, n in zip(tabs, lens)]
    assert plan.pos_i32.cpu().tolist() == lens
    mgr.end_forward(ctx)
