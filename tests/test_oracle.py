"""Pins of the CPU oracle (oracle/kv_oracle.py) against closed forms, brute
force and library routines — so that the oracle can be trusted as the checker
of the HIP kernels. The reference ships no tests or golden vectors for this
path, so these are the pins."""
import math
import random

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import kv_oracle as O


def _rand(*shape, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g, dtype=dtype)


# ---------------------------------------------------------------- attention pins


def test_sdpa_gqa_matches_repeat_interleave_formulation():
    # kv_cache.py:52-54: without enable_gqa the reference repeats each KV head Hq/Hkv
    # times, so q head h reads kv head h // (Hq/Hkv).
    q, k, v = _rand(2, 8, 3, 16, seed=1), _rand(2, 2, 7, 16, seed=2), _rand(2, 2, 7, 16, seed=3)
    ref = F.scaled_dot_product_attention(q, k.repeat_interleave(4, 1), v.repeat_interleave(4, 1))
    assert torch.allclose(O.sdpa_gqa(q, k, v), ref, atol=1e-6)
    # a plausible mistake (q head h -> kv head h % Hkv) is caught
    wrong = F.scaled_dot_product_attention(q, k.repeat(1, 4, 1, 1), v.repeat(1, 4, 1, 1))
    assert not torch.allclose(wrong, ref, atol=1e-3)


@pytest.mark.parametrize("Hq,Hkv,Sq,Skv,D", [(8, 2, 3, 7, 16), (4, 4, 1, 5, 8), (8, 1, 2, 9, 32)])
def test_sdpa_gqa_matches_f64_brute_force(Hq, Hkv, Sq, Skv, D):
    q, k, v = _rand(1, Hq, Sq, D, seed=4), _rand(1, Hkv, Skv, D, seed=5), _rand(1, Hkv, Skv, D, seed=6)
    vis = np.tril(np.ones((Sq, Skv), bool), k=Skv - Sq)  # bottom-right causal
    mask = torch.zeros(Sq, Skv).masked_fill(torch.from_numpy(~vis), float("-inf"))
    got = O.sdpa_gqa(q, k, v, attn_mask=mask[None, None])[0].numpy()
    ref = O.sdpa_brute_f64(q[0].numpy(), k[0].numpy(), v[0].numpy(), vis)
    np.testing.assert_allclose(got, ref, atol=2e-6, rtol=1e-5)


def test_brute_force_closed_forms():
    rng = np.random.default_rng(0)
    # one key: output is that key's value, whatever q is
    q, k, v = rng.normal(size=(4, 1, 8)), rng.normal(size=(2, 1, 8)), rng.normal(size=(2, 1, 8))
    out = O.sdpa_brute_f64(q, k, v)
    np.testing.assert_allclose(out[:, 0], v[np.arange(4) // 2, 0], atol=1e-12)
    # identical keys: softmax is uniform, output is the mean of V
    k = np.repeat(rng.normal(size=(2, 1, 8)), 6, axis=1)
    v = rng.normal(size=(2, 6, 8))
    out = O.sdpa_brute_f64(q, k, v)
    np.testing.assert_allclose(out[:, 0], v[np.arange(4) // 2].mean(axis=1), atol=1e-12)
    # one dominant score: output is the value of that key
    k = np.zeros((1, 5, 8))
    k[0, 3] = 100.0
    q = np.ones((1, 1, 8))
    v = rng.normal(size=(1, 5, 8))
    np.testing.assert_allclose(O.sdpa_brute_f64(q, k, v)[0, 0], v[0, 3], atol=1e-9)


def test_causal_mask_fast_paths_and_pattern():
    f = O.build_causal_mask
    assert f(1, 4, [0], [4], [0], [4], 4) is None                      # single prefill from 0
    assert f(3, 1, [5, 5, 5], [1, 1, 1], [0, 0, 0], [6, 6, 6], 6) is None  # uniform decode
    assert f(2, 3, [0, 0], [3, 3], [0, 0], [3, 3], 3) is None          # uniform prefill from 0
    m = f(2, 1, [3, 5], [1, 1], [0, 0], [4, 6], 6)                      # mixed-length decode
    assert m.shape == (2, 1, 1, 6)
    assert torch.equal(torch.isfinite(m[0, 0, 0]), torch.tensor([1, 1, 1, 1, 0, 0], dtype=torch.bool))
    assert torch.equal(torch.isfinite(m[1, 0, 0]), torch.ones(6, dtype=torch.bool))
    # left-padded prefill: seq 1 has 2 new tokens at offset 1 after 3 cached ones
    m = f(2, 3, [0, 3], [3, 2], [0, 1], [3, 5], 5)
    vis1 = torch.isfinite(m[1, 0])
    assert not vis1[0].any()                                            # pad row fully masked
    assert torch.equal(vis1[1], torch.tensor([1, 1, 1, 1, 0], dtype=torch.bool))
    assert torch.equal(vis1[2], torch.tensor([1, 1, 1, 1, 1], dtype=torch.bool))
    assert m.dtype == torch.float32 and m[0, 0, 0, 1].item() == float("-inf")
    m16 = f(2, 1, [3, 5], [1, 1], [0, 0], [4, 6], 6, dtype=torch.float16)
    assert m16[0, 0, 0, 5].item() == -65504.0


def test_position_ids_closed_form():
    pos = O.position_ids([4, 0], [2, 3], [1, 0])
    assert pos.tolist() == [[0, 4, 5], [0, 1, 2]]
    assert O.position_ids([4, 0], [2, 3], [1, 0], S=2).tolist() == [[0, 4], [0, 1]]
    assert O.position_ids([7], [1], [0], S=3).tolist() == [[7, 0, 0]]


# ---------------------------------------------------------------- paging pins


def test_plan_csr_closed_form():
    indptr, indices, lpl = O.plan_csr([[5, 9, 2], [7], [3, 4]], [33, 16, 40], 16)
    assert indptr.tolist() == [0, 3, 4, 7]
    # seq 2 needs 3 pages but has 2: the missing entry is the null page 0 (kv_cache.py:606-607)
    assert indices.tolist() == [5, 9, 2, 7, 3, 4, 0]
    assert lpl.tolist() == [1, 16, 8]
    assert O.seq_lens_from_csr(indptr, lpl, 16) == [33, 16, 40]


def test_append_then_gather_round_trip_and_identity_table():
    rng = np.random.default_rng(1)
    P, ps, H, D = 32, 4, 2, 8
    pool = np.zeros((P * ps, H, D), np.float16)
    lens = [7, 12, 1]
    perm = rng.permutation(np.arange(1, P))
    tables, off = [], 0
    for L in lens:
        n = math.ceil(L / ps)
        tables.append(perm[off:off + n].tolist())
        off += n
    rows = [rng.normal(size=(L, H, D)).astype(np.float16) for L in lens]
    for bt, r in zip(tables, rows):
        slots = [bt[t // ps] * ps + t % ps for t in range(len(r))]
        O.append_rows(pool, r, np.array(slots))
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    got = O.gather_rows(pool, ps, indptr, indices, lpl, 12)
    for b, r in enumerate(rows):
        assert np.array_equal(got[b, :len(r)], r)
        assert not got[b, len(r):].any()
    # identity table over a contiguous pool (page_size = Smax) is a plain slice
    Smax = 12
    cpool = rng.normal(size=(3 * Smax, H, D)).astype(np.float16)
    g2 = O.gather_rows(cpool, Smax, np.arange(4), np.array([2, 0, 1]), np.array([5, 12, 3]), 12)
    assert np.array_equal(g2[0, :5], cpool[2 * Smax:2 * Smax + 5])
    assert np.array_equal(g2[1], cpool[0:12])
    # negative / out-of-range slots are skipped
    before = pool.copy()
    O.append_rows(pool, rows[0][:2], np.array([-1, P * ps]))
    assert np.array_equal(pool, before)


def test_zero_and_copy_pages():
    rng = np.random.default_rng(2)
    pool = rng.normal(size=(3, 6, 4, 2, 8)).astype(np.float32)
    src = pool.copy()
    O.copy_pages(pool, [1, 2], [4, 5])
    assert np.array_equal(pool[:, 4], src[:, 1]) and np.array_equal(pool[:, 5], src[:, 2])
    assert np.array_equal(pool[:, :4], src[:, :4])
    O.zero_pages(pool, [4, 99])
    assert not pool[:, 4].any() and np.array_equal(pool[:, 5], src[:, 2])


def test_pagepool_invariants_random_ops():
    rnd = random.Random(3)
    pool = O.PagePoolRef(2, 20, 4, 1, 4)
    held = []
    for _ in range(400):
        op = rnd.random()
        if op < 0.5:
            n = rnd.randint(1, 5)
            before = pool.num_free
            got = pool.alloc(n)
            if got is None:
                assert before < n and pool.num_free == before
            else:
                assert 0 not in got and len(set(got)) == n
                assert not set(got) & set(held)
                for p in got:
                    assert not pool.k[:, p].any()
                    pool.k[:, p] = 1.0
                held.extend(got)
        elif held:
            p = held.pop(rnd.randrange(len(held)))
            pool.release(p)
        assert pool.num_free + len(held) == 19
        assert pool.ref_count[0] == 1
    # double release of a free page does not duplicate it
    p = pool.alloc(1)[0]
    pool.release(p)
    pool.release(p)
    assert pool.num_free + len(held) == 19


def _insert_seq(tree, pool, tokens):
    ps = tree.ps
    n = len(tokens) // ps
    pages = pool.alloc(n)
    tree.insert(tokens[:n * ps], pages)
    for p in pages:  # the sequence itself releases its refs; the tree keeps one
        pool.release(p)
    return pages


def test_radix_match_is_longest_common_full_page_prefix():
    rnd = random.Random(4)
    ps = 4
    for trial in range(30):
        pool = O.PagePoolRef(1, 200, ps, 1, 2)
        tree = O.RadixTreeRef(ps, pool)
        vocab = [rnd.randint(0, 3) for _ in range(2)]
        seqs, pagemap = [], []
        for _ in range(rnd.randint(1, 5)):
            s = [rnd.choice(vocab) for _ in range(rnd.randint(0, 20))]
            pages = _insert_seq(tree, pool, s)
            seqs.append(s)
            pagemap.append(pages)
        q = [rnd.choice(vocab) for _ in range(rnd.randint(0, 24))]
        plen, pages = tree.match(q)
        # brute force: longest full-page prefix of q shared with any inserted sequence
        best = 0
        for s in seqs:
            k = 0
            while (k + 1) * ps <= min(len(s), len(q)) and s[k * ps:(k + 1) * ps] == q[k * ps:(k + 1) * ps]:
                k += 1
            best = max(best, k)
        assert plen == best * ps and len(pages) == best
        # the page for each matched prefix page is the one inserted first for that prefix
        for i, p in enumerate(pages):
            first = next(pm[i] for s, pm in zip(seqs, pagemap)
                         if len(s) >= (i + 1) * ps and s[:(i + 1) * ps] == q[:(i + 1) * ps])
            assert p == first


def test_radix_eviction_lru_and_pins():
    ps = 2
    pool = O.PagePoolRef(1, 10, ps, 1, 2)
    tree = O.RadixTreeRef(ps, pool)
    a = _insert_seq(tree, pool, [1, 1, 2, 2])
    b = _insert_seq(tree, pool, [3, 3])
    assert tree.cached_pages == 3 and pool.num_free == 6
    tree.match([3, 3])            # b is now most recent
    tree.add_refs([1, 1])         # pin a's first page
    freed = tree.evict_lru(1)
    assert freed == 1 and pool.ref_count[a[1]] == 0   # a's second page (unpinned, LRU) went
    assert pool.ref_count[a[0]] == 1 and pool.ref_count[b[0]] == 1
    tree.dec_refs([1, 1])
    assert tree.evict_lru(5) == 2 and pool.num_free == 9 and tree.cached_pages == 0


def test_radix_match_over_an_evicted_interior_page():
    """Three cached pages on one path, the middle one evicted (its node keeps its
    children, kv_cache.py:512-516). The reference's match walks on and returns the
    first and third pages, a prefix with a gap (:459-472); with stop_at_gap the
    match ends at the evicted page."""
    ps = 2
    toks = [1, 1, 2, 2, 3, 3]
    for stop, want_pages in ((False, [0, 2]), (True, [0])):
        pool = O.PagePoolRef(1, 10, ps, 1, 2)
        tree = O.RadixTreeRef(ps, pool, stop_at_gap=stop)
        pages = _insert_seq(tree, pool, toks)
        node = tree.root
        for t in toks[:4]:
            node = node.children[t]
        assert node.page_id == pages[1]
        node.page_id = -1           # the eviction of the middle page
        pool.release(pages[1])
        plen, got = tree.match(toks)
        assert got == [pages[i] for i in want_pages]
        assert plen == len(got) * ps


# ---------------------------------------------------------------- backend pins


def _run_both(seed, dtype=torch.float32):
    """Same prefill + decode sequence through ContiguousRef and PagedRef."""
    torch.manual_seed(seed)
    L, Hq, Hkv, D, ps = 2, 4, 2, 8, 4
    cont = O.ContiguousRef(L, 3, 40, Hkv, D, dtype)
    paged = O.PagedRef(L, 64, ps, Hkv, D, dtype, enable_prefix_caching=False)
    ids = ["a", "b", "c"]
    lens = [5, 9, 3]
    for s, n in zip(ids, lens):
        cont.allocate_sequence(s)
        paged.allocate_sequence(s, num_tokens=n)
    outs = []
    steps = [(lens, [max(lens) - n for n in lens])] + [([1, 1, 1], [0, 0, 0])] * 4
    for ntok, offs in steps:
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(3, S, Hq, D, dtype=dtype)
        k = torch.randn(3, S, Hkv, D, dtype=dtype)
        v = torch.randn(3, S, Hkv, D, dtype=dtype)
        c1 = cont.begin_forward(ids, ntok, offs)
        c2 = paged.begin_forward(ids, ntok, offs)
        for layer in range(L):
            o1 = c1.attend(layer, q, k, v, Hq, Hkv)
            o2 = c2.attend(layer, q, k, v, Hq, Hkv)
            outs.append((o1, o2, ntok, offs))
        cont.end_forward(c1)
        paged.end_forward(c2)
    return cont, paged, outs


def test_contiguous_and_paged_oracles_agree():
    cont, paged, outs = _run_both(0)
    for o1, o2, ntok, offs in outs:
        for b in range(3):
            rows = slice(offs[b], offs[b] + ntok[b])  # pad rows: zeros here, masked averages in the reference
            torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=1e-5, rtol=1e-5)
    for b, s in enumerate(["a", "b", "c"]):
        n = paged.seqs[s].num_tokens
        for layer in range(2):
            k, v = paged.logical_kv(s, layer)
            assert torch.equal(k, cont.k[layer, b, :n]) and torch.equal(v, cont.v[layer, b, :n])


def test_contiguous_oracle_matches_brute_force():
    torch.manual_seed(5)
    Hq, Hkv, D = 4, 2, 8
    c = O.ContiguousRef(1, 1, 16, Hkv, D)
    c.allocate_sequence("s")
    q = torch.randn(1, 6, Hq, D)
    k = torch.randn(1, 6, Hkv, D)
    v = torch.randn(1, 6, Hkv, D)
    ctx = c.begin_forward(["s"], [6])
    out = ctx.attend(0, q, k, v, Hq, Hkv).reshape(6, Hq, D).transpose(0, 1).numpy()
    ref = O.sdpa_brute_f64(q[0].transpose(0, 1).numpy(), k[0].transpose(0, 1).numpy(),
                           v[0].transpose(0, 1).numpy(), np.tril(np.ones((6, 6), bool)))
    np.testing.assert_allclose(out, ref, atol=2e-6)


def test_paged_oracle_cow_order_rule():
    # refcount R held by R sharers: the first R-1 writers copy, the last writes in place
    ps = 4
    p = O.PagedRef(1, 32, ps, 1, 2, enable_prefix_caching=False)
    shared = p.pool.alloc(1)[0]
    p.pool.k[:, shared] = 7.0
    for s in ["x", "y", "z"]:
        p.allocate_sequence(s)
        p.seqs[s].block_table = [shared]
        p.seqs[s].num_tokens = 2
    p.pool.add_ref(shared)
    p.pool.add_ref(shared)          # refcount 3
    p.pool.release(shared)          # drop the allocation's own ref -> 2 ... rebuild to 3
    p.pool.add_ref(shared)
    assert p.pool.ref_count[shared] == 3
    ctx = p.begin_forward(["x", "y", "z"], [1, 1, 1])
    assert [e[0] for e in ctx.cow_events] == [shared, shared]
    assert p.seqs["z"].block_table == [shared]
    assert p.seqs["x"].block_table != [shared] and p.seqs["y"].block_table != [shared]
    assert p.pool.ref_count[shared] == 1
    for s in ["x", "y"]:
        assert torch.equal(p.pool.k[:, p.seqs[s].block_table[0]], p.pool.k[:, shared])


def test_timed_contiguous_decode_runs():
    sec, threads = O.timed_contiguous_decode(num_steps=4, prefill=32, warmup=1, repeats=1)
    assert sec > 0 and threads >= 1
