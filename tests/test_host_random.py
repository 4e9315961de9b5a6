"""Randomised serving traffic through the host layer against the oracle.

Each seed drives one PagedKVCache (CPU stand-in kernels, tests/fake_kernels.py) and
the oracle's PagedRef with the same stream of calls, the way nanoslg's worker
drives its manager (worker.py:169-213, 398-426; kv_cache.py:707-777):

  * admissions with token ids from a 3-symbol vocabulary, so prompts share
    prefixes and the radix tree matches, inserts and evicts pages;
  * ragged prefill forwards of several admitted sequences with left padding
    (input offsets), decode forwards of every running sequence (steady decode
    batches are planned on the device after the first);
  * partial pages shared by reference (add_ref, as kv_cache.py:713 does for full
    pages) so that the next write copies them (copy-on-write order rule);
  * releases (which cache the full pages in the tree) and OOM on both sides.

After every forward: outputs (rows with new tokens), positions, the number of
copy-on-writes, free pages, cached pages and every sequence's K/V read through
its block table are compared; pad rows must be zero."""
import random

import pytest
import torch

import fake_kernels as FK
from nanoslg_amd import kv_cache as KC
from oracle import kv_oracle as O

L = 2
CPU = dict(device=None, dtype=torch.float32, HQ=4, HKV=2, D=8, atol=1e-5, rtol=1e-5)


def _make(ps, pages, env):
    partial = env.get("partial", True)
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=env["HKV"], num_qo_heads=env["HQ"], head_dim=env["D"],
                           page_size=ps, max_pages=pages, dtype=env["dtype"], device=env["device"],
                           enable_prefix_caching=True, backend="paged", share_partial_pages=partial)
    kernels = FK if env["device"] is None else None
    mgr = KC.PagedKVCache(cfg, kernels=kernels)
    if env.get("arena"):  # a small device block-table arena: it grows and rows move often
        mgr._tables = KC._BlockTableArena(mgr.pool.device, env["arena"])
    # the oracle's match stops at an evicted page, as the product's does (the
    # reference's match returns the pages past it, a block table with a gap)
    return (mgr, O.PagedRef(L, pages, ps, env["HKV"], env["D"], torch.float32, enable_prefix_caching=True,
                            stop_at_gap=True, share_partial_pages=partial))


def _logical(cache, sid, layer, ps):
    st = cache.seqs[sid]
    bt = st.block_table
    n = st.num_tokens
    if n == 0:
        return None, None
    rows = torch.tensor([bt[t // ps] * ps + t % ps for t in range(n)], device=cache.pool.k.device)
    k = cache.pool.k[layer].reshape(-1, *cache.pool.k.shape[-2:])[rows]
    v = cache.pool.v[layer].reshape(-1, *cache.pool.v.shape[-2:])[rows]
    return k.cpu().float(), v.cpu().float()


def _forward(mgr, ref, ids, ntok, offs, g, env):
    S = max(o + n for o, n in zip(offs, ntok))
    B = len(ids)
    HQ, HKV, D, dt = env["HQ"], env["HKV"], env["D"], env["dtype"]
    # inputs in the pool's dtype; the oracle gets the same values in fp32
    q = torch.randn(B, S, HQ, D, generator=g).to(dt)
    k = torch.randn(B, S, HKV, D, generator=g).to(dt)
    v = torch.randn(B, S, HKV, D, generator=g).to(dt)
    dev = env["device"]
    qd, kd, vd = (q, k, v) if dev is None else (q.to(dev), k.to(dev), v.to(dev))
    try:
        c1 = mgr.begin_forward(ids, ntok, offs)
    except RuntimeError as e:
        with pytest.raises(RuntimeError):
            ref.begin_forward(ids, ntok, offs)
        return str(e)
    c2 = ref.begin_forward(ids, ntok, offs)
    assert c1.start_positions == c2.start_positions and c1.seq_lens == c2.seq_lens
    assert torch.equal(c1.get_position_ids(S).cpu(), c2.get_position_ids(S))
    assert len(c1.cow_pairs) == len(c2.cow_events)
    for layer in range(L):
        o1 = c1.attend(layer, qd, kd, vd, HQ, HKV).cpu().float()
        o2 = c2.attend(layer, q.float(), k.float(), v.float(), HQ, HKV)
        for b in range(B):
            rows = slice(offs[b], offs[b] + ntok[b])
            torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=env["atol"], rtol=env["rtol"])
            pad = torch.ones(S, dtype=torch.bool)
            pad[rows] = False
            assert not o1[b, pad].any()
    mgr.end_forward(c1)
    ref.end_forward(c2)
    return None


def check_device_tables(mgr):
    """The device-resident block tables: every live sequence's row holds its host
    table up to the synced mark, and the rows of live sequences do not overlap."""
    tables = mgr._tables.dev.cpu()
    spans = []
    for st in mgr.seqs.values():
        if st.row < 0:
            continue
        # (a table may outgrow its row between forwards: the next forward moves it)
        assert 0 <= st.synced <= min(st.n_pages, st.row_cap)
        assert st.row + st.row_cap <= tables.numel()
        assert tables[st.row:st.row + st.synced].tolist() == st.bt[:st.synced].tolist(), st.seq_id
        spans.append((st.row, st.row + st.row_cap))
    spans.sort()
    assert all(a[1] <= b[0] for a, b in zip(spans, spans[1:]))


def tree_pages(tree):
    """The cached pages of a radix tree as (token path, pins, last access): the
    product's page tree and the oracle's per-token trie must hold the same set (page
    ids aside: allocation order is not part of the contract)."""
    out = set()
    stack = [(tree.root, ())]
    while stack:
        nd, path = stack.pop()
        if nd.page_id >= 0:
            out.add((path, nd.ref, int(nd.last_access)))
        for k, ch in nd.children.items():
            stack.append((ch, path + (tuple(k) if isinstance(k, tuple) else (k,))))
        for k, ch in getattr(nd, "partials", {}).items():
            stack.append((ch, path + tuple(k)))
    return out


def _check(mgr, ref, live, ps):
    assert mgr.pool.num_free == ref.pool.num_free
    assert mgr.tree.cached_pages == ref.tree.cached_pages
    assert tree_pages(mgr.tree) == tree_pages(ref.tree)
    check_device_tables(mgr)
    for sid in live:
        assert mgr.seqs[sid].num_tokens == ref.seqs[sid].num_tokens
        for layer in range(L):
            k1, v1 = _logical(mgr, sid, layer, ps)
            k2, v2 = ref.logical_kv(sid, layer)
            if k1 is None:
                assert k2.shape[0] == 0
            else:
                assert torch.equal(k1, k2) and torch.equal(v1, v2)


@pytest.mark.parametrize("seed,ps,pages", [(1, 4, 48), (2, 2, 40), (3, 4, 24), (4, 3, 64), (5, 1, 60),
                                           (6, 4, 20), (7, 2, 24), (8, 8, 40), (9, 3, 30), (10, 16, 12)])
def test_random_serving_traffic_matches_oracle(seed, ps, pages):
    run_traffic(seed, ps, pages, CPU)


@pytest.mark.parametrize("seed,ps,pages", [(1, 4, 48), (3, 4, 24), (5, 1, 60), (8, 8, 40)])
def test_random_serving_traffic_full_pages_only(seed, ps, pages):
    """The same traffic with partial-page sharing off: the reference's rule (only full
    pages are cached and matched, kv_cache.py:459-486)."""
    run_traffic(seed, ps, pages, dict(CPU, partial=False))


@pytest.mark.parametrize("seed,ps,pages", [(11, 1, 90), (12, 2, 60), (13, 1, 40)])
def test_random_serving_traffic_with_a_small_block_table_arena(seed, ps, pages):
    """The same traffic with the device block tables in a 16-entry arena: it grows
    (device copy) and tables move to larger rows (re-uploaded) many times."""
    run_traffic(seed, ps, pages, dict(CPU, arena=16))


@pytest.mark.parametrize("seed,ps,pages", [(1, 4, 48), (5, 1, 60), (8, 8, 40), (10, 16, 12)])
def test_random_serving_traffic_numpy_planner(monkeypatch, seed, ps, pages):
    """The same traffic with the native planner off: every forward planned by the numpy
    path (host plans below 256 new tokens, device plans above), which otherwise only
    takes the forwards that copy a shared page."""
    monkeypatch.setattr(KC.PagedKVCache, "NATIVE_PLAN", False)
    run_traffic(seed, ps, pages, CPU)


@pytest.mark.parametrize("native", [True, False])
@pytest.mark.parametrize("seed,ps,pages", [(21, 4, 48), (22, 1, 60), (23, 16, 12), (25, 3, 40)])
def test_random_serving_traffic_device_planned(monkeypatch, seed, ps, pages, native):
    """The same traffic with every forward that is not a plain decode step planned on
    the device (the token threshold lowered from 256 to 1), its host part from the
    native planner or from the numpy path."""
    monkeypatch.setattr(KC.PagedCacheContext, "DEVICE_PLAN_TOKENS", 1)
    monkeypatch.setattr(KC.PagedKVCache, "NATIVE_PLAN", native)
    run_traffic(seed, ps, pages, CPU)


def run_traffic(seed, ps, pages, env):
    """One seeded serving run (see the module docstring); env: device (None = the
    CPU stand-in kernels), pool dtype, head shape, output tolerance."""
    rnd = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    mgr, ref = _make(ps, pages, env)
    pending = {}   # admitted, prompt not yet prefilled: sid -> new tokens to feed
    running = []   # prefilled, decoding
    tokens = {}
    counts = {"prefill": 0, "decode": 0, "cow": 0, "oom": 0, "release": 0, "shared": 0}
    for it in range(120):
        r = rnd.random()
        if r < 0.25 and len(pending) + len(running) < 6:
            sid = f"s{it}"
            toks = [rnd.randint(0, 2) for _ in range(rnd.randint(1, 3 * ps + 4))]
            if tokens and rnd.random() < 0.35:
                # a prompt that continues an earlier sequence's tokens (a released one's are
                # cached, with its last partial page when partial pages are shared)
                base = tokens[rnd.choice(sorted(tokens))]
                cut = len(base) if rnd.random() < 0.5 else rnd.randint(1, len(base))
                toks = base[:cut] + toks[:rnd.randint(0, ps)]
            try:
                p1 = mgr.allocate_sequence(sid, token_ids=toks)
            except RuntimeError:
                with pytest.raises(RuntimeError):
                    ref.allocate_sequence(sid, token_ids=toks)
                counts["oom"] += 1
                continue
            p2 = ref.allocate_sequence(sid, token_ids=toks)
            assert p1 == p2
            tokens[sid] = list(toks)
            if len(toks) - p1 > 0:
                pending[sid] = len(toks) - p1
            else:
                running.append(sid)  # a full prefix hit: straight to decode
        elif r < 0.45 and pending:
            ids = sorted(pending)[: rnd.randint(1, len(pending))]
            ntok = [pending[s] for s in ids]
            offs = [rnd.randint(0, 2) for _ in ids]
            err = _forward(mgr, ref, ids, ntok, offs, g, env)
            if err:
                counts["oom"] += 1
                continue
            counts["prefill"] += 1
            for s in ids:
                del pending[s]
                running.append(s)
        elif r < 0.8 and running:
            # decode: usually the whole running batch (steady steps), sometimes a
            # subset (a batch change), sometimes together with pending prompts (a
            # mixed forward of prefill and decode rows)
            mode = rnd.random()
            ids = list(running)
            if mode < 0.2 and len(running) > 1:
                ids = sorted(rnd.sample(running, rnd.randint(1, len(running) - 1)))
            ntok = [1] * len(ids)
            if 0.2 <= mode < 0.35 and pending:
                extra = sorted(pending)[: rnd.randint(1, len(pending))]
                ids += extra
                ntok += [pending[s] for s in extra]
            offs = [rnd.randint(0, 1) if n > 1 else 0 for n in ntok]
            err = _forward(mgr, ref, ids, ntok, offs, g, env)
            if err:
                counts["oom"] += 1
                continue
            counts["decode"] += 1
            for s, n in zip(ids, ntok):
                if s in pending:
                    del pending[s]
                    running.append(s)
                    counts["prefill"] += 1
                    continue
                tok = rnd.randint(0, 2)
                tokens[s].append(tok)
                mgr.append_token_ids(s, [tok])
                ref.append_token_ids(s, [tok])
        elif r < 0.88 and len(running) >= 2:
            # share the last (partial) page of one running sequence with another one
            # admitted on it: the next write of either copies it, in batch order
            src = rnd.choice(running)
            st1, st2 = mgr.seqs[src], ref.seqs[src]
            n = st1.num_tokens
            if n == 0 or n % ps == 0:
                continue
            sid = f"c{it}"
            for impl, st in ((mgr, st1), (ref, st2)):
                impl.allocate_sequence(sid)
                pages_ = list(st.block_table[: (n + ps - 1) // ps])
                for p in pages_:
                    impl.pool.add_ref(p)
                nst = impl.seqs[sid]
                if hasattr(nst, "bt"):
                    nst.extend(pages_)
                else:
                    nst.block_table = list(pages_)
                nst.num_tokens = n
            tokens[sid] = list(tokens[src][:n])
            running.append(sid)
            counts["shared"] += 1
        elif running or pending:
            sid = rnd.choice(running + sorted(pending))
            mgr.release_sequence(sid)
            ref.release_sequence(sid)
            if sid in pending:
                del pending[sid]
            else:
                running.remove(sid)
            counts["release"] += 1
        _check(mgr, ref, running + sorted(pending), ps)
    # the traffic reached the paths it is meant to cover
    assert counts["prefill"] >= 3 and counts["decode"] >= 10 and counts["release"] >= 2, counts
    for s in running + sorted(pending):
        mgr.release_sequence(s)
        ref.release_sequence(s)
    assert mgr.pool.num_free == ref.pool.num_free


def run_contiguous_traffic(seed, env, max_batch=4, max_seq=64):
    """The contiguous backend (kv_cache.py:227-379) over random forwards: every
    forward carries all live sequences in allocation order (the reference indexes
    its pool by batch row, which equals the slot only then), each with a random
    number of new tokens (prefill and decode rows in one forward) and a random left
    pad; sequences are released all together (the reference resets its slot counter
    only then). Outputs and the pool bytes against the oracle after every forward."""
    rnd = random.Random(seed)
    g = torch.Generator().manual_seed(seed)
    HQ, HKV, D, dt = env["HQ"], env["HKV"], env["D"], env["dtype"]
    cfg = KC.KVCacheConfig(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, max_batch_size=max_batch,
                           max_seq_len=max_seq, dtype=dt, device=env["device"], backend="contiguous")
    mgr = KC.ContiguousKVCache(cfg, kernels=FK if env["device"] is None else None)
    ref = O.ContiguousRef(L, max_batch, max_seq, HKV, D)
    live, lens, forwards = [], {}, 0
    for it in range(60):
        r = rnd.random()
        if (r < 0.2 or not live) and len(live) < max_batch:
            sid = f"s{it}"
            mgr.allocate_sequence(sid)
            ref.allocate_sequence(sid)
            live.append(sid)
            lens[sid] = 0
        elif r < 0.9:
            room = [max_seq - lens[s] for s in live]
            if min(room) < 1:
                continue
            ntok = [rnd.choice([1, 1, 1, rnd.randint(1, min(12, rm))]) for rm in room]
            offs = [rnd.randint(0, 2) for _ in live]
            if all(n == 1 for n in ntok):
                # a decode forward is one token wide, unpadded (worker.py:398-426): the
                # reference's decode write takes input column 0 (kv_cache.py:301-303)
                offs = [0] * len(live)
            S = max(o + n for o, n in zip(offs, ntok))
            q = torch.randn(len(live), S, HQ, D, generator=g).to(dt)
            k = torch.randn(len(live), S, HKV, D, generator=g).to(dt)
            v = torch.randn(len(live), S, HKV, D, generator=g).to(dt)
            dev = env["device"]
            qd, kd, vd = (q, k, v) if dev is None else (q.to(dev), k.to(dev), v.to(dev))
            c1, c2 = mgr.begin_forward(live, ntok, offs), ref.begin_forward(live, ntok, offs)
            assert torch.equal(c1.get_position_ids(S).cpu(), c2.get_position_ids(S))
            for layer in range(L):
                o1 = c1.attend(layer, qd, kd, vd, HQ, HKV).cpu().float()
                o2 = c2.attend(layer, q.float(), k.float(), v.float(), HQ, HKV)
                for b in range(len(live)):
                    rows = slice(offs[b], offs[b] + ntok[b])
                    torch.testing.assert_close(o1[b, rows], o2[b, rows], atol=env["atol"], rtol=env["rtol"])
            mgr.end_forward(c1)
            ref.end_forward(c2)
            for s, n in zip(live, ntok):
                lens[s] += n
            forwards += 1
            assert torch.equal(mgr.k.cpu().float(), ref.k) and torch.equal(mgr.v.cpu().float(), ref.v)
        else:
            for s in live:
                mgr.release_sequence(s)
                ref.release_sequence(s)
            live, lens = [], {}
    assert forwards >= 20, forwards


@pytest.mark.parametrize("seed", [1, 2, 3, 4, 5])
def test_random_contiguous_traffic_matches_oracle(seed):
    run_contiguous_traffic(seed, CPU)
