"""Decode steps replayed from captured HIP graphs (DecodeGraph) on the GPU: against
the same steps run eagerly on a second cache, and against the oracle through the
fused-RoPE attention forward with grouped decode inside the graph. Kept apart from
the eager parity tests and collected after them: graph capture is an optional path.
Page contents are compared bit-exactly; attention outputs within 2e-3 abs + 1e-2 rel
of fp32 SDPA."""
import contextlib
import gc
import weakref

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O
from test_gpu_cache import ATOL, D, DEV, HKV, HQ, L, RTOL, _log, check_state, make

pytestmark = pytest.mark.gpu


@contextlib.contextmanager
def _no_collector():
    """The cyclic collector off: what is freed inside is freed by reference counting."""
    was = gc.isenabled()
    gc.disable()
    try:
        yield
    finally:
        if was:
            gc.enable()


def test_decode_graph_replays_match_eager_steps():
    """Decode steps replayed from the captured graphs (planner + per-layer append and
    decode) against the same steps run eagerly on a second cache with the same
    history: every replay's outputs, the pool bytes, tokens_used and block tables
    are identical, over steps that open pages (in-graph zeroing)."""
    _log("decode graph vs eager")
    from nanoslg_amd import kv_cache as KC
    g = torch.Generator().manual_seed(23)
    lens = [15, 16, 100, 257]
    ids = ["a", "b", "c", "d"]
    caches = [make(ps=16, pages=400, prefix=False)[0] for _ in range(2)]
    S = max(lens)
    q0 = torch.randn(4, S, HQ, D, generator=g).half().to(DEV)
    k0 = torch.randn(4, S, HKV, D, generator=g).half().to(DEV)
    for m in caches:
        for s, n in zip(ids, lens):
            m.allocate_sequence(s, num_tokens=n)
        c = m.begin_forward(ids, lens)
        for layer in range(L):
            c.attend(layer, q0, k0, k0, HQ, HKV)
        m.end_forward(c)
    gm, em = caches
    qs = torch.zeros(4, 1, HQ, D, dtype=torch.float16, device=DEV)
    ks = torch.zeros(4, 1, HKV, D, dtype=torch.float16, device=DEV)
    vs = torch.zeros(4, 1, HKV, D, dtype=torch.float16, device=DEV)
    graph = KC.DecodeGraph(gm, ids, lambda ctx: [ctx.attend(layer, qs, ks, vs, HQ, HKV) for layer in range(L)])
    for step in range(40):
        q = torch.randn(4, 1, HQ, D, generator=g).half().to(DEV)
        k = torch.randn(4, 1, HKV, D, generator=g).half().to(DEV)
        v = torch.randn(4, 1, HKV, D, generator=g).half().to(DEV)
        qs.copy_(q)
        ks.copy_(k)
        vs.copy_(v)
        outs = graph.step()
        c = em.begin_forward(ids, [1] * 4)
        ref = [c.attend(layer, q, k, v, HQ, HKV) for layer in range(L)]
        em.end_forward(c)
        torch.cuda.synchronize()
        for a, b in zip(outs, ref):
            assert torch.equal(a, b), step
    assert torch.equal(gm.pool.k, em.pool.k) and torch.equal(gm.pool.v, em.pool.v)
    assert np.array_equal(gm.pool.tokens_used, em.pool.tokens_used)
    for s in ids:
        assert gm.seqs[s].num_tokens == em.seqs[s].num_tokens
        assert gm.seqs[s].block_table == em.seqs[s].block_table
    wr = weakref.ref(graph)
    with _no_collector():  # no reference cycle: the graph goes with its last reference
        del graph
        assert wr() is None


def test_decode_graph_steps_match_the_oracle():
    """Steady decode steps replayed from HIP graphs against the oracle. The steps go
    through attention_forward, so the rotary embedding is fused into the append
    (models.py:86-105). Five requests share a radix prefix, so grouped decode runs
    inside the graph. One request has pages taken ahead by extend_sequence, whose
    zeroing the cache defers. Every replayed step is checked: the plan it ran on
    equals the oracle's CSR of the cache's own block tables (kv_cache.py:598-615),
    with the new tokens' slots and positions, and its outputs equal the oracle's
    (eager rotation, then fp32 SDPA). Eager steps then continue on the same cache,
    and at the end every page's contents are bit-exact with the oracle's."""
    _log("decode graph (rope, grouped prefix, deferred zeroing) vs oracle")
    from nanoslg_amd import kv_cache as KC
    g = torch.Generator().manual_seed(31)
    ps = 16
    mgr, ref = make(ps=ps, pages=400, prefix=True)
    cos, sin = O.rope_tables(D, 1024, 500000.0)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)

    def draw(B, S):
        return (torch.randn(B, S, HQ, D, generator=g).half(), torch.randn(B, S, HKV, D, generator=g).half(),
                torch.randn(B, S, HKV, D, generator=g).half())

    def oracle_attend(c2, q, k, v, S):
        qr, kr = O.rope_forward_ref(q, k, cos, sin, c2.get_position_ids(S))
        return [c2.attend(layer, qr.float(), kr.float(), v.float(), HQ, HKV) for layer in range(L)]

    def eager_both(ids, ntok, offs):
        S = max(o + n for o, n in zip(offs, ntok))
        q, k, v = draw(len(ids), S)
        c1, c2 = mgr.begin_forward(ids, ntok, offs), ref.begin_forward(ids, ntok, offs)
        want = oracle_attend(c2, q, k, v, S)
        for layer in range(L):
            o1 = KC.attention_forward(q.to(DEV), k.to(DEV), v.to(DEV), layer, HQ, HKV, cos_d, sin_d, c1)
            o1 = o1.float().cpu()
            for b in range(len(ids)):
                rows = slice(offs[b], offs[b] + ntok[b])
                torch.testing.assert_close(o1[b, rows], want[layer][b, rows], atol=ATOL, rtol=RTOL)
        mgr.end_forward(c1)
        ref.end_forward(c2)

    prompt = list(range(1, 16 * 6 + 6))  # 6 full pages and 5 tokens
    for impl in (mgr, ref):
        impl.allocate_sequence("p", token_ids=prompt)
    eager_both(["p"], [len(prompt)], [0])
    for impl in (mgr, ref):
        impl.release_sequence("p")  # its 6 full pages stay cached in the radix tree
    ids = [f"r{i}" for i in range(5)]
    for i, sid in enumerate(ids):
        toks = prompt[:96] + [500 + i] * (3 + 2 * i)
        for impl in (mgr, ref):
            assert impl.allocate_sequence(sid, token_ids=toks) == 96
    B = len(ids)
    eager_both(ids, [3 + 2 * i for i in range(B)], [0] * B)
    eager_both(ids, [1] * B, [0] * B)
    for impl in (mgr, ref):
        impl.extend_sequence(ids[0], 20)  # pages taken ahead of the tokens
    qs = torch.zeros(B, 1, HQ, D, dtype=torch.float16, device=DEV)
    ks = torch.zeros(B, 1, HKV, D, dtype=torch.float16, device=DEV)
    vs = torch.zeros(B, 1, HKV, D, dtype=torch.float16, device=DEV)
    graph = KC.DecodeGraph(mgr, ids, lambda ctx: [KC.attention_forward(qs, ks, vs, layer, HQ, HKV, cos_d, sin_d,
                                                                       ctx) for layer in range(L)])
    grp = graph.plans[0].groups
    assert grp is not None and grp.num_groups == 1 and len(grp.members[0]) == 4  # 16 / G = 4 members
    for step in range(24):
        q, k, v = draw(B, 1)
        qs.copy_(q.to(DEV))
        ks.copy_(k.to(DEV))
        vs.copy_(v.to(DEV))
        starts = [mgr.seqs[s].num_tokens for s in ids]
        outs = graph.step()
        c2 = ref.begin_forward(ids, [1] * B)
        want = oracle_attend(c2, q, k, v, 1)
        ref.end_forward(c2)
        torch.cuda.synchronize()
        for layer in range(L):
            torch.testing.assert_close(outs[layer].float().cpu(), want[layer], atol=ATOL, rtol=RTOL,
                                       msg=lambda m, step=step: f"step {step}: {m}")
        # the plan this replay ran on
        p = graph.plans[graph.parity]
        tables = [mgr.seqs[s].block_table for s in ids]
        lens = [mgr.seqs[s].num_tokens for s in ids]
        assert lens == [x + 1 for x in starts]
        e_ip, e_ix, e_lpl = O.plan_csr(tables, lens, ps)
        n = int(e_ip[-1])
        assert p.indptr.cpu().tolist() == e_ip.tolist(), step
        assert p.indices.cpu()[:n].tolist() == e_ix[:n].tolist(), step
        assert p.lpl.cpu().tolist() == e_lpl.tolist(), step
        assert p.slot.cpu().tolist() == [tables[b][x // ps] * ps + x % ps for b, x in enumerate(starts)], step
        assert p.pos.cpu().tolist() == starts, step
    for _ in range(4):  # back to eager steps on the same cache
        eager_both(ids, [1] * B, [0] * B)
    check_state(mgr, ref, ids)
    wr = weakref.ref(graph)
    with _no_collector():  # no reference cycle: the graph goes with its last reference
        del graph
        assert wr() is None
