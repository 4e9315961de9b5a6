"""The radix prefix tree and the page pool against operation sequences recorded from
the reference's own RadixTree and PagePool (nanoslg/kv_cache.py:380-531), in
tests/golden/radix_vectors.json (written by tests/golden/make_radix_vectors.py).

The oracle reproduces every recorded output: match results, pages freed by each
eviction, refcounts of the whole pool and the number of cached pages. The product
reproduces them too, except that its match returns pages only up to the first page
evicted from inside the path, where the reference returns the deeper pages as well
(a gap); every later operation still agrees, because the product walks and stamps
the path as the reference does. Allocation ids are replayed from the recording
(which free page an allocation returns is not part of the contract)."""
import json
import sys
from pathlib import Path

import pytest
import torch

from oracle import kv_oracle as O

sys.path.insert(0, str(Path(__file__).resolve().parent))
import fake_kernels as FK  # noqa: E402

VECTORS = json.loads((Path(__file__).resolve().parent / "golden" / "radix_vectors.json").read_text())
CASES = VECTORS["cases"]


def _oracle(case):
    pool = O.PagePoolRef(1, case["pages"], case["page_size"], 1, 2)
    return pool, O.RadixTreeRef(case["page_size"], pool)


def _product(case):
    from nanoslg_amd import kv_cache as KC
    cfg = KC.KVCacheConfig(num_layers=1, num_kv_heads=1, num_qo_heads=1, head_dim=2,
                           page_size=case["page_size"], max_pages=case["pages"], dtype=torch.float32,
                           device=torch.device("cpu"), backend="paged")
    pool = KC.PagePool(cfg, kernels=FK)
    return pool, KC.RadixTree(case["page_size"], pool)


def _take_oracle(pool, ids):
    for pid in ids:
        pool.free_set.remove(pid)
        pool.ref_count[pid] = 1
        pool.tokens_used[pid] = 0


def _take_product(pool, ids):
    for pid in ids:
        pool._free.remove(pid)
        pool._is_free[pid] = False
        pool.ref_count[pid] = 1
        pool.tokens_used[pid] = 0


def _contiguous_prefix(pages, depths, ps):
    """The pages of a reference match that lie at depths ps, 2ps, ... without a hole."""
    n = 0
    while n < len(depths) and depths[n] == ps * (n + 1):
        n += 1
    return pages[:n]


def _replay(case, pool, tree, take, gap_truncates):
    ps = case["page_size"]
    gaps = 0
    for i, op in enumerate(case["ops"]):
        kind = op["op"]
        where = f"seed {case['seed']} op {i} ({kind})"
        if kind == "match":
            plen, pages = tree.match(op["tokens"])
            exp_plen, exp_pages = op["out"]
            if gap_truncates:
                exp_pages = _contiguous_prefix(exp_pages, op["page_depths"], ps)
                exp_plen = ps * len(exp_pages)
            gaps += len(_contiguous_prefix(op["out"][1], op["page_depths"], ps)) != len(op["out"][1])
            assert (plen, list(pages)) == (exp_plen, exp_pages), where
        elif kind == "insert":
            tree.insert(op["tokens"], op["pages"])
        elif kind == "add_refs":
            tree.add_refs(op["tokens"], op["n"])
        elif kind == "dec_refs":
            tree.dec_refs(op["tokens"], op["n"])
        elif kind == "evict_lru":
            assert tree.evict_lru(op["need"]) == op["out"], where
        elif kind == "alloc":
            take(pool, op["out"])
        elif kind == "release":
            pool.release(op["pid"])
        elif kind == "add_ref":
            pool.add_ref(op["pid"])
        else:
            raise AssertionError(f"unknown op {kind}")
        if "ref_count" in op:
            assert [int(x) for x in pool.ref_count] == op["ref_count"], where
            assert tree.cached_pages == op["cached_pages"], where
    return gaps


def test_vectors_cover_the_quirks():
    gaps = sum(1 for c in CASES for o in c["ops"] if o["op"] == "match"
               and len(_contiguous_prefix(o["out"][1], o["page_depths"], c["page_size"])) != len(o["out"][1]))
    evictions = sum(1 for c in CASES for o in c["ops"] if o["op"] == "evict_lru" and o["out"] > 0)
    hits = sum(1 for c in CASES for o in c["ops"] if o["op"] == "match" and o["out"][0] > 0)
    assert gaps >= 3 and evictions >= 20 and hits >= 50


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c['seed']}-ps{c['page_size']}" for c in CASES])
def test_oracle_reproduces_reference_radix_tree(case):
    pool, tree = _oracle(case)
    _replay(case, pool, tree, _take_oracle, gap_truncates=False)


@pytest.mark.parametrize("case", CASES, ids=[f"seed{c['seed']}-ps{c['page_size']}" for c in CASES])
def test_product_radix_tree_matches_reference_up_to_gaps(case):
    pool, tree = _product(case)
    _replay(case, pool, tree, _take_product, gap_truncates=True)
