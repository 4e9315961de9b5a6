"""Writes radix_vectors.json: operation sequences on nanoslg's own RadixTree and
PagePool (nanoslg/kv_cache.py:380-531), run here on the CPU, with every
operation's inputs and outputs.

These vectors pin the two radix behaviours nothing else fixes: `match` walks on
past a page node whose page was evicted (kv_cache.py:467), and `evict_lru` orders
equal access times by DFS pre-order (the stable sort at :507). The JSON is data
(inputs and expected outputs); this script is the only thing that reads the
reference, and only when run by hand:

    python tests/golden/make_radix_vectors.py [path/to/nanoslg/kv_cache.py]

Timestamps: the reference stamps nodes with time.monotonic() once per call; here
the module's clock is replaced by a counter (one tick per call), which orders
calls the same way and makes ties reproducible.
"""
import importlib.util
import json
import sys
import types
from pathlib import Path

import numpy as np
import torch

REF = Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference/nanoslg/kv_cache.py")
OUT = Path(__file__).resolve().parent / "radix_vectors.json"


def load_reference():
    spec = importlib.util.spec_from_file_location("_nanoslg_kv_cache_reference", REF)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    tick = {"t": 0}

    def monotonic():
        tick["t"] += 1
        return float(tick["t"])

    mod.time = types.SimpleNamespace(monotonic=monotonic)
    return mod


def page_depths(tree, tokens):
    """Depths (multiples of ps) of the pages `match(tokens)` will return, read from
    the reference tree without touching it (the walk ends where match ends)."""
    node, out = tree.root, []
    for i, tok in enumerate(tokens):
        node = node.children.get(tok)
        if node is None:
            break
        if (i + 1) % tree.ps == 0 and node.page_id >= 0:
            if tree.pool.ref_count[node.page_id] <= 0:
                break
            out.append(i + 1)
    return out


def scenario(mod, seed, ps, pages, vocab, n_ops):
    """Manager-like traffic: admit a request (match, pin, allocate the rest), finish
    it (insert its full pages, unpin, release), or evict; tokens from a tiny
    vocabulary so prefixes collide."""
    rng = np.random.default_rng(seed)
    cfg = mod.KVCacheConfig(num_layers=1, num_kv_heads=1, num_qo_heads=1, head_dim=2, page_size=ps,
                            max_pages=pages, dtype=torch.float32, device=torch.device("cpu"),
                            backend="flashinfer")
    pool = mod.PagePool(cfg)
    tree = mod.RadixTree(ps, pool)
    live = {}
    past = []
    ops = []
    for _ in range(n_ops):
        r = rng.random()
        if (r < 0.45 and len(live) < 4) or not live:
            n = int(rng.integers(ps, 6 * ps + 1))
            pool_of = [st["tokens"] for st in live.values()] + past
            if pool_of and rng.random() < 0.7:  # share a prefix with a live or past request
                base = pool_of[int(rng.integers(len(pool_of)))]
                k = int(rng.integers(1, len(base) + 1))
                tokens = base[:k] + rng.integers(0, vocab, size=max(0, n - k)).tolist()
            else:
                tokens = rng.integers(0, vocab, size=n).tolist()
            depths = page_depths(tree, tokens)
            plen, mpages = tree.match(tokens)
            ops.append({"op": "match", "tokens": tokens, "out": [plen, mpages], "page_depths": depths})
            for p in mpages:
                pool.add_ref(p)
                ops.append({"op": "add_ref", "pid": p})
            tree.add_refs(tokens[:plen])
            ops.append({"op": "add_refs", "tokens": tokens[:plen], "n": 1})
            need = -(-(len(tokens) - plen) // ps)
            got = pool.alloc(need) if need else []
            if got is None:
                short = need - pool.num_free
                freed = tree.evict_lru(short)
                ops.append({"op": "evict_lru", "need": short, "out": freed})
                got = pool.alloc(need)
            if got is None:  # still out of pages: drop the request
                tree.dec_refs(tokens[:plen])
                ops.append({"op": "dec_refs", "tokens": tokens[:plen], "n": 1})
                for p in mpages:
                    pool.release(p)
                    ops.append({"op": "release", "pid": p})
                continue
            ops.append({"op": "alloc", "n": need, "out": got})
            rid = f"r{len(ops)}"
            live[rid] = {"tokens": tokens, "plen": plen, "pages": mpages + got}
        elif r < 0.85:
            rid = list(live)[int(rng.integers(len(live)))]
            st = live.pop(rid)
            past.append(st["tokens"])
            full = len(st["tokens"]) // ps
            tree.insert(st["tokens"][:full * ps], st["pages"][:full])
            ops.append({"op": "insert", "tokens": st["tokens"][:full * ps], "pages": st["pages"][:full]})
            tree.dec_refs(st["tokens"][:st["plen"]])
            ops.append({"op": "dec_refs", "tokens": st["tokens"][:st["plen"]], "n": 1})
            for p in st["pages"]:
                pool.release(p)
                ops.append({"op": "release", "pid": p})
        else:
            need = int(rng.integers(1, 4))
            freed = tree.evict_lru(need)
            ops.append({"op": "evict_lru", "need": need, "out": freed})
        if ops[-1]["op"] in ("match", "evict_lru"):
            ops[-1]["ref_count"] = list(pool.ref_count)
            ops[-1]["cached_pages"] = tree.cached_pages
    ops[-1]["ref_count"] = list(pool.ref_count)
    ops[-1]["cached_pages"] = tree.cached_pages
    return {"seed": seed, "page_size": ps, "pages": pages, "vocab": vocab, "ops": ops}


def main():
    mod = load_reference()
    cases = [scenario(mod, seed, ps, pages, vocab, n_ops)
             for seed, ps, pages, vocab, n_ops in [(1, 2, 24, 2, 120), (2, 2, 16, 3, 120), (3, 4, 20, 2, 120),
                                                   (4, 1, 12, 3, 100), (5, 3, 40, 2, 150), (6, 2, 12, 2, 150)]]
    gaps = sum(1 for c in cases for o in c["ops"]
               if o["op"] == "match" and o["page_depths"] != [c["page_size"] * (i + 1)
                                                              for i in range(len(o["page_depths"]))])
    OUT.write_text(json.dumps({"source": "nanoslg/kv_cache.py:380-531", "cases": cases}, separators=(",", ":")))
    print(f"wrote {OUT} ({OUT.stat().st_size} bytes): {sum(len(c['ops']) for c in cases)} ops, "
          f"{gaps} matches with a page gap")


if __name__ == "__main__":
    main()
