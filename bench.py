#!/usr/bin/env python3
"""Benchmark of the paged decode attention + append hot path on one MI355X.

Default workload (kv_pressure): one Llama-3.1-8B attention layer (32 query / 8 KV
heads, head_dim 128, fp16, page size 16), batch 64, context lengths log-uniform
in [2048, 32768], pool sized to 90 % occupancy with pages shuffled across
sequences, 10 % of pages released and re-allocated mid-run. One step = one decode
step of that layer through the drop-in API (begin_forward -> attend -> end_forward):
planning, the split-K decode kernel (which writes the step's new K/V rows) and
the merge.

Prints ONE JSON line. `value` = algorithmic HBM bytes per step / wall time per
step (GB/s). `roofline` = the nslg_paged_decode_append call (split-K decode kernel
+ merge kernel), timed with HIP events on its stream around every call of a second pass of
`--steps` steps of the same workload (timing events slow the queue by ~10 us per
step, so the pass that gives `value` runs without them).
`cpu_baseline` = the CPU restatement of the reference's contiguous SDPA path on a
bounded sample of the same workload, on this host's cores.

  python bench.py [--steps 256] [--warmup 16] [--workload kv_pressure|small_batch|radix|prefill|rope]
  python bench.py --workload copy_calibration   (a plain 1 GiB copy, for counter scaling)
"""
from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

HQ, HKV, D, PS = 32, 8, 128, 16
HBM_PEAK_GBS = 8000.0

# HBM bytes an nslg_paged_decode call (split-K kernel + merge) moves per algorithmic
# byte: the FETCH_SIZE and WRITE_SIZE counters of the roofline pass of
# `bench.py --steps 20 --warmup 5`, each scaled by what the counter reads for a plain
# copy of known size, over that pass's algorithmic bytes
# (profiles/paged_decode_hbm_traffic_kv_pressure_b64.md). `traffic` in the JSON line is
# this ratio times the algorithmic bytes of the run being reported.
TRAFFIC_PER_ALGORITHMIC_BYTE = {"kv_pressure": 1.0056}
# The same for the chunked-prefill launch over the 8 chunks of a batch (q, out, the
# K/V of every visible key once, the chunk's K/V rows written once and the page
# ids): FETCH_SIZE and WRITE_SIZE of `bench.py --workload prefill --steps 4
# --warmup 8`, scaled as above (profiles/paged_prefill_chunked_b8x4096.md). Above 1
# because the row tiles of one KV head re-fetch its K/V once it leaves the XCD's L2.
PREFILL_TRAFFIC_PER_ALGORITHMIC_BYTE = 1.424
MFMA_F16_PEAK_TFLOPS = 2500.0


def _parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=256)
    ap.add_argument("--warmup", type=int, default=16)
    ap.add_argument("--workload", default="kv_pressure",
                    choices=["kv_pressure", "small_batch", "radix", "prefill", "rope", "copy_calibration"])
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="decode workloads: replay each step from captured HIP graphs (DecodeGraph)")
    ap.add_argument("--layers", type=int, default=1,
                    help="small_batch workload: layers per decode step (each with its own pool layer; "
                         "one forward attends every layer, as a model's decode step does)")
    ap.add_argument("--head-dim", type=int, default=128, choices=[64, 128, 256],
                    help="prefill workload: head dim (heads scaled to keep Hq*D = 4096, Hkv*D = 1024)")
    ap.add_argument("--dtype", default="fp16", choices=["fp16", "bf16"],
                    help="prefill workload: the pool's and Q/K/V's dtype")
    return ap.parse_args()


def _settle_gc():
    """Before the warmup steps: one collection, then every object alive so far moved
    out of the collector's generations (gc.freeze, as serving processes do after
    start-up), so later collections only walk the few objects the steps create."""
    import gc
    gc.collect()
    gc.freeze()


class _GcPaused:
    """A timed region with Python's cyclic garbage collector paused, as timeit runs
    its loops: a collection walks every object of the process (tens of milliseconds
    with torch loaded) and would land in whichever step happened to trigger it.
    Reference counting frees the steps' objects as usual inside it."""

    def __enter__(self):
        import gc
        self.was_enabled = gc.isenabled()
        gc.disable()
        return self

    def __exit__(self, *exc):
        import gc
        if self.was_enabled:
            gc.enable()
        return False


def _log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


# --------------------------------------------------------------------------- workloads


class DecodeWorkload:
    """A batch of sequences with random K/V already resident in a paged pool."""

    def __init__(self, name, lens, pool_pages, seed, churn_frac=0.0, shuffle=True, layers=1):
        import torch
        from nanoslg_amd.kv_cache import KVCacheConfig, PagedKVCache
        self.torch = torch
        self.name = name
        self.layers = layers
        self.lens0 = list(lens)
        self.B = len(lens)
        self.seed = seed
        self.churn_frac = churn_frac
        self.rng = np.random.default_rng(seed)
        cfg = KVCacheConfig(num_layers=layers, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=PS,
                            max_pages=pool_pages, dtype=torch.float16, device=torch.device("cuda:0"),
                            enable_prefix_caching=False, backend="paged")
        self.mgr = PagedKVCache(cfg)
        pool = self.mgr.pool
        if shuffle:
            free = np.array(pool._free, np.int64)
            self.rng.shuffle(free)
            pool._free = free.tolist()
        self.ids = [f"s{b}" for b in range(self.B)]
        for sid, L in zip(self.ids, lens):
            self._admit(sid, L)
        g = torch.Generator(device="cuda:0").manual_seed(seed)
        # the K/V of the sequences re-admitted at the churn: N(0,1) rows drawn here, at
        # set-up, and written into their new pages by the cache's append kernel at the
        # churn, as the prefill of those sequences would write them (drawing them at
        # the churn would leave ~300 MB of freshly written temporaries in the caches,
        # which the next decode then writes back: a harness cost, not the cache's)
        self.fresh = None
        if churn_frac > 0:
            rows = int(churn_frac * sum(math.ceil(L / PS) for L in lens) * PS * 1.5) + 2048 * PS
            self.fresh = (torch.randn(rows, HKV, D, generator=g, device="cuda:0", dtype=torch.float16),
                          torch.randn(rows, HKV, D, generator=g, device="cuda:0", dtype=torch.float16))
        # prefill content: every page (allocated ones were zeroed on allocation) ~ N(0,1)
        pool.k.normal_(generator=g)
        pool.v.normal_(generator=g)
        # per-step inputs: a ring of seeded N(0,1) q/k/v, [B, 1, H, D]
        ring = 8
        self.q = torch.randn(ring, self.B, 1, HQ, D, generator=g, device="cuda:0", dtype=torch.float16)
        self.kn = torch.randn(ring, self.B, 1, HKV, D, generator=g, device="cuda:0", dtype=torch.float16)
        self.vn = torch.randn(ring, self.B, 1, HKV, D, generator=g, device="cuda:0", dtype=torch.float16)
        # the ring's per-step tensors, sliced once (a model hands its q/k/v to attend
        # without this harness's indexing in between)
        self.inputs = [(self.q[i], self.kn[i], self.vn[i]) for i in range(ring)]
        self.step_idx = 0
        self.last_ctx = None

    def _admit(self, sid, L):
        """Allocate a sequence of L tokens whose pages already hold N(0,1) K/V."""
        mgr = self.mgr
        mgr.allocate_sequence(sid, num_tokens=L)
        st = mgr.seqs[sid]
        st.num_tokens = L
        pages = st.bt[:st.n_pages]
        for i, p in enumerate(pages.tolist()):
            mgr.pool.tokens_used[p] = PS if i < len(pages) - 1 else L - PS * (len(pages) - 1)

    def churn(self):
        """Release whole sequences until >= churn_frac of the used pages are free, then
        re-admit them at the same lengths on freshly shuffled pages with fresh K/V
        (every slot of their pages, written with the append kernel from the rows drawn
        at set-up)."""
        torch = self.torch
        from nanoslg_amd import kernels
        mgr = self.mgr
        used = sum(mgr.seqs[s].n_pages for s in self.ids)
        order = self.rng.permutation(self.B)
        freed, victims = 0, []
        for b in order:
            if freed >= self.churn_frac * used:
                break
            sid = self.ids[b]
            victims.append((sid, mgr.seqs[sid].num_tokens))
            freed += mgr.seqs[sid].n_pages
            mgr.release_sequence(sid)
        free = np.array(mgr.pool._free, np.int64)
        self.rng.shuffle(free)
        mgr.pool._free = free.tolist()
        fk, fv = self.fresh
        o = 0
        for sid, L in victims:
            self._admit(sid, L)
            st = mgr.seqs[sid]
            pages = st.bt[:st.n_pages].astype(np.int64)
            slots = (pages[:, None] * PS + np.arange(PS)).reshape(-1).astype(np.int32)
            n = slots.size
            if o + n > fk.shape[0]:
                o = 0
            kernels.append_kv(fk[o:o + n], fv[o:o + n], torch.from_numpy(slots).to(fk.device),
                              mgr.pool.k[0], mgr.pool.v[0])
            o += n
        return freed

    def seq_lens(self):
        return [self.mgr.seqs[s].num_tokens for s in self.ids]

    def step(self):
        q, kn, vn = self.inputs[self.step_idx % len(self.inputs)]
        self.step_idx += 1
        ctx = self.mgr.begin_forward(self.ids, [1] * self.B)
        for layer in range(self.layers):
            out = ctx.attend(layer, q, kn, vn, HQ, HKV)
        self.mgr.end_forward(ctx)
        self.last_ctx = ctx
        return out

    def forward(self, ctx):
        """The attend calls of one decode forward on the ring's first inputs (what a
        captured step replays)."""
        return [ctx.attend(layer, self.q[0], self.kn[0], self.vn[0], HQ, HKV) for layer in range(self.layers)]


def step_bytes(lens_after, B, total_pages):
    """Algorithmic HBM bytes of one decode+append step (fp16, one layer)."""
    kv = sum(lens_after) * HKV * D * 2 * 2
    append = B * HKV * D * 2 * 2 * 2
    qo = B * HQ * D * 2 * 2
    csr = 4 * (total_pages + 2 * B + 1)
    return kv, append, qo, csr


def decode_call_bytes(lens_after, B, total_pages):
    """Algorithmic HBM bytes of one nslg_paged_decode_append call: K and V of every
    cached token once, the step's new K/V rows read and written once, q read and out
    written once, the CSR block table once."""
    kv = sum(lens_after) * HKV * D * 2 * 2
    append = B * HKV * D * 2 * 2 * 2
    qo = B * HQ * D * 2 * 2
    csr = 4 * (total_pages + 2 * B + 1)
    return kv + append + qo + csr


def kv_pressure_lens(seed, B=64):
    rng = np.random.default_rng(seed)
    return [int(round(math.exp(x))) for x in rng.uniform(math.log(2048), math.log(32768), size=B)]


# --------------------------------------------------------------------------- measurement


class EventTimedKernels:
    """The kernel module with nslg_paged_decode bracketed by HIP events on the stream it
    is launched on, so the decode call is timed live inside the timed steps."""

    def __init__(self, kernels):
        import torch
        self._k = kernels
        self._torch = torch
        self.events = []
        self.recording = False

    def __getattr__(self, name):
        return getattr(self._k, name)

    def DecodeLaunch(self, k_pool, v_pool, slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                     num_qo_heads, workspace=None, sm_scale=None, groups=None):
        """The per-forward launcher (re-bound from forward to forward as the product's
        is); while recording, each layer's call (nslg_paged_decode_append: the decode
        with the step's new rows written inside it) is bracketed by events."""
        real = self._k.DecodeLaunch(k_pool, v_pool, slot_mapping, kv_indptr, kv_indices, kv_last_page_len,
                                    total_pages, num_qo_heads, workspace=workspace, sm_scale=sm_scale,
                                    groups=groups)
        return _TimedLaunch(self, real)

    def paged_decode(self, *args, **kw):
        return self._timed(self._k.paged_decode, *args, **kw)

    def _timed(self, fn, *args, **kw):
        if not self.recording:
            return fn(*args, **kw)
        torch = self._torch
        stream = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        out = fn(*args, **kw)
        b.record(stream)
        self.events.append((a, b))
        return out

    def paged_prefill(self, *args, **kw):
        return self._timed(self._k.paged_prefill, *args, **kw)

    def _paged_prefill_layer(self, *args, **kw):  # the cache manager's prefill launch
        return self._timed(self._k._paged_prefill_layer, *args, **kw)

    def _paged_prefill_append_layer(self, *args, **kw):  # the same with the chunk's K/V write inside
        return self._timed(self._k._paged_prefill_append_layer, *args, **kw)

    def mean_ms(self):
        return float(np.mean([a.elapsed_time(b) for a, b in self.events]))

    def total_ms(self):
        return float(np.sum([a.elapsed_time(b) for a, b in self.events]))


class _TimedLaunch:
    """A kernels.DecodeLaunch whose calls are event-timed while recording."""

    def __init__(self, timed, real):
        self.timed, self.real = timed, real
        self.B, self.Hq, self.workspace = real.B, real.Hq, real.workspace

    def rebind(self, slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages, groups=None, check=True):
        self.real.rebind(slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages, groups, check=check)
        return self

    def __call__(self, layer, q, k_new, v_new, rope=None):
        timed = self.timed
        if not timed.recording or rope is not None:
            return self.real(layer, q, k_new, v_new, rope=rope)
        torch = timed._torch
        stream = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record(stream)
        out = self.real(layer, q, k_new, v_new)
        b.record(stream)
        timed.events.append((a, b))
        return out


def copy_calibration():
    """A plain 1 GiB device-to-device copy (torch's copy kernel), for scaling the
    FETCH_SIZE / WRITE_SIZE counters to bytes."""
    import torch
    n = 1 << 30
    x = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    y = torch.empty_like(x)
    for _ in range(4):
        y.copy_(x)
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(8):
        y.copy_(x)
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / 8
    return {"workload": "copy_calibration", "bytes_read": n, "bytes_written": n,
            "ms_per_copy": round(ms, 4), "GB_s": round(2 * n / (ms * 1e-3) / 1e9, 1)}


def cpu_baseline_sample(lens, seed, budget_s=12.0, max_steps=32):
    """The reference's contiguous SDPA decode path restated on the CPU (fp32): a bounded
    sample of the workload — its first 4 sequences, stepped until `budget_s` seconds."""
    import torch
    from oracle import kv_oracle as O
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    torch.set_num_threads(threads)
    sample = list(lens[:4])
    B = len(sample)
    g = torch.Generator().manual_seed(seed)
    Smax = max(sample) + max_steps + 4
    cache = O.ContiguousRef(1, B, Smax, HKV, D, torch.float32)
    ids = [f"c{b}" for b in range(B)]
    for b, (sid, L) in enumerate(zip(ids, sample)):
        cache.allocate_sequence(sid)
        cache.k[0, b, :L] = torch.randn(L, HKV, D, generator=g)
        cache.v[0, b, :L] = torch.randn(L, HKV, D, generator=g)
        cache.states[sid]["num_tokens"] = L
    q = torch.randn(B, 1, HQ, D, generator=g) / math.sqrt(D)
    kn = torch.randn(B, 1, HKV, D, generator=g)
    vn = torch.randn(B, 1, HKV, D, generator=g)
    # warm up once
    ctx = cache.begin_forward(ids, [1] * B)
    ctx.attend(0, q, kn, vn, HQ, HKV)
    cache.end_forward(ctx)
    steps, nbytes = 0, 0
    t0 = time.perf_counter()
    while steps < max_steps and time.perf_counter() - t0 < budget_s:
        ctx = cache.begin_forward(ids, [1] * B)
        ctx.attend(0, q, kn, vn, HQ, HKV)
        cache.end_forward(ctx)
        lens_after = ctx.seq_lens
        nbytes += sum(lens_after) * HKV * D * 4 * 2 + B * HKV * D * 4 * 4 + B * HQ * D * 4 * 2
        steps += 1
    dt = time.perf_counter() - t0
    try:
        model = open("/proc/cpuinfo").read().split("model name")[1].split(":")[1].split("\n")[0].strip()
    except Exception:
        model = "unknown"
    # the reference's own CPU case: B=1, 512-token context, 64 decode steps, fp32
    # (median of 5 repeats after 8 warmup steps)
    sec, _ = O.timed_contiguous_decode(num_steps=64, prefill=512, Hq=HQ, Hkv=HKV, D=D, seed=seed, warmup=8,
                                       repeats=5, threads=threads)
    lens1 = [512 + i + 1 for i in range(64)]
    b1 = np.mean([2 * HKV * D * 4 * L + 2 * HKV * D * 4 * 2 + 2 * HQ * D * 4 for L in lens1])
    contiguous_b1 = {"ms_per_step": round(sec * 1e3, 4), "tok_s_layer": round(1.0 / sec, 1),
                     "GB_s": round(float(b1) / sec / 1e9, 3),
                     "context": "513..576 tokens (8 warmup steps on a separate cache)", "repeats": 5}
    return {
        "value": round(nbytes / dt / 1e9, 3),
        "unit": "GB/s",
        "contiguous_b1_ctx512": contiguous_b1,
        "tok_s_layer": round(B * steps / dt, 2),
        "ms_per_step": round(dt / steps * 1e3, 3),
        "cores": threads,
        "kind": "port",
        "cpu": model,
        "sample": (f"contiguous SDPA path (write, slice read, transpose copy, masked SDPA) in fp32, "
                   f"sequences 0-3 of the workload (lengths {sample}), {steps} decode steps"),
    }


# --------------------------------------------------------------------------- main


def run_decode(args):
    import torch
    if args.workload == "kv_pressure":
        lens = kv_pressure_lens(args.seed)
        total_steps = args.warmup + 3 * args.steps  # timed pass + roofline pass + step-timing pass
        npages = sum(math.ceil(L / PS) for L in lens)
        pool_pages = int(math.ceil(npages / 0.9)) + 1
        # room for the steps' growth inside the 10 % headroom
        grow = len(lens) * (math.ceil(total_steps / PS) + 1)
        assert pool_pages - 1 - npages >= grow, "pool headroom too small for the run"
        w = DecodeWorkload("kv_pressure", lens, pool_pages, args.seed, churn_frac=0.10)
        cfg = {"workload": "kv_pressure_decode_append", "batch": 64, "ctx": "log-uniform[2048,32768]",
               "pool_occupancy": 0.9, "page_size": PS, "heads": f"{HQ}q/{HKV}kv", "head_dim": D,
               "layers": 1, "churn": "10% of pages at mid-run", "seed": args.seed}
    else:  # small_batch
        rng = np.random.default_rng(args.seed)
        lens = [int(x) for x in rng.integers(1024, 4097, size=4)]
        w = DecodeWorkload("small_batch", lens, 65536, args.seed, layers=args.layers)
        cfg = {"workload": "small_batch_decode_append", "batch": 4, "ctx": "uniform[1024,4096]",
               "pool_pages": 65536, "page_size": PS, "heads": f"{HQ}q/{HKV}kv", "head_dim": D,
               "layers": args.layers, "seed": args.seed}
    cfg["step"] = "graph replay (DecodeGraph)" if args.graph else "eager (begin_forward / attend / end_forward)"
    _log(f"workload {w.name}: B={w.B} pages={w.mgr.cfg.max_pages} sum(L)={sum(lens)}")
    from nanoslg_amd import kernels
    timed = EventTimedKernels(kernels)
    w.mgr.kernels = timed
    _settle_gc()
    for _ in range(args.warmup):
        w.step()
    torch.cuda.synchronize()
    step = w.step
    if args.graph:
        from nanoslg_amd.kv_cache import DecodeGraph

        def make_graph(warm):
            g = DecodeGraph(w.mgr, w.ids, w.forward)
            for _ in range(warm):
                g.step()
            torch.cuda.synchronize()
            return g
        graph = make_graph(4)
        step = graph.step
    lens_before = w.seq_lens()
    churn_at = args.steps // 2 if w.churn_frac > 0 else -1
    # Every sequence gains one token per step and the churn re-admits sequences at
    # their lengths, so the bytes of step i follow from the lengths before the loop;
    # they are summed here, outside the timed region.
    nbytes = [0, 0, 0, 0]
    for i in range(args.steps):
        lens_i = [L + 1 + i for L in lens_before]
        tp = sum(math.ceil(L / PS) for L in lens_i)
        for j, x in enumerate(step_bytes(lens_i, w.B, tp)):
            nbytes[j] += x * w.layers
    kbytes = 0
    churn_s = 0.0
    with _GcPaused():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(args.steps):
            if i == churn_at:
                # re-admission of released sequences is not a decode step: timed apart
                torch.cuda.synchronize()
                c0 = time.perf_counter()
                w.churn()
                if args.graph:  # the batch changed: capture the step again
                    graph = make_graph(0)
                    step = graph.step
                torch.cuda.synchronize()
                churn_s = time.perf_counter() - c0
            step()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0 - churn_s
    assert w.seq_lens() == [L + args.steps for L in lens_before]
    ms_step = wall / args.steps * 1e3
    total_bytes = sum(nbytes)
    value = total_bytes / wall / 1e9
    _log(f"{args.steps} steps in {wall*1e3:.1f} ms -> {ms_step:.3f} ms/step, {value:.1f} GB/s")

    # Roofline pass: the same workload continues for another `steps` steps with HIP
    # events around every decode call on its stream. Timing events add about 10 us
    # of queue overhead per step, so the pass that gives `value` runs without them.
    timed.recording = True
    with _GcPaused():
        for _ in range(args.steps):
            lens_i = [L + 1 for L in w.seq_lens()]
            kbytes += w.layers * decode_call_bytes(lens_i, w.B, sum(math.ceil(L / PS) for L in lens_i))
            w.step()
        torch.cuda.synchronize()
    timed.recording = False
    mean_ms = timed.mean_ms()
    kbytes /= args.steps * w.layers
    achieved = kbytes / (mean_ms * 1e-3) / 1e9
    _log(f"decode call: mean {mean_ms*1e3:.1f} us over {len(timed.events)} launches, {achieved:.1f} GB/s")
    ratio = TRAFFIC_PER_ALGORITHMIC_BYTE.get(w.name)
    traffic = int(round(ratio * kbytes)) if ratio else None
    if traffic:
        _log(f"decode call: {int(kbytes)} algorithmic bytes per launch, traffic {traffic} bytes "
             f"(x{ratio} from the HBM counters)")

    # Step-timing pass: the timed pass's structure again (the same step count, the
    # churn at mid-run) with one event per step boundary on the compute stream. An
    # interval is a step's time on the GPU's clock; after the churn's synchronisation
    # the next interval starts from a fresh event, so it also holds that step's host
    # planning, which the idle GPU waits for (as step 0's does).
    stream = torch.cuda.current_stream()
    mark = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    spans = []
    post_churn = -1
    with _GcPaused():
        torch.cuda.synchronize()
        prev = mark()
        prev.record(stream)
        for i in range(args.steps):
            if i == churn_at:
                torch.cuda.synchronize()
                w.churn()
                if args.graph:
                    graph = make_graph(0)
                    step = graph.step
                torch.cuda.synchronize()
                prev = mark()
                prev.record(stream)
                post_churn = i
            step()
            e = mark()
            e.record(stream)
            spans.append((prev, e))
            prev = e
        torch.cuda.synchronize()
    step_ms = [a.elapsed_time(b) for a, b in spans]
    med = float(np.median(step_ms))
    worst = int(np.argmax(step_ms))
    _log("step wall ms (step-timing pass): " + ", ".join(f"{x:.3f}" for x in step_ms))
    _log(f"step wall: median {med:.3f} ms, max {step_ms[worst]:.3f} ms (step {worst}), "
         f"max/median {step_ms[worst] / med:.2f}"
         + (f", step after the churn {step_ms[post_churn]:.3f} ms" if post_churn >= 0 else ""))
    # Small batches: kernel time of the last step's decode call alone (its events
    # above also hold launch gaps): the call captured 10 times in a HIP graph, replayed
    # with events around the replays. It writes the same new rows again, so the pool
    # does not change.
    call_us = None
    ctx = w.last_ctx
    launch = getattr(ctx, "_decode_launch", None) if ctx is not None else None
    if launch is not None and not args.graph and w.B <= 16:
        q, kn, vn = w.inputs[(w.step_idx - 1) % len(w.inputs)]
        call_us = _graph_time_us(torch, torch.device("cuda:0"), lambda: launch(0, q, kn, vn))
        _log(f"decode call, kernel time (graph-timed): {call_us} us")
    res = {
        "metric": "paged decode attn+append: achieved HBM GB/s (% of peak) and decode tok/s/layer",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic: K/V/Q ~ N(0,1), seeded",
        "config": cfg,
        "pct_of_hbm_peak": round(100.0 * value / HBM_PEAK_GBS, 2),
        "decode_tok_s_layer": round(w.B * args.steps * w.layers / wall, 1),
        "bytes_per_step": {k: int(v / args.steps) for k, v in zip(["kv_read", "append", "q_out", "csr"], nbytes)},
        "roofline": {
            "bound": "hbm",
            "kernel": "nslg_paged_decode_append (split-K decode kernel, which also writes the step's new K/V rows, + LSE merge kernel)",
            "timing": (f"HIP events on the launch stream around each of {args.steps} decode calls, "
                       "in a second pass of the same workload after the timed steps"),
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "traffic_note": (f"{ratio} x the algorithmic bytes per launch (FETCH_SIZE/WRITE_SIZE of the decode "
                             "call, calibrated on a plain copy, over its algorithmic bytes)") if ratio else None,
            "avg_launch_us": round(mean_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": int(kbytes),
        },
        "decode_call_kernel_us": call_us,
        "churn_ms": round(churn_s * 1e3, 2),
        "step_wall_ms": {"median": round(med, 4), "max": round(step_ms[worst], 4), "max_step": worst,
                         "max_over_median": round(step_ms[worst] / med, 3),
                         "after_churn": round(step_ms[post_churn], 4) if post_churn >= 0 else None,
                         "pass": "a third pass of the same structure, one HIP event per step boundary"},
    }
    return res, lens


RADIX_B, RADIX_PREFIX = 16, 2040


def run_radix(args):
    """Radix prefix sharing + copy-on-write: a 2040-token prompt (127 full pages and a
    page holding 8 tokens) is prefilled once and released, which caches its pages in
    the radix tree, the partial last page included; 16 requests whose prompts start
    with it are admitted through the tree (all 2040 tokens matched by token ids: the
    partial page is shared, refcount 17 with the tree's). Their suffixes (128..1024
    tokens) are then prefilled in one ragged forward: each request's first write
    lands in slot 8 of the shared page, so each copies it (kv_cache.py:586-591) and
    the tree keeps the original. Then `--steps` decode steps of all 16.
    Decode bytes count the 127 shared pages once (distinct pages); the kernel reads
    them once per request, and how many of those reads reach HBM is the caches'
    business, so the per-request total is reported beside it as effective GB/s."""
    import torch
    from nanoslg_amd import kernels
    from nanoslg_amd.kv_cache import KVCacheConfig, PagedKVCache
    B, PRE = RADIX_B, RADIX_PREFIX
    full = PRE // PS
    rng = np.random.default_rng(args.seed)
    suffix = [int(x) for x in rng.integers(128, 1025, size=B)]
    steps = args.steps
    # prompt pages, then per request: its suffix and 2 * steps + warmup decode tokens
    # (timed pass + roofline pass) after the 8 shared tokens, plus its copy of the page
    pages = full + 1 + sum(math.ceil((PRE % PS + s + 2 * steps + args.warmup) / PS) + 1 for s in suffix) + 64
    dev = torch.device("cuda:0")
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=PS,
                        max_pages=pages, dtype=torch.float16, device=dev, enable_prefix_caching=True,
                        backend="paged")
    ids = [f"r{b}" for b in range(B)]

    def admitted(mgr, rng, randn):
        """The owner's prompt prefilled and released into the tree, then the B requests
        admitted on it: their prompts all match the 2040 tokens."""
        prompt = rng.integers(0, 128256, size=PRE).tolist()
        mgr.allocate_sequence("owner", token_ids=prompt)
        ctx = mgr.begin_forward(["owner"], [PRE])
        ctx.attend(0, randn(1, PRE, HQ, D), randn(1, PRE, HKV, D), randn(1, PRE, HKV, D), HQ, HKV)
        mgr.end_forward(ctx)
        owner_pages = mgr.seqs["owner"].bt[:full + 1].tolist()
        mgr.release_sequence("owner")  # caches its 127 full pages and its partial page
        for sid, n in zip(ids, suffix):
            tids = prompt + rng.integers(0, 128256, size=n).tolist()
            plen = mgr.allocate_sequence(sid, token_ids=tids)
            assert plen == PRE, plen
        assert mgr.pool.ref_count[owner_pages[full]] == B + 1
        return owner_pages

    # The whole scenario once on a throwaway manager of the same size (its own token
    # ids and K/V), so the timed forward below measures the work and not what a
    # process pays once: kernels loaded on their first launch, the upload ring's
    # pinned buffers and the side stream of large plans
    gw = torch.Generator(device=dev).manual_seed(args.seed + 1)
    randn_w = lambda *shape: torch.randn(*shape, generator=gw, device=dev, dtype=torch.float16)  # noqa: E731
    warm = PagedKVCache(cfg)
    admitted(warm, np.random.default_rng(args.seed + 1), randn_w)
    S = max(suffix)
    wctx = warm.begin_forward(ids, suffix)
    wctx.attend(0, randn_w(B, S, HQ, D), randn_w(B, S, HKV, D), randn_w(B, S, HKV, D), HQ, HKV)
    warm.end_forward(wctx)
    assert len(wctx.cow_pairs) == B
    torch.cuda.synchronize()
    del warm, wctx

    mgr = PagedKVCache(cfg)
    timed = EventTimedKernels(kernels)
    mgr.kernels = timed
    g = torch.Generator(device=dev).manual_seed(args.seed)
    randn = lambda *shape: torch.randn(*shape, generator=g, device=dev, dtype=torch.float16)  # noqa: E731
    owner_pages = admitted(mgr, rng, randn)
    # suffix prefill with copy-on-write of the shared page (the collector settled and
    # paused as around the decode steps: a full collection walks every object of the
    # process, 15-36 ms here, and had landed in this forward in some runs)
    S = max(suffix)
    q, k, v = randn(B, S, HQ, D), randn(B, S, HKV, D), randn(B, S, HKV, D)
    _settle_gc()
    torch.cuda.synchronize()
    with _GcPaused():
        t0 = time.perf_counter()
        ctx = mgr.begin_forward(ids, suffix)
        ctx.attend(0, q, k, v, HQ, HKV)
        mgr.end_forward(ctx)
        torch.cuda.synchronize()
        suffix_ms = (time.perf_counter() - t0) * 1e3
    cow = len(ctx.cow_pairs)
    assert cow == B and all(mgr.seqs[s].bt[full] != owner_pages[full] for s in ids)
    # decode
    ring = 8
    qd, kd, vd = randn(ring, B, 1, HQ, D), randn(ring, B, 1, HKV, D), randn(ring, B, 1, HKV, D)
    inputs = [(qd[i], kd[i], vd[i]) for i in range(ring)]  # sliced once, outside the steps

    def step(i):
        c = mgr.begin_forward(ids, [1] * B)
        q, k, v = inputs[i % ring]
        c.attend(0, q, k, v, HQ, HKV)
        mgr.end_forward(c)

    def lens():
        return [mgr.seqs[s].num_tokens + 1 for s in ids]

    _settle_gc()
    for i in range(args.warmup):
        step(i)
    torch.cuda.synchronize()
    shared_bytes = full * PS * HKV * D * 2 * 2
    nbytes = eff = kbytes = 0
    L0 = lens()
    for i in range(steps):  # bytes of each step, from the lengths (one token per step)
        L = [x + i for x in L0]
        tp = sum(math.ceil(x / PS) for x in L)
        kv, app, qo, csr = step_bytes(L, B, tp)
        nbytes += kv - (B - 1) * shared_bytes + app + qo + csr
        eff += kv + app + qo + csr
    with _GcPaused():
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for i in range(steps):
            step(i)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    assert lens() == [x + steps for x in L0]
    timed.recording = True
    with _GcPaused():
        for i in range(steps):
            L = lens()
            kbytes += decode_call_bytes(L, B, sum(math.ceil(x / PS) for x in L)) - (B - 1) * shared_bytes
            step(i)
        torch.cuda.synchronize()
    timed.recording = False
    mean_ms = timed.mean_ms()
    kbytes /= steps
    value = nbytes / wall / 1e9
    _log(f"suffix prefill + {cow} copy-on-writes: {suffix_ms:.2f} ms; decode {wall / steps * 1e3:.3f} ms/step, "
         f"{value:.1f} GB/s distinct, {eff / wall / 1e9:.1f} GB/s effective; decode call {mean_ms * 1e3:.1f} us")
    # The decode call of one steady step with and without the prefix groups (the
    # shared prefix read once per group of 4, or once per request), kernel time only:
    # 10 calls captured in a HIP graph, replayed with events around the replays.
    c = mgr.begin_forward(ids, [1] * B)
    plan = c.plan
    kl, vl = mgr.pool.k[0], mgr.pool.v[0]
    qs = qd[0][:, 0]
    ab = {}
    for label, grp in (("grouped", plan.groups), ("per_request", None)):
        if label == "grouped" and grp is None:
            continue
        out = torch.empty(B, HQ, D, dtype=torch.float16, device=dev)
        ab[label] = _graph_time_us(torch, dev, lambda: kernels.paged_decode(
            qs, kl, vl, plan.indptr, plan.indices, plan.lpl, plan.total_pages, out=out,
            workspace=mgr.workspace, groups=grp))
    ngroups = plan.groups.num_groups if plan.groups is not None else 0
    _log(f"decode call, kernel time: {ab} ({ngroups} prefix groups)")
    long_ab = _grouped_decode_ab(kernels, dev, B=16, prefix=16384, seed=args.seed)
    _log(f"same with a 16384-token shared prefix: {long_ab}")
    return {
        "metric": "paged decode attn+append with a shared radix prefix: HBM GB/s (distinct pages) and tok/s/layer",
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall / steps * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16 (fp32 accumulate)",
        "data": "synthetic: Q/K/V ~ N(0,1), token ids ~ U[0,128256), seeded",
        "config": {"workload": "radix_prefix_cow", "batch": B, "shared_prefix": PRE, "suffix": "U[128,1024]",
                   "page_size": PS, "heads": f"{HQ}q/{HKV}kv", "head_dim": D, "layers": 1, "seed": args.seed},
        "effective_GB_s": round(eff / wall / 1e9, 2),
        "decode_tok_s_layer": round(B * steps / wall, 1),
        "suffix_prefill_ms": round(suffix_ms, 3),
        "copy_on_write_pages": cow,
        "prefix_groups": ngroups,
        "decode_call_kernel_us": ab,
        "decode_call_kernel_us_prefix16384": long_ab,
        "roofline": {
            "bound": "hbm",
            "kernel": "nslg_paged_decode_append (split-K decode kernel, which also writes the step's new K/V rows, + LSE merge kernel)",
            "timing": f"HIP events around each of {steps} decode calls in a second pass",
            "achieved": round(kbytes / (mean_ms * 1e-3) / 1e9, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(kbytes / (mean_ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": round(mean_ms * 1e3, 2),
            "algorithmic_bytes_per_launch": int(kbytes),
        },
    }


def _graph_time_us(torch, dev, call, n=10, reps=20):
    """Kernel time per call: n calls captured in a HIP graph, replayed `reps` times
    with events around the replays (no host overhead in the figure)."""
    call()
    torch.cuda.synchronize()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        call()
        torch.cuda.current_stream(dev).synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(n):
                call()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    return round(e0.elapsed_time(e1) / (n * reps) * 1e3, 2)


def _grouped_decode_ab(kernels, dev, B, prefix, seed):
    """Decode of B requests sharing a `prefix`-token prefix (own suffixes U[128,1024]),
    with the prefix grouped (read once per group of 4) and per request: kernel time
    of each, straight on the kernels with a block table built here."""
    import torch
    rng = np.random.default_rng(seed + 1)
    pp = prefix // PS
    suf = rng.integers(128, 1025, size=B)
    lens = [prefix + int(x) for x in suf]
    own = [math.ceil(int(x) / PS) for x in suf]
    P = pp + sum(own) + 8
    perm = rng.permutation(np.arange(1, P)).tolist()
    shared, off, tables = perm[:pp], pp, []
    for n in own:
        tables.append(shared + perm[off:off + n])
        off += n
    indptr = np.zeros(B + 1, np.int32)
    np.cumsum([len(t) for t in tables], out=indptr[1:])
    indices = np.concatenate(tables).astype(np.int32)
    lpl = np.array([L - (len(t) - 1) * PS for L, t in zip(lens, tables)], np.int32)
    g = torch.Generator(device=dev).manual_seed(seed)
    k = torch.randn(P, PS, HKV, D, generator=g, device=dev, dtype=torch.float16)
    v = torch.randn(P, PS, HKV, D, generator=g, device=dev, dtype=torch.float16)
    q = torch.randn(B, HQ, D, generator=g, device=dev, dtype=torch.float16)
    ip, ix, lp = (torch.from_numpy(a).to(dev) for a in (indptr, indices, lpl))
    M = 16 // (HQ // HKV)
    groups = kernels.DecodeGroups(B, [list(range(i, min(B, i + M))) for i in range(0, B, M)],
                                  [pp] * ((B + M - 1) // M), dev)
    ws = kernels.Workspace(dev)
    out = torch.empty(B, HQ, D, dtype=torch.float16, device=dev)
    res = {}
    for label, grp in (("grouped", groups), ("per_request", None)):
        res[label] = _graph_time_us(torch, dev, lambda: kernels.paged_decode(
            q, k, v, ip, ix, lp, int(indptr[-1]), out=out, workspace=ws, groups=grp))
    distinct = (pp + sum(own)) * PS * HKV * D * 2 * 2
    res["distinct_GB_s_grouped"] = round(distinct / (res["grouped"] * 1e-6) / 1e9, 1)
    return res


PREFILL_B, PREFILL_LEN, PREFILL_CHUNK = 8, 4096, 512


def prefill_flops(B, L, Hq, D, start=0, n=None):
    """Algorithmic flops of causal attention for rows [start, start+n) of B sequences:
    4*Hq*D per (row, visible key); row p sees keys 0..p."""
    n = L - start if n is None else n
    keys = (start + 1 + start + n) * n // 2
    return 4 * Hq * D * B * keys


def prefill_bytes(B, L, CH, Hq, Hkv, D, ps):
    """Algorithmic HBM bytes of the prefill launch over the L // CH chunks of a batch
    (fp16): per chunk q read and out written once, the K and V of every key the chunk
    sees (its own and the earlier chunks') read once, the chunk's own K/V rows written
    into their pages once (the write is inside the launch), and the page ids."""
    total = 0
    for c in range(L // CH):
        keys = (c + 1) * CH
        total += (2 * B * CH * Hq * D * 2 + B * keys * Hkv * D * 2 * 2 + B * CH * Hkv * D * 2 * 2
                  + 4 * B * (keys // ps))
    return total


def run_prefill(args):
    """Chunked prefill: 8 sequences x 4096 tokens, each fed as 8 chunks of 512 through
    the drop-in API (begin_forward -> attend -> end_forward): every chunk appends its
    K/V to fresh pages, then attends causally (bottom-right) to all earlier pages and
    itself. One step = the whole batch prefilled (8 chunked forwards); sequences are
    released and re-admitted between steps, outside the timed region."""
    import torch
    from nanoslg_amd import kernels
    from nanoslg_amd.kv_cache import KVCacheConfig, PagedKVCache
    B, L, CH = PREFILL_B, PREFILL_LEN, PREFILL_CHUNK
    # the layer's width stays Llama-3.1-8B's (Hq*D = 4096, Hkv*D = 1024, GQA 4) at other head dims
    D = args.head_dim
    HQ, HKV = 4096 // D, 1024 // D
    nchunks = L // CH
    dev = torch.device("cuda:0")
    dt = torch.bfloat16 if args.dtype == "bf16" else torch.float16
    cfg = KVCacheConfig(num_layers=1, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=PS,
                        max_pages=B * L // PS + 64, dtype=dt, device=dev,
                        enable_prefix_caching=False, backend="paged")
    mgr = PagedKVCache(cfg)
    timed = EventTimedKernels(kernels)
    mgr.kernels = timed
    g = torch.Generator(device=dev).manual_seed(args.seed)
    q = torch.randn(nchunks, B, CH, HQ, D, generator=g, device=dev, dtype=dt)
    k = torch.randn(nchunks, B, CH, HKV, D, generator=g, device=dev, dtype=dt)
    v = torch.randn(nchunks, B, CH, HKV, D, generator=g, device=dev, dtype=dt)
    ids = [f"p{b}" for b in range(B)]

    def admit():
        for sid in ids:
            mgr.allocate_sequence(sid)

    def prefill():
        for c in range(nchunks):
            ctx = mgr.begin_forward(ids, [CH] * B)
            ctx.attend(0, q[c], k[c], v[c], HQ, HKV)
            mgr.end_forward(ctx)

    def release():
        for sid in ids:
            mgr.release_sequence(sid)

    _settle_gc()
    for _ in range(max(1, args.warmup // 8)):
        admit()
        prefill()
        release()
    torch.cuda.synchronize()
    steps = args.steps
    wall = 0.0
    with _GcPaused():
        for _ in range(steps):
            admit()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            prefill()
            torch.cuda.synchronize()
            wall += time.perf_counter() - t0
            release()
    ms_step = wall / steps * 1e3
    flops = prefill_flops(B, L, HQ, D)
    tflops = flops / (wall / steps) / 1e12
    _log(f"{steps} prefills in {wall*1e3:.1f} ms -> {ms_step:.3f} ms each, {tflops:.1f} TFLOP/s")
    # roofline pass: events around each prefill kernel call
    timed.recording = True
    for _ in range(steps):
        admit()
        prefill()
        release()
    torch.cuda.synchronize()
    timed.recording = False
    kernel_ms = timed.total_ms() / steps
    achieved = flops / (kernel_ms * 1e-3) / 1e12
    alg_per_launch = prefill_bytes(B, L, CH, HQ, HKV, D, PS) / nchunks
    _log(f"prefill kernel: {kernel_ms:.3f} ms per 8 chunks ({len(timed.events)} launches), {achieved:.1f} TFLOP/s")
    res = {
        "metric": "chunked prefill attention: TFLOP/s (causal, algorithmic) and prefill tok/s/layer",
        "value": round(tflops, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": f"{args.dtype} (fp32 accumulate)",
        "data": "synthetic: Q/K/V ~ N(0,1), seeded",
        "config": {"workload": "chunked_prefill", "batch": B, "tokens_per_seq": L, "chunk": CH,
                   "page_size": PS, "heads": f"{HQ}q/{HKV}kv", "head_dim": D, "layers": 1},
        "prefill_tok_s_layer": round(B * L / (wall / steps), 1),
        "flops_per_step": flops,
        "roofline": {
            "bound": "mfma",
            "kernel": "nslg_paged_prefill_append (8 chunk launches per step, each writing its chunk's K/V)",
            "timing": f"HIP events around each of {len(timed.events)} prefill calls in a second pass",
            "achieved": round(achieved, 2),
            "peak": MFMA_F16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_F16_PEAK_TFLOPS, 4),
            "traffic": (int(round(PREFILL_TRAFFIC_PER_ALGORITHMIC_BYTE * alg_per_launch)) if D == 128 else None),
            "algorithmic_bytes_per_launch": int(alg_per_launch),
            "avg_launch_us": round(timed.mean_ms() * 1e3, 2),
        },
    }
    return res


def _eager_rope(x, cos, sin, pos_ids):
    """The model's rotation as eager tensor ops (nanoslg/models.py:69-83, 96-103), for
    timing beside the fused kernel."""
    import torch
    c = cos[pos_ids][:, :, None, :].to(dtype=x.dtype)
    s = sin[pos_ids][:, :, None, :].to(dtype=x.dtype)
    half = x.shape[-1] // 2
    return x * c + torch.cat((-x[..., half:], x[..., :half]), dim=-1) * s


def _graph_kernel_us(torch, dev, fn, steps):
    """Kernel time of fn: 10 calls captured in a HIP graph, replayed with events around
    the replays (no host overhead in the figure)."""
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        fn()
        torch.cuda.current_stream(dev).synchronize()
        with torch.cuda.graph(graph, stream=side):
            for _ in range(10):
                fn()
    torch.cuda.synchronize()
    graph.replay()
    torch.cuda.synchronize()
    reps = max(1, steps // 10)
    st = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(st)
    for _ in range(reps):
        graph.replay()
    e1.record(st)
    torch.cuda.synchronize()
    del graph
    return round(e0.elapsed_time(e1) / (reps * 10) * 1e3, 2)


def _rope_decode_layer(args, kernels, cos, sin, rng, g):
    """A RoPE model's decode layer at the small-batch shape (4 sequences of 1-4k
    tokens, fp16, pages 16): nslg_rope_append then nslg_paged_decode (the rotated q
    through memory, two launches and the merge) against nslg_paged_decode_rope_append
    (q and the new K rows rotated in the decode launch). Time per call from a loop of
    `--steps` calls (host included) and graph-timed kernel time; outputs and pool
    bytes compared."""
    import torch
    dev = torch.device("cuda:0")
    B = 4
    lens = [int(x) for x in rng.integers(1024, 4097, size=B)]
    npg = [-(-n // PS) for n in lens]
    P = sum(npg) + 64
    ids = rng.permutation(np.arange(1, P)).astype(np.int32)
    tabs, o = [], 0
    for n in npg:
        tabs.append(ids[o:o + n])
        o += n
    i32 = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(dev)  # noqa: E731
    indptr = i32(np.concatenate([[0], np.cumsum(npg)]))
    indices = i32(np.concatenate(tabs))
    lpl = i32([n - (k - 1) * PS for n, k in zip(lens, npg)])
    slots = i32([int(t[(n - 1) // PS]) * PS + (n - 1) % PS for t, n in zip(tabs, lens)])
    pos = i32([n - 1 for n in lens])
    k_pool = torch.randn(P, PS, HKV, D, generator=g, device=dev, dtype=torch.float16)
    v_pool = torch.randn(P, PS, HKV, D, generator=g, device=dev, dtype=torch.float16)
    q = torch.randn(B, HQ, D, generator=g, device=dev, dtype=torch.float16)
    k = torch.randn(B, HKV, D, generator=g, device=dev, dtype=torch.float16)
    v = torch.randn(B, HKV, D, generator=g, device=dev, dtype=torch.float16)
    total = sum(npg)
    ws_a, ws_b = kernels.Workspace(dev), kernels.Workspace(dev)
    q_rot, out_a, out_b = torch.empty_like(q), torch.empty_like(q), torch.empty_like(q)

    def two_launch():
        kernels.rope_append(q, k, v, pos, slots, cos, sin, k_pool, v_pool, q_out=q_rot)
        return kernels.paged_decode(q_rot, k_pool, v_pool, indptr, indices, lpl, total, out=out_a, workspace=ws_a)

    def fused():
        return kernels.paged_decode_rope_append(q, k, v, pos, cos, sin, k_pool, v_pool, indptr, indices, lpl, total,
                                                out=out_b, workspace=ws_b)

    a = two_launch().clone()
    pool_a = k_pool.clone()
    b = fused()
    torch.cuda.synchronize()
    res = {"sequences": B, "contexts": lens, "bit_exact": bool(torch.equal(a, b) and torch.equal(pool_a, k_pool))}
    for label, fn in (("rope_append_then_decode", two_launch), ("decode_rope_append", fused)):
        for _ in range(args.warmup):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(args.steps):
            fn()
        torch.cuda.synchronize()
        res[f"{label}_us"] = round((time.perf_counter() - t0) / args.steps * 1e6, 2)
        res[f"{label}_kernel_us"] = _graph_kernel_us(torch, dev, fn, args.steps)
    _log(f"decode_layer_b4: {res}")
    return res


def run_rope(args):
    """Fused rotary embedding + K/V append (nslg_rope_append) against the model's
    sequence it replaces (gather cos/sin at the positions, eager rotation of q and
    k_new, then the append kernel), per layer, at two shapes: a decode step of 64
    sequences (positions log-uniform in [2048, 32768]) and a prefill chunk of 8 x 512
    tokens. Both write the same pool bytes and q (checked here). One step = one call
    of each at each shape; time per call from a loop of `--steps` calls."""
    import torch
    from nanoslg_amd import kernels
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(args.seed)
    R = 32768
    # Llama-3.1 tables (theta 500000, llama3 scaling), float32 [R, D] on the device
    f = 1.0 / (500000.0 ** (torch.arange(0, D, 2)[: D // 2].float() / D))
    wl = 2 * math.pi / f
    s_ = (8192 / wl - 1.0) / 3.0
    f = torch.where(wl < 2048, f, torch.where(wl > 8192, f / 8, (1 - s_) * f / 8 + s_ * f))
    ang = torch.outer(torch.arange(R, dtype=torch.float32), f)
    ang = torch.cat((ang, ang), -1)
    cos, sin = ang.cos().to(dev), ang.sin().to(dev)
    P = 8192
    k_pool = torch.zeros(P, PS, HKV, D, dtype=torch.float16, device=dev)
    v_pool = torch.zeros_like(k_pool)
    rng = np.random.default_rng(args.seed)
    out = {}
    for name, B, S in (("decode_b64", 64, 1), ("prefill_8x512", 8, 512)):
        T = B * S
        if S == 1:
            pos = np.exp(rng.uniform(math.log(2048), math.log(32768), size=B)).astype(np.int64).reshape(B, 1)
        else:
            pos = (np.arange(S)[None, :] + rng.integers(0, R - S, size=(B, 1))).astype(np.int64)
        pos_ids = torch.from_numpy(pos).to(dev)
        pos32 = pos_ids.reshape(-1).to(torch.int32)
        slots = torch.from_numpy(rng.permutation(P * PS)[:T].astype(np.int32)).to(dev)
        q = torch.randn(B, S, HQ, D, generator=g, device=dev, dtype=torch.float16)
        k = torch.randn(B, S, HKV, D, generator=g, device=dev, dtype=torch.float16)
        v = torch.randn(B, S, HKV, D, generator=g, device=dev, dtype=torch.float16)

        def eager():
            qr = _eager_rope(q, cos, sin, pos_ids)
            kr = _eager_rope(k, cos, sin, pos_ids)
            kernels.append_kv(kr, v, slots, k_pool, v_pool)
            return qr

        q_out = torch.empty_like(q)

        def fused():
            return kernels.rope_append(q, k, v, pos32, slots, cos, sin, k_pool, v_pool, q_out=q_out)

        qa = eager().clone()
        ka = k_pool.clone()
        qb = fused()
        torch.cuda.synchronize()
        same = bool(torch.equal(qa, qb) and torch.equal(ka, k_pool))
        res = {"tokens": T, "bit_exact_with_eager": same}
        for label, fn in (("eager", eager), ("fused", fused)):
            for _ in range(args.warmup):
                fn()
            torch.cuda.synchronize()
            with _GcPaused():
                t0 = time.perf_counter()
                for _ in range(args.steps):
                    fn()
                torch.cuda.synchronize()
                res[f"{label}_us"] = round((time.perf_counter() - t0) / args.steps * 1e6, 2)
        # kernel-only time of the fused launch: 20 launches captured in a HIP graph
        # (the launch itself allocates nothing and sets no memory), replayed with events
        # around the replays on the replay stream, so host overhead does not show
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(side):
            fused()
            torch.cuda.current_stream(dev).synchronize()
            with torch.cuda.graph(graph, stream=side):
                for _ in range(20):
                    fused()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        reps = max(1, args.steps // 20)
        st = torch.cuda.current_stream(dev)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(st)
        for _ in range(reps):
            graph.replay()
        e1.record(st)
        torch.cuda.synchronize()
        res["fused_kernel_us"] = round(e0.elapsed_time(e1) / (reps * 20) * 1e3, 2)
        qc = fused().clone()
        torch.cuda.synchronize()
        res["bit_exact_with_eager"] = same and bool(torch.equal(qc, qa))
        del graph
        nbytes = T * (HQ * D * 2 * 2 + HKV * D * 2 * 4 + D * 4 * 2 + 8)
        res["algorithmic_bytes"] = nbytes
        res["fused_GB_s"] = round(nbytes / (res["fused_kernel_us"] * 1e-6) / 1e9, 1)
        res["speedup"] = round(res["eager_us"] / res["fused_us"], 2)
        _log(f"{name}: {res}")
        out[name] = res
    out["decode_layer_b4"] = _rope_decode_layer(args, kernels, cos, sin, rng, g)
    big = out["prefill_8x512"]
    return {
        "metric": "fused RoPE + K/V append: achieved HBM GB/s (prefill chunk) and us per layer",
        "value": big["fused_GB_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round((big["fused_us"] + out["decode_b64"]["fused_us"]) / 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: Q/K/V ~ N(0,1), seeded; Llama-3.1 rope tables (theta 5e5, llama3 scaling)",
        "config": {"workload": "rope_append", "shapes": {"decode_b64": "64 x 1", "prefill_8x512": "8 x 512"},
                   "heads": f"{HQ}q/{HKV}kv", "head_dim": D, "page_size": PS, "layers": 1},
        "shapes": out,
        "roofline": {
            "bound": "hbm",
            "kernel": "nslg_rope_append at the 8 x 512 prefill chunk",
            "timing": "HIP events around replays of a HIP graph of 20 launches (kernel time without host overhead)",
            "achieved": big["fused_GB_s"],
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(big["fused_GB_s"] / HBM_PEAK_GBS, 4),
            "traffic": None,
            "avg_launch_us": big["fused_kernel_us"],
            "algorithmic_bytes_per_launch": big["algorithmic_bytes"],
        },
    }


def main():
    args = _parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}).", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(1)
    if args.workload == "copy_calibration":
        print(json.dumps(copy_calibration()), flush=True)
        return
    if args.workload == "prefill":
        print(json.dumps(run_prefill(args)), flush=True)
        return
    if args.workload == "radix":
        print(json.dumps(run_radix(args)), flush=True)
        return
    if args.workload == "rope":
        print(json.dumps(run_rope(args)), flush=True)
        return
    if args.workload in ("kv_pressure", "small_batch"):
        res, lens = run_decode(args)
    else:
        print(f"workload {args.workload} is not implemented yet", file=sys.stderr)
        sys.exit(2)
    if not args.no_cpu_baseline:
        _log("cpu baseline ...")
        res["cpu_baseline"] = cpu_baseline_sample(lens, args.seed)
    print(json.dumps(res), flush=True)


if __name__ == "__main__":
    main()
