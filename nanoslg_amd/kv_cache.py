"""KV cache for MI355X: paged pool + radix prefix sharing + contiguous fallback.

Drop-in for nanoslg/kv_cache.py. The public surface keeps the reference's names
and call shapes so the model code is unchanged:

  KVCacheConfig            kv_cache.py:59-145
  CacheContext (ABC)       kv_cache.py:149-163   get_position_ids / attend / get_start_pos
  KVCacheManager (ABC)     kv_cache.py:166-189   allocate/extend/begin/end/release/...
  PagePool                 kv_cache.py:382-442
  RadixTree                kv_cache.py:445-531
  PagedKVCache             kv_cache.py:694-777   (the reference's FlashInferPagedKVCache)
  PagedCacheContext        kv_cache.py:545-691   (the reference's FlashInferCacheContext)
  ContiguousKVCache        kv_cache.py:328-379
  ContiguousCacheContext   kv_cache.py:247-325
  create_cache_manager     kv_cache.py:780-805

Below `attend` every byte of K/V is moved and every attention output computed
by the hand-written gfx950 kernels in libnslg_kv.so (see ``kernels``): the
append scatter, the batched zero/copy of pages, split-K paged decode and the
MFMA chunked-prefill kernel. The host side here only keeps integer bookkeeping
(free list, refcounts, block tables, radix tree) and builds each forward's plan
(slot mapping, CSR block table, positions) with numpy, uploaded in one pinned
host-to-device copy. There is no CPU attention path.
"""
from __future__ import annotations

import gc
import math
import threading
import weakref
from abc import ABC, abstractmethod
from dataclasses import dataclass
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

_BACKENDS = ("paged", "contiguous")


def _check_head_dim(cfg: "KVCacheConfig", kernels) -> None:
    """A cache is only built for a (dtype, head_dim) every kernel it uses supports,
    so an unsupported model fails at construction rather than at its first prefill."""
    dims = getattr(kernels, "HEAD_DIMS", None)
    dev = torch.device(cfg.device) if cfg.device is not None else None
    if dims is not None and dev is not None and dev.type == "cuda" and cfg.head_dim not in dims.get(cfg.dtype, ()):
        raise ValueError(f"KV cache: head_dim {cfg.head_dim} is not supported for {cfg.dtype} "
                         f"(supported: {dims.get(cfg.dtype, ())})")


def _default_kernels():
    from . import kernels
    return kernels


def _host_planner():
    from . import _lib
    return _lib.host().plan_forward


# --------------------------------------------------------------------------------------
# configuration
# --------------------------------------------------------------------------------------


@dataclass
class KVCacheConfig:
    """Pool geometry and backend choice (kv_cache.py:59-145).

    backend: "auto" and "flashinfer" select the paged HIP backend; "contiguous"
    selects the [L, Bmax, Smax, Hkv, D] pool. Heads are per tensor-parallel rank."""
    num_layers: int
    num_kv_heads: int
    num_qo_heads: int
    head_dim: int
    page_size: int = 16
    max_pages: int = 0            # 0 = size from free device memory (paged)
    max_batch_size: int = 8       # contiguous
    max_seq_len: int = 4096       # contiguous
    memory_fraction: float = 0.30
    dtype: torch.dtype = torch.bfloat16
    device: torch.device = None
    enable_prefix_caching: bool = True
    backend: str = "auto"
    max_pages_cap: int = 65536    # the reference's auto-size cap (kv_cache.py:97)
    # Radix sharing of partial last pages (the reference shares full pages only,
    # kv_cache.py:459-486): a released sequence also caches its last partial page,
    # prompts shorter than a page are matched too, and a prefix ending inside a page
    # shares that page; the first write into it copies it (copy-on-write).
    share_partial_pages: bool = True

    def __post_init__(self):
        if self.backend in ("auto", "flashinfer"):
            self.backend = "paged"
        if self.backend not in _BACKENDS:
            raise ValueError(f"unknown KV backend {self.backend!r}; use auto|paged|contiguous")
        if self.num_qo_heads % self.num_kv_heads:
            raise ValueError("num_qo_heads must be a multiple of num_kv_heads")
        if self.backend == "paged" and self.max_pages <= 0:
            self.max_pages = self._auto_pages()
        if self.backend == "contiguous":
            self._auto_seq_len()

    def _elem_bytes(self) -> int:
        return {torch.float16: 2, torch.bfloat16: 2, torch.float32: 4}.get(self.dtype, 2)

    def _device_mem(self) -> Optional[Tuple[int, int]]:
        if self.device is None:
            return None
        dev = torch.device(self.device)
        if dev.type != "cuda" or not torch.cuda.is_available():
            return None
        return torch.cuda.mem_get_info(dev)

    def _auto_pages(self) -> int:
        """kv_cache.py:88-102: budget = (free - max(2 GiB, 15% total)) * fraction."""
        mem = self._device_mem()
        if mem is None:
            return 256
        free, total = mem
        headroom = max(2 << 30, int(total * 0.15))
        budget = int(max(0, free - headroom) * self.memory_fraction)
        per_page = (2 * self.num_layers * self.page_size * self.num_kv_heads * self.head_dim
                    * self._elem_bytes())
        return max(64, min(budget // max(per_page, 1), self.max_pages_cap))

    def _auto_seq_len(self):
        """kv_cache.py:104-117."""
        mem = self._device_mem()
        if mem is None:
            return
        free, _ = mem
        budget = int(free * self.memory_fraction * 0.5)
        per_tok = 2 * self.num_layers * self.num_kv_heads * self.head_dim * self._elem_bytes()
        cap = budget // max(per_tok, 1) // max(self.max_batch_size, 1)
        self.max_seq_len = min(self.max_seq_len, max(512, cap))

    @classmethod
    def from_hf_config(cls, hf_config, parallel_config=None, device=None, **kw) -> "KVCacheConfig":
        """kv_cache.py:119-145 (heads divided by tp; PP layer split if configured)."""
        nl = getattr(hf_config, "num_hidden_layers", getattr(hf_config, "num_layers", 32))
        nkv = getattr(hf_config, "num_key_value_heads",
                      getattr(hf_config, "multi_query_group_num",
                              getattr(hf_config, "num_attention_heads", 32)))
        nq = getattr(hf_config, "num_attention_heads", 32)
        hd = getattr(hf_config, "head_dim",
                     getattr(hf_config, "kv_channels", hf_config.hidden_size // nq))
        if parallel_config is not None:
            tp = getattr(parallel_config, "tp_size", 1)
            if tp > 1:
                nkv //= tp
                nq //= tp
            splits = getattr(parallel_config, "pp_layer_splits", None)
            rank = getattr(parallel_config, "pp_rank", None)
            if getattr(parallel_config, "pp_size", 1) > 1 and splits and rank in splits:
                nl = len(splits[rank])
        return cls(num_layers=nl, num_kv_heads=nkv, num_qo_heads=nq, head_dim=hd, device=device, **kw)


# --------------------------------------------------------------------------------------
# the drop-in ABCs (kv_cache.py:149-189)
# --------------------------------------------------------------------------------------


class CacheContext(ABC):
    seq_ids: List[str]
    new_token_counts: List[int]
    input_offsets: List[int]
    batch_size: int
    seq_lens: List[int]

    @abstractmethod
    def get_position_ids(self, max_input_len: int) -> torch.Tensor: ...

    @abstractmethod
    def attend(self, layer_idx: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
               n_heads: int, n_kv_heads: int) -> torch.Tensor: ...

    @abstractmethod
    def get_start_pos(self, batch_idx: int = 0) -> int: ...

    def get_position(self, max_input_len: int) -> torch.Tensor:
        """Alias of get_position_ids (the name used in the reference's README)."""
        return self.get_position_ids(max_input_len)


class KVCacheManager(ABC):
    cfg: KVCacheConfig

    @abstractmethod
    def allocate_sequence(self, seq_id: str, token_ids: Optional[List[int]] = None,
                          num_tokens: int = 0) -> int: ...

    @abstractmethod
    def extend_sequence(self, seq_id: str, num_new: int = 1): ...

    @abstractmethod
    def begin_forward(self, seq_ids: List[str], new_token_counts: List[int],
                      input_offsets: Optional[List[int]] = None) -> CacheContext: ...

    @abstractmethod
    def end_forward(self, ctx: CacheContext): ...

    @abstractmethod
    def release_sequence(self, seq_id: str): ...

    @abstractmethod
    def append_token_ids(self, seq_id: str, new_ids: List[int]): ...

    @abstractmethod
    def reset(self): ...

    @property
    @abstractmethod
    def stats(self) -> Dict: ...


# --------------------------------------------------------------------------------------
# host -> device plan upload
# --------------------------------------------------------------------------------------


_STREAMS: Dict[int, torch.cuda.Stream] = {}


def _current_stream(index: int) -> torch.cuda.Stream:
    """Device `index`'s current stream as a torch Stream (one object per stream id),
    without the device lookup torch.cuda.current_stream() and Event.record() do on
    every call (about 15 us each)."""
    sid, di, dt = torch._C._cuda_getCurrentStream(index)
    st = _STREAMS.get(sid)
    if st is None:
        st = _STREAMS[sid] = torch.cuda.Stream(stream_id=sid, device_index=di, device_type=dt)
    return st


class _PlanStaging:
    """Host-to-device staging of per-forward int32 plans on one device.

    The plan is written straight into a pinned host buffer taken from a small ring
    (a buffer is refilled only after the copy that last read it has completed, which
    its event records) and moved with one async copy.

    Large plans (big batches, where the GPU has a long queue of work) are copied on
    a side stream of default priority into memory allocated on that stream; the
    compute stream waits for the copy through the same event, so the copy of forward
    i+1 overlaps the kernels of forward i, and the destination is recorded on the
    compute stream, so the allocator does not hand it out again while those kernels
    may still read it. Small plans are copied on the compute stream itself: there
    the GPU waits on the host anyway, and a cross-stream wait costs the host about
    20 us per forward."""

    RING = 4
    SIDE_STREAM_BYTES = 64 << 10

    def __init__(self, device: torch.device):
        self.device = device
        self.index = device.index if device.index is not None else torch.cuda.current_device()
        self.side = torch.cuda.Stream(device=device)  # default priority
        self.host: List[Optional[torch.Tensor]] = [None] * self.RING
        self.host_np: List[Optional[np.ndarray]] = [None] * self.RING
        self.copied = [torch.cuda.Event() for _ in range(self.RING)]
        self.pending = [False] * self.RING
        self.next = 0

    def reserve(self, n: int) -> None:
        """Pin ring buffers of at least n int32 each now, so that no forward whose plan
        fits pays for a pinned allocation (which costs milliseconds)."""
        for k in range(self.RING):
            buf = self.host[k]
            if buf is None or buf.numel() < n:
                if self.pending[k]:
                    self.copied[k].synchronize()
                    self.pending[k] = False
                buf = torch.empty(n, dtype=torch.int32, pin_memory=True)
                self.host[k], self.host_np[k] = buf, buf.numpy()

    def take(self, total: int = 0) -> Tuple[int, np.ndarray]:
        """The next ring buffer (slot, its numpy view), holding at least `total`
        entries, free to write: the copy that last read it has completed."""
        k = self.next
        self.next = (k + 1) % self.RING
        if self.pending[k]:
            self.copied[k].synchronize()
            self.pending[k] = False
        return k, self.grow(k, total)

    def grow(self, k: int, total: int) -> np.ndarray:
        """Slot k's buffer, replaced by a larger one if it holds fewer than `total`."""
        buf = self.host[k]
        if buf is None or buf.numel() < total:
            buf = torch.empty(max(total, 1 << 12) * 2, dtype=torch.int32, pin_memory=True)
            self.host[k], self.host_np[k] = buf, buf.numpy()
        return self.host_np[k]

    def upload(self, parts: List[np.ndarray], total: int, extra: int = 0) -> torch.Tensor:
        """The concatenated parts on the device, followed by `extra` entries left
        uninitialised (device outputs of the same forward)."""
        k, host = self.take(total)
        if total:  # one pass over every part (each cast to int32 as it is written)
            np.concatenate(parts, out=host[:total], casting="unsafe")
        return self.send(k, total, extra)

    def send(self, k: int, total: int, extra: int = 0) -> torch.Tensor:
        """Slot k's first `total` entries, written by the caller, copied to a new
        device buffer of total + extra entries."""
        buf = self.host[k]
        self.pending[k] = True
        size = max(total + extra, 1)
        if 4 * total <= self.SIDE_STREAM_BYTES:
            dev = torch.empty(size, dtype=torch.int32, device=self.device)
            if total:
                (dev if total == size else dev[:total]).copy_(buf[:total], non_blocking=True)
            self.copied[k].record(_current_stream(self.index))  # on the compute stream
            return dev
        main = _current_stream(self.index)
        with torch.cuda.stream(self.side):
            dev = torch.empty(size, dtype=torch.int32, device=self.device)
            dev[:total].copy_(buf[:total], non_blocking=True)
            self.copied[k].record(self.side)
        main.wait_event(self.copied[k])
        dev.record_stream(main)
        return dev


_STAGING: Dict[int, _PlanStaging] = {}


def _staging(device: torch.device) -> _PlanStaging:
    idx = device.index if device.index is not None else torch.cuda.current_device()
    st = _STAGING.get(idx)
    if st is None:
        st = _PlanStaging(torch.device("cuda", idx))
        _STAGING[idx] = st
    return st


def _upload_i32(parts: List[np.ndarray], device: torch.device, extra: int = 0) -> List[torch.Tensor]:
    """Concatenate int32 arrays, copy them to `device` at once, return the views (one
    per part; with extra > 0, one more view of `extra` uninitialised entries in the
    same buffer, for a device output). On a GPU this goes through the device's
    _PlanStaging."""
    parts = [a if isinstance(a, np.ndarray) and a.ndim == 1 else np.asarray(a).reshape(-1) for a in parts]
    sizes = [a.size for a in parts]
    total = sum(sizes)
    if device.type == "cuda":
        dev = _staging(device).upload(parts, total, extra)
    else:
        dev = torch.from_numpy(np.concatenate([np.asarray(a, dtype=np.int32).reshape(-1) for a in parts]
                                              + [np.zeros(extra, np.int32)])).clone()
    if extra:
        sizes = sizes + [extra]
    if dev.numel() > sum(sizes):
        sizes = sizes + [dev.numel() - sum(sizes)]
        return list(dev.split(sizes))[:-1]
    return list(dev.split(sizes))


def _ragged_layout(start_positions, new_token_counts, input_offsets, iw):
    """Vectorised input-grid layout of one forward.

    Returns (positions [B*iw] int32, rows [T] int64, qo_indptr [B+1] int64): positions
    pos[b, off_b+t] = start_b + t and zero elsewhere (kv_cache.py:267-278); rows are the
    flat [B*iw] indices of the new tokens in ragged (sequence-major) order."""
    B = len(start_positions)
    n = np.asarray(new_token_counts, np.int64).reshape(B)
    start = np.asarray(start_positions, np.int64).reshape(B)
    offs = np.asarray(input_offsets, np.int64).reshape(B)
    qo = np.zeros(B + 1, np.int64)
    np.cumsum(n, out=qo[1:])
    T = int(qo[-1])
    b_idx = np.repeat(np.arange(B, dtype=np.int64), n)
    t_in = np.arange(T, dtype=np.int64) - np.repeat(qo[:-1], n)
    rows = b_idx * iw + offs[b_idx] + t_in
    pos = np.zeros(B * iw, np.int32)
    pos[rows] = start[b_idx] + t_in
    return pos, rows, qo


class _ForwardPlan:
    """Device-side metadata of one forward, shared by every layer's attend()."""

    def __init__(self, device, batch, iw, slot_grid, positions, indptr, indices, lpl, qo_indptr,
                 q_rows, cow_src, cow_dst, zero_ids=None, group_slot=None):
        zero_ids = np.zeros(0, np.int32) if zero_ids is None else np.asarray(zero_ids, np.int32)
        parts = [slot_grid, positions, indptr, indices, lpl, qo_indptr, q_rows, cow_src, cow_dst, zero_ids]
        if group_slot is not None:
            parts.append(group_slot)
        up = _upload_i32(parts, device)
        (self.slot, self.pos_i32, self.indptr, self.indices, self.lpl, self.qo_indptr, self.q_rows,
         self.cow_src, self.cow_dst, self.zero_ids) = up[:10]
        self.group_slot = up[10] if group_slot is not None else None
        self.groups = None  # kernels.DecodeGroups of a decode batch with shared prefixes
        self.batch, self.iw = batch, iw
        self.total_pages = int(indptr[-1]) if len(indptr) else 0
        self.total_q = int(qo_indptr[-1]) if len(qo_indptr) else 0
        self._slot_by_S: Dict[int, torch.Tensor] = {iw: self.slot}
        self._pos_long: Optional[torch.Tensor] = None

    @classmethod
    def from_device(cls, batch, slot, pos, indptr, indices, lpl, qo_indptr, q_rows, zero_ids, total_pages,
                    groups=None):
        """A decode plan whose tables were built on the device (decode_plan_step); the
        prefix groups carry over from the previous step (shared pages are never
        written, so a group's prefix does not change while the batch stays)."""
        self = cls.__new__(cls)
        self.groups = groups
        self.group_slot = groups.seq_group_slot if groups is not None else None
        self.slot, self.pos_i32, self.indptr, self.indices, self.lpl = slot, pos, indptr, indices, lpl
        self.qo_indptr, self.q_rows = qo_indptr, q_rows
        self.cow_src = self.cow_dst = None  # a decode step planned on the device copies no page
        self.zero_ids = zero_ids
        self.batch, self.iw = batch, 1
        self.total_pages = int(total_pages)
        self.total_q = batch
        self._slot_by_S = {1: slot}
        self._pos_long = None
        return self

    @classmethod
    def from_tensors(cls, batch, iw, slot, pos, indptr, indices, lpl, qo_indptr, q_rows, cow_src, cow_dst, zero_ids,
                     total_pages, total_q):
        """A plan whose per-token arrays were expanded on the device (forward_plan)."""
        self = cls.__new__(cls)
        self.slot, self.pos_i32, self.indptr, self.indices, self.lpl = slot, pos, indptr, indices, lpl
        self.qo_indptr, self.q_rows = qo_indptr, q_rows
        self.cow_src, self.cow_dst, self.zero_ids = cow_src, cow_dst, zero_ids
        self.batch, self.iw = batch, iw
        self.total_pages = int(total_pages)
        self.total_q = int(total_q)
        self._slot_by_S = {iw: slot}
        self._pos_long = None
        self.groups = None
        self.group_slot = None
        return self

    def slots_for(self, S: int) -> torch.Tensor:
        s = self._slot_by_S.get(S)
        if s is None:
            grid = self.slot.view(self.batch, self.iw)
            if S < self.iw:
                s = grid[:, :S].contiguous().view(-1)
            else:
                pad = torch.full((self.batch, S - self.iw), -1, dtype=torch.int32, device=grid.device)
                s = torch.cat([grid, pad], 1).view(-1)
            self._slot_by_S[S] = s
        return s

    def rows_for(self, S: int) -> torch.Tensor:
        """Rows of the [B, S] input grid holding the forward's tokens, in ragged order
        (q_rows is for the plan's own width iw: sequence b's rows move by b * (S - iw))."""
        if S == self.iw:
            return self.q_rows
        cache = self.__dict__.setdefault("_rows_by_S", {})
        r = cache.get(S)
        if r is None:
            if S < self.iw:
                raise ValueError(f"the input grid has {S} columns; this forward's tokens need {self.iw}")
            r = cache[S] = self.q_rows + torch.div(self.q_rows, self.iw, rounding_mode="floor") * (S - self.iw)
        return r

    def pos_for(self, S: int) -> torch.Tensor:
        """int32 positions of the [B, S] input grid, flattened (zeros on padding)."""
        if S == self.iw:
            return self.pos_i32
        p = self._pos_by_S.get(S) if hasattr(self, "_pos_by_S") else None
        if p is None:
            grid = self.pos_i32.view(self.batch, self.iw)
            if S < self.iw:
                p = grid[:, :S].contiguous().view(-1)
            else:
                p = torch.cat([grid, grid.new_zeros(self.batch, S - self.iw)], 1).view(-1)
            if not hasattr(self, "_pos_by_S"):
                self._pos_by_S = {}
            self._pos_by_S[S] = p
        return p

    def positions_long(self) -> torch.Tensor:
        if self._pos_long is None:
            self._pos_long = self.pos_i32.view(self.batch, self.iw).long()
        return self._pos_long


def _get_positions(plan: _ForwardPlan, batch: int, iw: int, S: int) -> torch.Tensor:
    pos = plan.positions_long()
    if S <= iw:
        return pos[:, :S]
    return torch.cat([pos, pos.new_zeros(batch, S - iw)], 1)


# --------------------------------------------------------------------------------------
# page pool (kv_cache.py:382-442)
# --------------------------------------------------------------------------------------


class PagePool:
    """K and V pools [L, P, page_size, Hkv, D] on the device; page 0 is the permanent
    null/sink page. Host state: int32 refcounts and tokens_used, a LIFO free stack
    (lowest ids first on a fresh pool). Zero-on-alloc and copy-on-write are batched
    device launches."""

    def __init__(self, cfg: KVCacheConfig, kernels=None):
        self.cfg = cfg
        self.kernels = kernels or _default_kernels()
        P = cfg.max_pages
        if P < 2:
            raise ValueError("max_pages must be >= 2 (page 0 is reserved)")
        shape = (cfg.num_layers, P, cfg.page_size, cfg.num_kv_heads, cfg.head_dim)
        dev = torch.device(cfg.device) if cfg.device is not None else torch.device("cpu")
        self.device = dev
        self.k = torch.zeros(shape, dtype=cfg.dtype, device=dev)
        self.v = torch.zeros(shape, dtype=cfg.dtype, device=dev)
        self.ref_count = np.zeros(P, np.int64)
        self.tokens_used = np.zeros(P, np.int64)
        self.ref_count[0] = 1
        self._is_free = np.zeros(P, bool)
        self._is_free[1:] = True
        self._free: List[int] = list(range(P - 1, 0, -1))
        self._mark = np.zeros(P, bool)  # scratch page set for mark_filter, all False between calls
        self._lock = threading.Lock()
        self._layers: List[Tuple[torch.Tensor, torch.Tensor]] = []

    def layer(self, i: int) -> Tuple[torch.Tensor, torch.Tensor]:
        """The K and V pool views of layer i ([P, ps, Hkv, D]), made once."""
        if not self._layers:
            self._layers = list(zip(self.k.unbind(0), self.v.unbind(0)))
        return self._layers[i]

    # -- allocation --------------------------------------------------------------------
    def alloc(self, n: int = 1, zero: bool = True) -> Optional[List[int]]:
        """All-or-nothing allocation of n pages (refcount 1, tokens_used 0).
        Returns None when fewer than n are free. zero=True zeroes them on the device
        (all layers, K and V) in one launch."""
        got = self.alloc_ids(n, zero)
        return None if got is None else got[0]

    def alloc_ids(self, n: int, zero: bool = True) -> Optional[Tuple[List[int], np.ndarray]]:
        """alloc(n, zero), the pages also as an int64 array."""
        with self._lock:
            if len(self._free) < n:
                return None
            # the same pages, in the same order, as n pops from the end of the stack
            out = self._free[:-n - 1:-1] if n else []
            del self._free[len(self._free) - n:]
            idx = np.asarray(out, np.int64)
            self.ref_count[idx] = 1
            self.tokens_used[idx] = 0
            self._is_free[idx] = False
        if zero and out:
            self.zero(out)
        return out, idx

    def mark_filter(self, ids: np.ndarray, drop: np.ndarray) -> np.ndarray:
        """The entries of ids that are not in drop, in order (np.isin's result, through
        a page-indexed mark: a few fancy-index passes instead of a sort)."""
        mark = self._mark
        mark[drop] = True
        keep = ids[~mark[ids]]
        mark[drop] = False
        return keep

    def zero(self, page_ids: List[int]) -> None:
        if not page_ids:
            return
        (ids,) = _upload_i32([np.asarray(page_ids, np.int32)], self.device)
        self.kernels.zero_pages(self.k, self.v, ids)

    def release(self, pid: int) -> None:
        if pid <= 0:
            return
        with self._lock:
            self.ref_count[pid] -= 1
            if self.ref_count[pid] <= 0:
                self.ref_count[pid] = 0
                self.tokens_used[pid] = 0
                if not self._is_free[pid]:
                    self._is_free[pid] = True
                    self._free.append(pid)

    def release_many(self, pids) -> None:
        """release(p) for each p of pids, in order (the same refcounts, tokens_used and
        free-list order), vectorised when the ids are distinct (a block table's are)."""
        ids = np.asarray(pids, np.int64)
        ids = ids[ids > 0]
        if ids.size == 0:
            return
        if np.unique(ids).size != ids.size:
            for p in ids.tolist():
                self.release(p)
            return
        with self._lock:
            rc = self.ref_count[ids] - 1
            gone = rc <= 0
            self.ref_count[ids] = np.where(gone, 0, rc)
            freed = ids[gone]
            self.tokens_used[freed] = 0
            freed = freed[~self._is_free[freed]]
            self._is_free[freed] = True
            self._free.extend(freed.tolist())

    def add_ref(self, pid: int) -> None:
        with self._lock:
            self.ref_count[pid] += 1

    def is_shared(self, pid: int) -> bool:
        return bool(self.ref_count[pid] > 1)

    def cow_alloc(self, pid: int) -> Optional[int]:
        """Host half of copy-on-write (kv_cache.py:429-436): a new page with the source's
        tokens_used; the device copy is issued by copy(). Does not release pid."""
        new = self.alloc(1, zero=False)
        if new is None:
            return None
        d = new[0]
        self.tokens_used[d] = self.tokens_used[pid]
        return d

    def copy(self, src_ids, dst_ids) -> None:
        if len(src_ids) == 0:
            return
        src, dst = _upload_i32([np.asarray(src_ids, np.int32), np.asarray(dst_ids, np.int32)], self.device)
        self.kernels.copy_pages(self.k, self.v, src, dst)

    def cow(self, pid: int) -> Optional[int]:
        """Single-page copy-on-write: allocate, copy all layers and slots, return the id."""
        d = self.cow_alloc(pid)
        if d is not None:
            self.copy([pid], [d])
        return d

    @property
    def num_free(self) -> int:
        return len(self._free)

    @property
    def utilization(self) -> float:
        return 1.0 - self.num_free / max(self.cfg.max_pages - 1, 1)


# --------------------------------------------------------------------------------------
# radix prefix tree (kv_cache.py:445-531), page granular
# --------------------------------------------------------------------------------------


class _RNode:
    __slots__ = ("children", "partials", "page_id", "ref", "last_access", "depth")

    def __init__(self, depth=0):
        self.children: Dict[tuple, "_RNode"] = {}  # full pages: edge = its ps token ids
        self.partials: Dict[tuple, "_RNode"] = {}  # partial pages (leaves): edge = their 1..ps-1 token ids
        self.page_id = -1
        self.ref = 0
        self.last_access = 0
        self.depth = depth


class RadixTree:
    """Prefix tree over pages of token ids. Node depth is in pages; each edge is the
    tuple of page_size token ids of one page; a node may hold the id of a pool page with
    those tokens' K/V. As in the reference (kv_cache.py:459-486) full pages are shared;
    with share_partial a node may also hold partial pages: leaves keyed by the 1 ..
    ps-1 token ids written into a released sequence's last page, whose page then holds
    those tokens' K/V. match returns, after its full pages, the longest partial page
    that continues the prompt; the first write into it (at the slot after its tokens)
    copies it (copy-on-write, kv_cache.py:575-594: the tree holds a reference, so it
    is always shared then).

    Differences from the reference's per-token trie, on purpose:
      * match returns pages only up to the first page node whose page was evicted
        (an interior eviction), so the pages always cover tokens [0, ps*len(pages));
        the reference returns the deeper pages too, leaving a gap (kv_cache.py:467).
        The walk itself, its access stamps and its invalidation of pages whose
        refcount dropped to zero are the reference's, so eviction order stays the same;
      * access times come from a counter, so ties only arise within one call, as
        with the reference's monotonic clock (LRU ties keep DFS pre-order). A call
        stamps the nodes of one token path, and on one path the trie's pre-order is
        depth order, so partial children are visited before full ones (shortest
        first): pre-order on every path is depth order here too."""

    def __init__(self, ps: int, pool: PagePool, share_partial: bool = False):
        self.root = _RNode()
        self.ps = ps
        self.pool = pool
        self.share_partial = share_partial
        self._lock = threading.Lock()
        self._clock = 0

    def _now(self) -> int:
        self._clock += 1
        return self._clock

    def _partials_on_path(self, node, tokens, at):
        """(length, node) of the partial children of `node` whose ids are a prefix of
        tokens[at:], shortest first (the token path passes through them in that
        order)."""
        if not node.partials:
            return []
        out = []
        for r in range(1, min(self.ps - 1, len(tokens) - at) + 1):
            pn = node.partials.get(tuple(tokens[at:at + r]))
            if pn is not None:
                out.append((r, pn))
        return out

    def _walk(self, tokens):
        """The page-tree nodes on the token path of `tokens`, in depth order: at each
        full-page node reached (the root first), its partial children on the path,
        then the next full page's node, while one continues the path. Yields
        (node, partial_len): partial_len > 0 for a partial page of that many tokens."""
        node, ps, i = self.root, self.ps, 0
        while True:
            for r, pn in self._partials_on_path(node, tokens, i * ps):
                yield pn, r
            if len(tokens) - i * ps < ps:
                return
            ch = node.children.get(tuple(tokens[i * ps:(i + 1) * ps]))
            if ch is None:
                return
            node = ch
            i += 1
            yield node, 0

    def match(self, tokens) -> Tuple[int, List[int]]:
        with self._lock:
            pages, now, ps = [], self._now(), self.ps
            contiguous = True
            best, best_len = -1, 0  # the longest partial page after the contiguous full pages
            full_seen = 0
            for node, r in self._walk(tokens):
                node.last_access = now
                if r:
                    if node.page_id >= 0 and self.pool.ref_count[node.page_id] <= 0:
                        node.page_id = -1
                    if self.share_partial and contiguous and node.page_id >= 0 and full_seen == len(pages):
                        best, best_len = node.page_id, r
                    continue
                full_seen += 1
                if node.page_id < 0:
                    contiguous = False  # evicted inside the path: no page past here
                    continue
                if self.pool.ref_count[node.page_id] > 0:
                    if contiguous:
                        pages.append(node.page_id)
                        best, best_len = -1, 0  # a partial page only extends the full pages before it
                else:
                    node.page_id = -1
                    break
            plen = len(pages) * ps
            if best >= 0:
                pages.append(best)
                plen += best_len
            return plen, pages

    def insert(self, tokens, page_ids) -> None:
        """Cache the pages of tokens: page i holds tokens [ps*i, ps*i + ps); with
        share_partial, a last page of fewer than ps tokens (page_ids holding one more
        id) becomes a partial page. A node keeps the page it already holds."""
        with self._lock:
            node, now, ps = self.root, self._now(), self.ps
            nf = len(tokens) // ps
            for i in range(nf + 1):
                # the token path passes through the partial pages on it: stamped as well
                for _, pn in self._partials_on_path(node, tokens, i * ps):
                    pn.last_access = now
                if i == nf:
                    break
                key = tuple(tokens[i * ps:(i + 1) * ps])
                ch = node.children.get(key)
                if ch is None:
                    ch = _RNode(i + 1)
                    node.children[key] = ch
                node = ch
                node.last_access = now
                if i < len(page_ids) and node.page_id < 0:
                    node.page_id = page_ids[i]
                    self.pool.add_ref(page_ids[i])
            r = len(tokens) - nf * ps
            if self.share_partial and r and nf < len(page_ids):
                key = tuple(tokens[nf * ps:])
                pn = node.partials.get(key)
                if pn is None:
                    pn = _RNode(nf + 1)
                    node.partials[key] = pn
                pn.last_access = now
                if pn.page_id < 0:  # a partial page starts unpinned
                    pn.page_id = page_ids[nf]
                    pn.ref = 0
                    self.pool.add_ref(page_ids[nf])

    def add_refs(self, tokens, n: int = 1) -> None:
        """Pin the nodes on the token path (kv_cache.py:488-495)."""
        with self._lock:
            for node, _ in self._walk(tokens):
                node.ref += n

    def dec_refs(self, tokens, n: int = 1) -> None:
        with self._lock:
            for node, _ in self._walk(tokens):
                node.ref = max(0, node.ref - n)

    def evict_lru(self, need: int) -> int:
        """Release unpinned cached pages, least recently used first (stable: DFS
        pre-order on ties), dropping emptied leaves. Returns pages released."""
        with self._lock:
            cands: list = []
            self._collect(self.root, cands)
            cands.sort(key=lambda x: x[0])
            freed = 0
            for _, nd, par, edge, partial in cands:
                if freed >= need:
                    break
                if nd.ref > 0:
                    continue
                if nd.page_id >= 0:
                    self.pool.release(nd.page_id)
                    nd.page_id = -1
                    freed += 1
                if par is not None and not nd.children and not nd.partials:
                    (par.partials if partial else par.children).pop(edge, None)
            return freed

    def _collect(self, node, out, par=None, edge=None):
        """Unpinned page nodes in DFS pre-order: a node, its partial children (shortest
        first), then its full children in insertion order."""
        stack = [(node, par, edge, False)]
        while stack:
            nd, pa, ed, partial = stack.pop()
            if nd.page_id >= 0 and nd.ref == 0:
                out.append((nd.last_access, nd, pa, ed, partial))
            for t, ch in reversed(list(nd.children.items())):
                stack.append((ch, nd, t, False))
            for t, ch in sorted(nd.partials.items(), key=lambda kv: -len(kv[0])):
                stack.append((ch, nd, t, True))

    @property
    def cached_pages(self) -> int:
        c, stack = 0, [self.root]
        while stack:
            n = stack.pop()
            if n.page_id >= 0:
                c += 1
            stack.extend(n.children.values())
            stack.extend(n.partials.values())
        return c


# --------------------------------------------------------------------------------------
# paged backend
# --------------------------------------------------------------------------------------


class _PagedSeqState:
    """Per-sequence state (kv_cache.py:534-542); the block table is an int32 array.

    The table also lives on the device, as a row of the cache's _BlockTableArena:
    `row`/`row_cap` locate it there (-1 before the sequence's first forward) and
    `synced` counts the leading entries the device row already holds. Entries are
    only appended (extend) or replaced through set_page, which lowers `synced`, so
    the device row never goes stale."""
    __slots__ = ("seq_id", "bt", "n_pages", "num_tokens", "prefix_len", "token_ids", "row", "row_cap", "synced")

    def __init__(self, sid, prefix_pages=None, plen=0, tids=None):
        self.seq_id = sid
        pages = list(prefix_pages or [])
        self.bt = np.zeros(max(16, 2 * len(pages)), np.int32)
        self.bt[:len(pages)] = pages
        self.n_pages = len(pages)
        self.num_tokens = plen
        self.prefix_len = plen
        self.token_ids = list(tids or [])
        self.row, self.row_cap, self.synced = -1, 0, 0

    @property
    def block_table(self) -> List[int]:
        return self.bt[:self.n_pages].tolist()

    def extend(self, pages: List[int]) -> None:
        need = self.n_pages + len(pages)
        if need > self.bt.size:
            nb = np.zeros(max(need, 2 * self.bt.size), np.int32)
            nb[:self.n_pages] = self.bt[:self.n_pages]
            self.bt = nb
        self.bt[self.n_pages:need] = pages
        self.n_pages = need

    def set_page(self, i: int, pid: int) -> None:
        """Logical page i now lives in pool page pid (copy-on-write, shared pages)."""
        self.bt[i] = pid
        if i < self.synced:
            self.synced = i


class _BlockTableArena:
    """The cache's block tables on the device: one int32 row per live sequence in a
    persistent device array (row entry i = the pool page of logical page i).

    A forward builds its CSR block table from these rows on the device
    (nslg_block_table_csr), uploading only the entries its sequences gained or
    changed since their rows were last used; that launch also writes those entries
    into the rows. Rows have power-of-two capacities (at least 1.5x the table when
    placed, so decode growth rarely moves them) and are recycled through
    per-capacity free lists; a table that outgrows its row moves to a larger one
    and is uploaded whole once. The array doubles when full (a device copy on the
    current stream, so every launch that used the old array comes first)."""

    MIN_ROW = 16

    def __init__(self, device: torch.device, capacity: int):
        self.device = device
        self.dev = torch.zeros(max(int(capacity), self.MIN_ROW), dtype=torch.int32, device=device)
        self.top = 0
        self.free: Dict[int, List[int]] = {}

    def _take(self, need: int) -> Tuple[int, int]:
        cap = self.MIN_ROW
        while cap < need:
            cap *= 2
        lst = self.free.get(cap)
        if lst:
            return lst.pop(), cap
        if self.top + cap > self.dev.numel():
            n = self.dev.numel()
            while n < self.top + cap:
                n *= 2
            grown = torch.zeros(n, dtype=torch.int32, device=self.device)
            grown[:self.top].copy_(self.dev[:self.top])
            self.dev = grown
        off = self.top
        self.top += cap
        return off, cap

    def place(self, st: _PagedSeqState) -> None:
        """Make sure st has a row that holds its whole table (a fresh row starts
        unsynced)."""
        if st.row >= 0 and st.n_pages <= st.row_cap:
            return
        self.release(st)
        st.row, st.row_cap = self._take(st.n_pages + st.n_pages // 2)
        st.synced = 0

    def release(self, st: _PagedSeqState) -> None:
        if st.row >= 0:
            self.free.setdefault(st.row_cap, []).append(st.row)
        st.row, st.row_cap, st.synced = -1, 0, 0


class PagedCacheContext(CacheContext):
    """Per-forward context (kv_cache.py:545-691): positions, the write plan with
    copy-on-write, the CSR block table; attend() = append kernel + paged attention."""

    def __init__(self, cache: "PagedKVCache", seq_ids, new_token_counts, input_offsets,
                 zero_pages: Optional[List[int]] = None):
        self.cache = cache
        self.seq_ids = list(seq_ids)
        self.new_token_counts = list(new_token_counts)
        self.input_offsets = list(input_offsets) if input_offsets else [0] * len(seq_ids)
        self.batch_size = B = len(seq_ids)
        cfg, pool, ps = cache.cfg, cache.pool, cache.cfg.page_size
        states = [cache.seqs[s] for s in self.seq_ids]
        self.start_positions = [st.num_tokens for st in states]
        self.seq_lens = [a + n for a, n in zip(self.start_positions, self.new_token_counts)]
        self.max_kv_len = max(self.seq_lens) if self.seq_lens else 0
        self._is_decode = B > 0 and self.new_token_counts.count(1) == B
        if self._is_decode and not input_offsets:
            self._iw = 1  # one token per sequence, no padding
        else:
            self._iw = max(o + n for o, n in zip(self.input_offsets, self.new_token_counts)) if B else 1
        iw = self._iw

        # write plan + copy-on-write, in batch order (kv_cache.py:575-594): a shared page
        # is copied by every writer but the last remaining sharer, which writes in place.
        cow_src: List[int] = []
        cow_dst: List[int] = []

        def _cow(st, p):
            pid = int(st.bt[p])
            new = pool.cow_alloc(pid)
            tree = cache.tree
            if new is None and tree is not None and tree.share_partial and tree.evict_lru(1) > 0:
                # with partial pages shared, copies are common: a copy may evict a cached
                # page, as any allocation does (kv_cache.py:760-768); if that released
                # the page's other reference, the page is written in place
                if not pool.is_shared(pid):
                    return
                new = pool.cow_alloc(pid)
            if new is None:
                # The copies made so far stand (the reference copies each page as it
                # goes, kv_cache.py:429-436, and does not undo them on the error).
                if cow_src:
                    pool.copy(cow_src, cow_dst)
                raise RuntimeError("KV OOM during CoW")
            cow_src.append(pid)
            cow_dst.append(new)
            st.set_page(p, new)
            pool.release(pid)

        self._decode_launch = None
        if self._is_decode and iw == 1:
            plan = cache._advance_decode_plan(self.seq_ids, states, zero_pages)
            if plan is not None:
                self.cow_pairs = []
                self._max_q, self._uniform_rows = 1, True
                self._plan = plan
                cache._record_decode_plan(self.seq_ids, plan, self.seq_lens)
                return
        # Every forward with new tokens takes the native planner and one device launch
        # for its CSR and per-token plan (PagedKVCache._plan_forward_native), unless it
        # writes a shared page: copy-on-write stays with the numpy path below.
        if cache.NATIVE_PLAN and hasattr(cache.kernels, "_forward_plan_csr"):
            T = sum(self.new_token_counts)
            if T >= self.NATIVE_PLAN_TOKENS:
                got = cache._plan_forward_native(states, self.new_token_counts, self.input_offsets, iw, T,
                                                 list(zero_pages) if zero_pages else None)
                if got is not None:
                    self._plan, nz, shared_first = got
                    self.cow_pairs = []
                    self._max_q = max(self.new_token_counts)
                    self._uniform_rows = T == B * iw
                    if self._is_decode and iw == 1 and shared_first:
                        # the decode batch's prefix groups (only sequences whose first page
                        # is shared can form one)
                        npg = [(n + ps) // ps for n in self.start_positions]  # pages after the step
                        groups = cache._prefix_groups(states, npg)
                        if groups is not None:
                            kern = cache.kernels
                            (slot,) = _upload_i32([groups[2]], pool.device)
                            self._plan.group_slot = slot
                            self._plan.groups = kern.DecodeGroups(B, groups[0], groups[1], pool.device,
                                                                  seq_group_slot=slot)
                    if nz:  # zero-on-alloc of the pages this forward's extensions took
                        cache.kernels.zero_pages(pool.k, pool.v, self._plan.zero_ids)
                    if self._is_decode and iw == 1:
                        cache._record_decode_plan(self.seq_ids, self._plan, self.seq_lens)
                    return
        # Below, the host works per sequence and per written page only. The CSR block
        # table itself (kv_cache.py:598-615) is built on the device from the cache's
        # device-resident block tables (PagedKVCache._plan_upload).
        start = np.fromiter(self.start_positions, np.int64, B)
        have = np.fromiter((st.n_pages for st in states), np.int64, B)
        zero = np.asarray(zero_pages if zero_pages else [], np.int32)
        groups = None
        device_plan = False
        if self._is_decode and iw == 1:
            # One token per sequence, vectorised over the batch. Only a page that is
            # shared before any copy can need one, so the candidates are re-checked in
            # batch order, which reproduces the sequential rule exactly.
            lens = start + 1
            npg = (lens + ps - 1) // ps
            pi = npg - 1
            sl = start - pi * ps
            ok = pi < have
            pids = np.fromiter((st.bt.item(p) if o else 0 for st, p, o in zip(states, pi.tolist(), ok.tolist())),
                               np.int64, B)
            cand = np.nonzero(ok & (pool.ref_count[pids] > 1))[0]
            for b in cand.tolist():
                st = states[b]
                if pool.is_shared(int(st.bt[pi[b]])):
                    _cow(st, int(pi[b]))
                    pids[b] = st.bt[pi[b]]
            slot = np.where(ok, pids * ps + sl, 0).astype(np.int32)
            if ok.any():  # the written pages are distinct after copy-on-write
                w = pids[ok]
                pool.tokens_used[w] = np.maximum(pool.tokens_used[w], sl[ok] + 1)
            lpl = lens - pi * ps
            pos = start.astype(np.int32)
            q_rows = np.arange(B, dtype=np.int32)
            qo = np.arange(B + 1, dtype=np.int32)
            groups = cache._prefix_groups(states, npg)
        else:
            ncnt = np.fromiter(self.new_token_counts, np.int64, B)
            lens = start + ncnt
            npg = np.where(lens > 0, (lens + ps - 1) // ps, 0)
            # The pages this forward writes that the sequences have: sequence b writes
            # pages p0_b .. p0_b + cnt_b - 1 (start//ps .. (start+n-1)//ps, those below
            # its page count); their ids, concatenated in batch order, are `wp`.
            n = np.maximum(ncnt, 0)
            p0 = start // ps
            plast = (start + n - 1) // ps
            cnt = np.where(n > 0, np.maximum(np.minimum(plast + 1, have) - p0, 0), 0)
            wfirst = np.zeros(B, np.int64)
            if B:
                np.cumsum(cnt[:-1], out=wfirst[1:])
            tot = int(cnt.sum())
            if tot:
                wp = np.concatenate([st.bt[a:a + c] for st, a, c in zip(states, p0.tolist(), cnt.tolist()) if c]
                                    ).astype(np.int64)
                # copy-on-write, in batch order. Copies only lower refcounts, so only a
                # page shared before any copy can need one: those are found on `wp` at
                # once, then the rule is applied to their sequences in batch order.
                rep = np.repeat(np.arange(B), cnt)
                hit = pool.ref_count[wp] > 1
                if bool(hit.any()):
                    for b in np.unique(rep[hit]).tolist():
                        st = states[b]
                        for p in range(int(p0[b]), int(p0[b] + cnt[b])):
                            if pool.is_shared(int(st.bt[p])):
                                _cow(st, p)
                                wp[wfirst[b] + p - p0[b]] = st.bt[p]
                # tokens_used (kv_cache.py:593): each written page once, with its last
                # slot written; the pages written are distinct after copy-on-write
                pidx = p0[rep] + (np.arange(tot, dtype=np.int64) - wfirst[rep])
                last = np.where(pidx == plast[rep], (start + n - 1 - plast * ps)[rep], ps - 1)
                pool.tokens_used[wp] = np.maximum(pool.tokens_used[wp], last + 1)
                if zero.size:
                    # a page this forward writes in every slot needs no zero-on-alloc: the
                    # append leaves the same bytes (a chunked prefill's pages, but the last)
                    full = (pidx * ps >= start[rep]) & ((pidx + 1) * ps <= (start + n)[rep])
                    if bool(full.any()):
                        zero = pool.mark_filter(zero, wp[full])
            else:
                wp = np.zeros(1, np.int64)
            T = int(ncnt.sum())
            device_plan = T >= self.DEVICE_PLAN_TOKENS and hasattr(cache.kernels, "_forward_plan")
            lpl = np.where(npg > 0, lens - (npg - 1) * ps, 0)
            if B == 0:
                lpl = np.zeros(1, np.int64)
            if not device_plan:
                # per new token: absolute position, page, slot; past a sequence's pages
                # the write goes to the null page's slot 0 (kv_cache.py:583-584)
                slot = np.full(B * iw, -1, np.int32)
                if T:
                    rep = np.repeat(np.arange(B), ncnt)
                    first = np.zeros(B, np.int64)
                    np.cumsum(ncnt[:-1], out=first[1:])
                    t_in = np.arange(T, dtype=np.int64) - first[rep]
                    ap = start[rep] + t_in
                    pi = ap // ps
                    ok = pi < have[rep]
                    pids = np.where(ok, wp[np.where(ok, wfirst[rep] + pi - p0[rep], 0)], 0)
                    sls = np.where(ok, ap - pi * ps, 0)
                    offs = np.fromiter(self.input_offsets, np.int64, B)
                    slot[rep * iw + offs[rep] + t_in] = (pids * ps + sls).astype(np.int32)
                pos, q_rows, qo = _ragged_layout(self.start_positions, self.new_token_counts, self.input_offsets, iw)
        indptr = np.zeros(B + 1, np.int64)
        np.cumsum(npg, out=indptr[1:])
        total_pages = int(indptr[-1])
        self.cow_pairs = list(zip(cow_src, cow_dst))
        self._max_q = max(self.new_token_counts) if B else 0
        cs, cd = np.asarray(cow_src, np.int32), np.asarray(cow_dst, np.int32)
        kern = cache.kernels
        if device_plan:
            # per-token slots, positions and the ragged layout expanded on the device
            offs = np.fromiter(self.input_offsets, np.int64, B)
            fp_sizes = [B * iw, B * iw, T, B + 1]  # forward_plan's outputs, after the CSR indices
            views, d_idx, fp_out = cache._plan_upload(states, indptr, [lpl, cs, cd, zero, start, ncnt, offs, have],
                                                      tail=sum(fp_sizes))
            d_indptr, d_lpl, d_cs, d_cd, d_zero, d_start, d_n, d_off, d_have = views
            slot_t, pos_t, rows_t, qo_t = kern._forward_plan(d_indptr, d_idx, d_start, d_n, d_off, d_have, B, iw,
                                                             ps, T, out=fp_out)
            self._uniform_rows = T == B * iw
            self._plan = _ForwardPlan.from_tensors(B, iw, slot_t, pos_t, d_indptr, d_idx, d_lpl, qo_t, rows_t,
                                                   d_cs, d_cd, d_zero, total_pages, T)
        else:
            parts = [slot.reshape(-1), pos, lpl, qo, q_rows, cs, cd, zero]
            if groups is not None:
                parts.append(groups[2])
            views, d_idx = cache._plan_upload(states, indptr, parts)
            d_indptr, d_slot, d_pos, d_lpl, d_qo, d_qr, d_cs, d_cd, d_zero = views[:9]
            self._uniform_rows = int(qo[-1]) == B * iw  # every grid row carries a new token
            self._plan = _ForwardPlan.from_tensors(B, iw, d_slot, d_pos, d_indptr, d_idx, d_lpl, d_qo, d_qr,
                                                   d_cs, d_cd, d_zero, total_pages, int(qo[-1]))
            if groups is not None:
                self._plan.group_slot = views[9]
                self._plan.groups = kern.DecodeGroups(B, groups[0], groups[1], pool.device,
                                                      seq_group_slot=views[9])
        if zero.size:  # zero-on-alloc of the pages this forward's extensions took
            kern.zero_pages(pool.k, pool.v, self._plan.zero_ids)
        if cow_src:
            kern.copy_pages(pool.k, pool.v, self._plan.cow_src, self._plan.cow_dst)
        if self._is_decode and iw == 1:
            cache._record_decode_plan(self.seq_ids, self._plan, self.seq_lens)

    DEVICE_PLAN_TOKENS = 256  # numpy path: forwards with at least this many new tokens expand their plan on the device
    NATIVE_PLAN_TOKENS = 1  # native path: forwards with at least this many new tokens

    # ---- CacheContext -----------------------------------------------------------------
    def get_position_ids(self, S: int) -> torch.Tensor:
        return _get_positions(self._plan, self.batch_size, self._iw, S)

    def get_start_pos(self, idx: int = 0) -> int:
        return self.start_positions[idx]

    def attend(self, layer_idx, q, k_new, v_new, n_heads, n_kv_heads):
        """Write k_new/v_new into the pages of `layer_idx`, then attend.
        q [B,S,Hq,D], k_new/v_new [B,S,Hkv,D] -> [B,S,Hq*D] in q's dtype."""
        cache, pool, plan = self.cache, self.cache.pool, self._plan
        kern = cache.kernels
        B, S = q.shape[0], q.shape[1]
        if self._is_decode and S == 1:
            launch = self._decode_launch
            if launch is None or launch.bound_plan is not plan:
                launch = self._decode_launch = cache._decode_launcher(plan, q.shape[2])
            return launch(layer_idx, q, k_new, v_new)
        k_layer, v_layer = pool.layer(layer_idx)
        o = self._prefill(q, k_layer, v_layer, k_new, v_new)  # the write and the attention in one launch
        if o is not None:
            return o
        kern._append_kv_layer(k_new, v_new, plan.slots_for(S), k_layer, v_layer)
        return self._prefill(q, k_layer, v_layer)

    def attend_rope(self, layer_idx, q, k_new, v_new, cos, sin, n_heads, n_kv_heads):
        """The position part of the model's attention forward fused with attend
        (models.py:96-105): q and k_new are rotated at this forward's positions
        (get_position_ids) with the model's cos/sin tables, the rotated k and v are
        written into the pages of `layer_idx` in the same launch, then attention runs
        as in attend(). Same result as attend() on q and k_new rotated by the eager
        apply_rotary_emb, bit for bit."""
        cache, pool, plan = self.cache, self.cache.pool, self._plan
        kern = cache.kernels
        B, S = q.shape[0], q.shape[1]
        if self.max_kv_len > cos.shape[0]:
            raise IndexError(f"position {self.max_kv_len - 1} is outside the rope tables ({cos.shape[0]} rows)")
        pos = plan.pos_for(S)
        if self._is_decode and S == 1:
            launch = self._decode_launch
            if launch is None or launch.bound_plan is not plan:
                launch = self._decode_launch = cache._decode_launcher(plan, q.shape[2])
            return launch(layer_idx, q, k_new, v_new, rope=(cos, sin, pos))
        k_layer, v_layer = pool.layer(layer_idx)
        q_rot = kern.rope_append(q, k_new, v_new, pos, plan.slots_for(S), cos, sin, k_layer, v_layer)
        return self._prefill(q_rot, k_layer, v_layer)

    def _prefill(self, q, k_layer, v_layer, k_new=None, v_new=None):
        """Causal attention of the forward's rows (K/V already written). With k_new and
        v_new ([B, S, Hkv, D], the forward's rows): their write into the pages in the
        same launch (16-bit pools), or None where that launch does not apply."""
        cache, plan = self.cache, self._plan
        kern = cache.kernels
        B, S = q.shape[0], q.shape[1]
        Hq, D = q.shape[2], q.shape[3]
        q_grid = q.reshape(B * S, Hq, D)
        if k_new is not None:
            uniform = self._uniform_rows and S == self._iw
            o = kern._paged_prefill_append_layer(
                q_grid, plan.qo_indptr, plan.total_q, self._max_q, k_new, v_new, k_layer, v_layer, plan.indptr,
                plan.indices, plan.lpl, cache.workspace, q_rows=None if uniform else plan.rows_for(S),
                grid_width=0 if uniform else S)
            return None if o is None else o.view(B, S, Hq * D)
        if self._uniform_rows and S == self._iw:  # every grid row is a token: the ragged rows themselves
            o = kern._paged_prefill_layer(q_grid, plan.qo_indptr, plan.total_q, self._max_q, k_layer, v_layer,
                                          plan.indptr, plan.indices, plan.lpl, cache.workspace)
        else:  # padded or ragged: the kernel reads and writes the grid rows (pad rows zero)
            o = kern._paged_prefill_layer(q_grid, plan.qo_indptr, plan.total_q, self._max_q, k_layer, v_layer,
                                          plan.indptr, plan.indices, plan.lpl, cache.workspace,
                                          q_rows=plan.rows_for(S), grid_width=S)
        return o.view(B, S, Hq * D)

    # ---- introspection used by tests and the bench -------------------------------------
    @property
    def plan(self) -> _ForwardPlan:
        return self._plan


class PagedKVCache(KVCacheManager):
    """Paged KV cache manager (kv_cache.py:694-777) on the HIP kernels."""

    def __init__(self, cfg: KVCacheConfig, kernels=None):
        self.cfg = cfg
        self.kernels = kernels or _default_kernels()
        _check_head_dim(cfg, self.kernels)
        self.pool = PagePool(cfg, self.kernels)
        self.tree = (RadixTree(cfg.page_size, self.pool, share_partial=cfg.share_partial_pages)
                     if cfg.enable_prefix_caching else None)
        self.seqs: Dict[str, _PagedSeqState] = {}
        self.workspace = self.kernels.Workspace(self.pool.device, 128 << 20)
        self._pending_zero: List[int] = []
        self._dev_plan = None  # the last decode forward's plan: (ids, plan, lens), see below
        self._launcher = None  # the last decode forward's kernels.DecodeLaunch
        self._pool_args = None  # the pools as the device planner takes them
        self._decode_rows: Dict[int, Tuple[torch.Tensor, torch.Tensor]] = {}
        self._plan_ring = None  # [batch, capacity, buffers, last used] of device-planned decode steps
        self._newp = None  # (batch, int32 [batch] opened-page list, -1 between steps, its address)
        # the block tables on the device (room for every pool page twice before growing)
        self._tables = _BlockTableArena(self.pool.device, 2 * cfg.max_pages + 4096)
        self._host_plan_buf = np.zeros(1 << 12, np.int32)  # the host planner's output off the GPU
        if self.pool.device.type == "cuda":
            _staging(self.pool.device).reserve(self.STAGING_INTS)

    STAGING_INTS = 1 << 16  # pinned plan-upload buffers (int32 each) set up with the cache

    # the host part of a device-planned forward in one native call (False: the numpy
    # path of PagedCacheContext, which takes every forward the native call declines)
    NATIVE_PLAN = True

    def _plan_forward_native(self, states, ntoks, offsets, iw, T, zero_pages):
        """The host part of a forward whose per-token plan is expanded on the device,
        in one call of the host planner (`_nslg_host.plan_forward`): the written
        pages' tokens_used, the pages to zero, the CSR pointers and last-page
        lengths, and the block-table entries the sequences' device rows lack, written
        straight into the upload buffer; then the upload, nslg_block_table_csr and
        nslg_forward_plan, as in PagedCacheContext and _plan_upload (the planner places
        the sequences' device rows itself, once it knows it plans the forward). Returns
        (plan, pages to zero), or None when a page the forward writes is shared
        (copy-on-write takes the numpy path; the call changed nothing then). The two device steps go
        out as one launch (nslg_forward_plan_csr)."""
        tables, pool, kern = self._tables, self.pool, self.kernels
        B, ps = len(states), self.cfg.page_size
        tail = 2 * B * iw + T + B + 1  # forward_plan's outputs: slots, positions, rows, qo_indptr
        plan_forward = _host_planner()
        zl = zero_pages if zero_pages else None
        args = (states, ntoks, offsets, ps, pool.ref_count, pool.tokens_used, pool._mark, zl)
        cuda = pool.device.type == "cuda"
        if cuda:
            stg = _staging(pool.device)
            k, host = stg.take()
        else:
            k, host = -1, self._host_plan_buf
        res = plan_forward(*args, host, tables.place)
        if isinstance(res, int):  # the buffer is too small: nothing was written
            if cuda:
                host = stg.grow(k, -res)
            else:
                host = self._host_plan_buf = np.zeros(2 * -res, np.int32)
            res = plan_forward(*args, host, tables.place)
        if res is None:
            return None
        total, total_pages, npatch, nz, shared_first = res
        extra = max(total_pages, 1) + tail
        if cuda:
            dev = stg.send(k, total, extra)
        else:
            dev = torch.zeros(total + extra, dtype=torch.int32)
            dev[:total] = torch.from_numpy(host[:total])
        # the buffer: indptr (B+1), last-page lengths (B), the pages to zero (nz), then
        # start, new tokens, offsets, pages held, row, pages held, synced (B each), the
        # patch pointers (B+1) and entries, the CSR indices, forward_plan's outputs;
        # views only of what the plan keeps (each view costs the host ~0.5 us)
        n_mid = 8 * B + 1 + max(npatch, 1)
        d_indptr, d_lpl, d_zero, d_mid, d_idx, fp_out = dev.split([B + 1, B, nz, n_mid, max(total_pages, 1), tail])
        if hasattr(kern, "_forward_plan_csr_at"):
            slot_t, pos_t, rows_t, qo_t = kern._forward_plan_csr_at(tables.dev, dev, 2 * B + 1 + nz, npatch, total_pages,
                                                                    B, iw, ps, T, fp_out)
        else:
            (d_start, d_n, d_off, d_have, d_row, d_have2, d_syn, d_pip, d_patch) = d_mid.split(
                [B, B, B, B, B, B, B, B + 1, max(npatch, 1)])
            slot_t, pos_t, rows_t, qo_t = kern._forward_plan_csr(tables.dev, d_row, d_have2, d_syn, d_pip, d_patch,
                                                                 npatch, d_indptr, d_idx, total_pages, d_start, d_n,
                                                                 d_off, B, iw, ps, T, fp_out)
        for st in states:
            st.synced = st.n_pages
        none = d_zero[:0]  # no page copies in this forward
        plan = _ForwardPlan.from_tensors(B, iw, slot_t, pos_t, d_indptr, d_idx, d_lpl, qo_t, rows_t, none, none, d_zero,
                                         total_pages, T)
        return plan, nz, shared_first

    def _plan_upload(self, states, indptr, parts, tail=0):
        """One upload of a forward's host-built plan arrays (`parts`, after the CSR
        pointers `indptr`) together with the block-table entries its sequences gained
        or changed since their device rows were last used; then the forward's CSR
        indices built on the device from those rows (nslg_block_table_csr), which
        also brings the rows up to date. Returns ([indptr] + views of parts,
        kv_indices) on the device; with tail > 0, also a third item: `tail` more
        entries of the same device buffer, left for other device outputs."""
        tables = self._tables
        B = len(states)
        for st in states:
            tables.place(st)
        row = np.fromiter((st.row for st in states), np.int32, B)
        have = np.fromiter((st.n_pages for st in states), np.int32, B)
        syn = np.minimum(np.fromiter((st.synced for st in states), np.int32, B), have)
        pip = np.zeros(B + 1, np.int32)
        np.cumsum(have - syn, out=pip[1:])
        npatch = int(pip[-1])
        patch = (np.concatenate([st.bt[s:h] for st, s, h in zip(states, syn.tolist(), have.tolist()) if h > s])
                 if npatch else np.zeros(1, np.int32))
        total = int(indptr[-1])
        up = _upload_i32([indptr] + list(parts) + [row, have, syn, pip, patch], self.pool.device,
                         extra=max(total, 1) + tail)
        k = len(parts) + 1
        d_row, d_have, d_syn, d_pip, d_patch, d_ext = up[k:k + 6]
        d_idx = d_ext[:max(total, 1)] if tail else d_ext
        self.kernels._block_table_csr(tables.dev, d_row, d_have, d_syn, d_pip, d_patch, npatch, up[0], d_idx,
                                      total, B)
        for st in states:
            st.synced = st.n_pages
        if tail:
            return up[:k], d_idx, d_ext[max(total, 1):]
        return up[:k], d_idx

    # ---- decode plans built on the device ---------------------------------------------
    def _record_decode_plan(self, seq_ids, plan, seq_lens) -> None:
        self._dev_plan = (tuple(seq_ids), plan, list(seq_lens))

    def _decode_launcher(self, plan: "_ForwardPlan", num_qo_heads: int):
        """The decode launcher of a forward: the previous forward's, re-bound to this
        plan, when the batch size and head count are the same (kernels.DecodeLaunch
        checks the pool geometry once)."""
        kern = self.kernels
        prev = self._launcher
        if (prev is not None and hasattr(prev, "rebind") and prev.B == plan.batch and prev.Hq == num_qo_heads
                and prev.workspace is self.workspace):
            prev.rebind(plan.slot, plan.indptr, plan.indices, plan.lpl, plan.total_pages, plan.groups,
                        check=False)
            prev.bound_plan = plan
            return prev
        pool = self.pool
        launch = kern.DecodeLaunch(pool.k, pool.v, plan.slot, plan.indptr, plan.indices, plan.lpl,
                                   plan.total_pages, num_qo_heads, workspace=self.workspace, groups=plan.groups)
        launch.bound_plan = plan
        self._launcher = launch
        return launch

    MIN_GROUP_PAGES = 4

    def _prefix_groups(self, states, npg):
        """Rows of a decode batch whose first pages are the same pages (a shared radix
        prefix): groups of 2 .. 16/G rows, each with the number of full pages all its
        rows share below their last page (at least MIN_GROUP_PAGES), at most 32
        groups. Returns (groups, prefix_pages, seq_group_slot) or None; the decode
        then reads each group's shared pages once for all its rows."""
        B = len(states)
        if B < 2 or getattr(self.kernels, "DecodeGroups", None) is None:
            return None
        if self.cfg.dtype not in getattr(self.kernels, "GROUPED_DECODE_DTYPES", ()):
            return None
        cfg = self.cfg
        M = 16 // max(1, cfg.num_qo_heads // cfg.num_kv_heads)
        if M < 2:
            return None
        first = np.fromiter((int(st.bt[0]) if st.n_pages else 0 for st in states), np.int64, B)
        cand = np.nonzero((first > 0) & (self.pool.ref_count[first] > 1))[0]
        if cand.size < 2:
            return None
        cand = cand[np.argsort(first[cand], kind="stable")]
        keys = first[cand]
        cuts = np.flatnonzero(np.diff(keys)) + 1
        groups, prefixes = [], []
        for run in np.split(cand, cuts):
            run = run.tolist()
            for s0 in range(0, len(run), M):
                sub = run[s0:s0 + M]
                if len(sub) < 2:
                    continue
                cap = min(int(npg[b]) - 1 for b in sub)  # full pages below each row's last page
                if cap < self.MIN_GROUP_PAGES:
                    continue
                tabs = np.stack([states[b].bt[:cap] for b in sub])
                same = (tabs == tabs[0]).all(axis=0)
                common = cap if bool(same.all()) else int(np.argmin(same))
                if common >= self.MIN_GROUP_PAGES:
                    groups.append(sub)
                    prefixes.append(common)
                if len(groups) == 32:
                    break
            if len(groups) == 32:
                break
        if not groups:
            return None
        slot = np.full(B, -1, np.int32)
        for g, sub in enumerate(groups):
            for m, b in enumerate(sub):
                slot[b] = 16 * g + m
        return groups, prefixes, slot

    SCALAR_PLAN_BATCH = 16  # decode batches up to this size are checked in plain Python (cheaper than numpy)
    # steady decode steps of batches up to this size take the one-pass begin_forward
    # (measured cheaper than the general path up to ~200 sequences: at 64, 69 vs 106 us
    # of host time on a slow host)
    ONE_PASS_BATCH = 128

    def _decode_step_pages(self, states, prev_lens, zero_pages):
        """The pages a decode step opens, for the device planner: (new_page [B] int32,
        -1 where the sequence's new token goes into its current last page; count), after
        checking that every sequence gained exactly the previous step's token, has the
        pages the step needs, and writes no shared page, and that the pages opened are
        the ones allocated for it. None when a check fails. Updates tokens_used."""
        B, ps, pool = len(states), self.cfg.page_size, self.pool
        start = np.fromiter((st.num_tokens for st in states), np.int64, B)
        if not np.array_equal(start, prev_lens):
            return None
        npg = start // ps + 1
        if not np.array_equal(np.fromiter((st.n_pages for st in states), np.int64, B), npg):
            return None
        opens = start % ps == 0
        pids = np.fromiter((int(st.bt[k - 1]) for st, k in zip(states, npg.tolist())), np.int64, B)
        if bool((pool.ref_count[pids] > 1).any()):
            return None  # a shared page is written: copy-on-write goes through the host plan
        new_page = np.where(opens, pids, -1).astype(np.int32)
        if sorted(zero_pages or []) != sorted(pids[opens].tolist()):
            return None
        sl = start % ps
        pool.tokens_used[pids] = np.maximum(pool.tokens_used[pids], sl + 1)
        return new_page, int(opens.sum())

    def _decode_step_pages_scalar(self, states, prev_lens, zero_pages):
        """_decode_step_pages for a small batch, one sequence at a time: the same
        checks, result and tokens_used update."""
        ps, rc = self.cfg.page_size, self.pool.ref_count
        pids, new_page, opened = [], [], []
        for st, n in zip(states, prev_lens):
            if st.num_tokens != n:
                return None
            k = n // ps + 1
            if st.n_pages != k:
                return None
            pid = int(st.bt[k - 1])
            if rc[pid] > 1:
                return None  # a shared page is written: copy-on-write goes through the host plan
            pids.append(pid)
            if n % ps == 0:
                new_page.append(pid)
                opened.append(pid)
            else:
                new_page.append(-1)
        if sorted(zero_pages or []) != sorted(opened):
            return None
        tu = self.pool.tokens_used
        for pid, n in zip(pids, prev_lens):
            used = n % ps + 1
            if tu[pid] < used:
                tu[pid] = used
        return np.array(new_page, np.int32), len(opened)

    def _advance_decode_plan(self, seq_ids, states, zero_pages) -> Optional[_ForwardPlan]:
        """This decode forward's plan built on the device from the previous one
        (kernels.decode_plan_step), when the batch is the one the previous decode
        forward planned, every sequence gained exactly that token, and no written page
        is shared; otherwise None and the host builds the plan. The result is the same
        plan as the host's, bit for bit."""
        prev = self._dev_plan
        kern = self.kernels
        if prev is None or prev[0] != tuple(seq_ids) or not hasattr(kern, "decode_plan_step"):
            return None
        B, ps, pool = len(states), self.cfg.page_size, self.pool
        if B == 0 or B > 512:
            return None
        if B <= self.SCALAR_PLAN_BATCH:
            step = self._decode_step_pages_scalar(states, prev[2], zero_pages)
        else:
            step = self._decode_step_pages(states, prev[2], zero_pages)
        if step is None:
            return None
        new_page, n_new = step
        return self._plan_on_device(B, prev[1], new_page, n_new)

    def _plan_on_device(self, B, plan, new_page, n_new, new_page_ptr=None) -> "_ForwardPlan":
        """The next decode plan from `plan` on the device (kernels.decode_plan_step):
        new_page int32 [B], the page sequence b opens this step or -1 (new_page_ptr: its
        address, if known)."""
        kern, pool, ps = self.kernels, self.pool, self.cfg.page_size
        fast = getattr(kern, "_decode_plan_step", None)
        if fast is not None:  # inputs are the previous plan's outputs: no argument checks
            if self._pool_args is None:
                L, P, _, Hkv, D = pool.k.shape
                self._pool_args = (pool.k.data_ptr(), pool.v.data_ptr(), L, P, Hkv, D, kern.dtype_code(pool.k.dtype))
            dst = self._plan_buffers(B, plan.total_pages + n_new)
            indptr, indices, lpl, slot, pos, new = fast(plan.indptr, plan.indices, plan.lpl, new_page, ps, n_new,
                                                        self._pool_args, out=dst, new_page_ptr=new_page_ptr)
        else:
            indptr, indices, lpl, slot, pos, new = kern.decode_plan_step(plan.indptr, plan.indices, plan.lpl,
                                                                        new_page, ps, n_new, pool.k, pool.v)
        rows = self._decode_rows.get(B)
        if rows is None:
            qo, qr = _upload_i32([np.arange(B + 1, dtype=np.int32), np.arange(B, dtype=np.int32)], pool.device)
            rows = self._decode_rows[B] = (qo, qr)
        return _ForwardPlan.from_device(B, slot, pos, indptr, indices, lpl, rows[0], rows[1], new,
                                        plan.total_pages + n_new, groups=plan.groups)

    def _begin_steady_decode(self, seq_ids, ntoks) -> Optional["PagedCacheContext"]:
        """begin_forward of a steady decode step of a batch of up to ONE_PASS_BATCH
        sequences, in one pass over it:
        the batch the previous decode forward planned on the device, one token per
        sequence, each at the length that forward left it with the pages it had then,
        no shared page written, the pages it opens free in the pool and no zeroing owed.
        Same pages, tokens_used, plan and context as the general path, which takes every
        other case (eviction, OOM, copy-on-write, a changed batch) and is left untouched
        when this returns None."""
        ids, plan, lens = self._dev_plan
        B = len(ids)
        if (B > self.ONE_PASS_BATCH or self._pending_zero or len(seq_ids) != B or tuple(seq_ids) != ids
                or list(ntoks).count(1) != B):
            return None
        ps, pool, seqs = self.cfg.page_size, self.pool, self.seqs
        rc = pool.ref_count
        states, opening = [], 0
        for s, n in zip(ids, lens):
            st = seqs[s]
            k = n // ps  # the page of the new token
            if st.num_tokens != n:
                return None
            if n % ps:
                if st.n_pages != k + 1 or rc[st.bt[k]] > 1:
                    return None
            elif st.n_pages != k:
                return None
            else:
                opening += 1
            states.append(st)
        if opening > pool.num_free:
            return None
        newp = self._newp
        if newp is None or newp[0] != B:
            buf = np.full(B, -1, np.int32)
            newp = self._newp = (B, buf, buf.ctypes.data)
        new_page = newp[1]  # -1 everywhere between steps
        if opening:
            pages = pool.alloc(opening, zero=False)  # zeroed by the planner, as the general path does
            it = iter(pages)
            for b, (st, n) in enumerate(zip(states, lens)):
                if n % ps == 0:
                    pid = next(it)
                    st.extend([pid])
                    new_page[b] = pid
        tu = pool.tokens_used
        for st, n in zip(states, lens):
            pid = int(st.bt[n // ps])
            used = n % ps + 1
            if tu[pid] < used:
                tu[pid] = used
        try:
            new_plan = self._plan_on_device(B, plan, new_page, opening, new_page_ptr=newp[2])
        finally:
            if opening:
                new_page.fill(-1)  # the planner took the list by value
        ctx = PagedCacheContext.__new__(PagedCacheContext)
        ctx.cache, ctx.seq_ids, ctx.batch_size = self, list(ids), B
        ctx.new_token_counts, ctx.input_offsets = [1] * B, [0] * B
        ctx.start_positions = list(lens)
        ctx.seq_lens = [n + 1 for n in lens]
        ctx.max_kv_len = max(ctx.seq_lens)
        ctx._is_decode, ctx._iw, ctx._max_q, ctx._uniform_rows = True, 1, 1, True
        ctx.cow_pairs, ctx._plan, ctx._decode_launch = [], new_plan, None
        self._dev_plan = (ids, new_plan, ctx.seq_lens)
        return ctx

    PLAN_RING = 3  # device-planned decode steps write their plans into a ring of this many buffers

    def _plan_buffers(self, B, total_pages):
        """The next plan buffer of the ring for decode batches of B sequences, with room
        for total_pages block-table entries. Plans of consecutive steps are distinct
        buffers; the plan of a step is overwritten PLAN_RING steps later (the kernels of
        those steps run after it on the same stream), so a context's plan stays valid
        for its own forward and the next ones."""
        ring = self._plan_ring
        if ring is None or ring[0] != B or ring[1] < total_pages:
            cap = total_pages + 16 * B + 4096
            ring = self._plan_ring = [B, cap, [_GraphPlan(self.pool.device, B, cap) for _ in range(self.PLAN_RING)],
                                      0]
        i = ring[3] = (ring[3] + 1) % self.PLAN_RING
        return ring[2][i]

    def allocate_sequence(self, seq_id, token_ids=None, num_tokens=0):
        """kv_cache.py:707-722: radix match, pin, allocate the rest. The matched prefix
        is whole pages, or (share_partial_pages) whole pages and a partial page, which
        the sequence's first write then copies."""
        self._dev_plan = None
        tids = list(token_ids or [])
        total = len(tids) if tids else num_tokens
        plen, ppages = 0, []
        ps = self.cfg.page_size
        if self.tree and len(tids) >= (1 if self.tree.share_partial else ps):
            plen, ppages = self.tree.match(tids)
            for p in ppages:
                self.pool.add_ref(p)
            if ppages:
                self.tree.add_refs(tids[:plen])
        st = _PagedSeqState(seq_id, ppages, plen, tids)
        need = -(-total // ps) - len(ppages)  # = ceil((total - plen) / ps) when plen is whole pages
        if need > 0:
            st.extend(self._alloc(need))
        old = self.seqs.get(seq_id)
        if old is not None:  # a re-used id: its old table's device row is free again
            self._tables.release(old)
        self.seqs[seq_id] = st
        return plen

    def extend_sequence(self, seq_id, num_new=1):
        st = self.seqs[seq_id]
        need = math.ceil((st.num_tokens + num_new) / self.cfg.page_size)
        if need > st.n_pages:
            st.extend(self._alloc(need - st.n_pages, defer_zero=True))

    def begin_forward(self, seq_ids, ntoks, offsets=None):
        if offsets is None and self._dev_plan is not None:
            ctx = self._begin_steady_decode(seq_ids, ntoks)
            if ctx is not None:
                return ctx
        ps = self.cfg.page_size
        if any(n != 1 for n in ntoks):
            self._dev_plan = None
        # extend_sequence for every sequence (kv_cache.py:724-728, 760-768), in batch
        # order: one pool allocation for all of them when the free pages suffice (the
        # same pages, in the same order, as one allocation per sequence), else per
        # sequence, with eviction and the OOM error at the sequence that runs out
        grow = []
        for s, n in zip(seq_ids, ntoks):
            st = self.seqs[s]
            need = -(-(st.num_tokens + n) // ps) - st.n_pages
            if need > 0:
                grow.append((st, need))
        if len(grow) > 1 and self.pool.num_free >= sum(k for _, k in grow):
            ids = self._alloc(sum(k for _, k in grow), defer_zero=True, as_array=True)
            o = 0
            for st, k in grow:
                st.extend(ids[o:o + k])
                o += k
        else:
            for st, k in grow:
                st.extend(self._alloc(k, defer_zero=True))
        zero, self._pending_zero = self._pending_zero, []
        try:
            return PagedCacheContext(self, seq_ids, ntoks, offsets, zero_pages=zero)
        except RuntimeError:
            # the pages this call took stay with their sequences and are zeroed, as
            # allocation zeroes them (kv_cache.py:411), whatever stopped the forward
            if zero:
                self.pool.zero(zero)
            raise

    def end_forward(self, ctx):
        for b in range(ctx.batch_size):
            self.seqs[ctx.seq_ids[b]].num_tokens += ctx.new_token_counts[b]

    def release_sequence(self, seq_id):
        """kv_cache.py:739-751: cache full pages in the tree, unpin, release."""
        self._dev_plan = None
        st = self.seqs.get(seq_id)
        if st is None:
            return
        ps = self.cfg.page_size
        if self.tree and st.token_ids:
            if self.tree.share_partial:  # the full pages and the last, partial one
                n = min(st.num_tokens, len(st.token_ids), st.n_pages * ps)
                if n:
                    self.tree.insert(st.token_ids[:n], st.block_table[:-(-n // ps)])
            else:
                nf = min(st.num_tokens // ps, st.n_pages)
                if nf:
                    self.tree.insert(st.token_ids[:nf * ps], st.block_table[:nf])
            if st.prefix_len:
                self.tree.dec_refs(st.token_ids[:st.prefix_len])
        self.pool.release_many(st.bt[:st.n_pages])
        self._tables.release(st)
        del self.seqs[seq_id]

    def append_token_ids(self, seq_id, ids):
        if seq_id in self.seqs:
            self.seqs[seq_id].token_ids.extend(ids)

    def reset(self):
        for s in list(self.seqs):
            self.release_sequence(s)

    def _alloc(self, n, defer_zero=False, as_array=False):
        """kv_cache.py:760-768: pool, else LRU-evict from the tree and retry, else OOM.
        The pages as a list, or (as_array) as an int64 array."""
        got = self.pool.alloc_ids(n, zero=not defer_zero)
        if got is None and self.tree and self.tree.evict_lru(n) > 0:
            got = self.pool.alloc_ids(n, zero=not defer_zero)
        if got is None:
            raise RuntimeError(f"KV OOM: need {n}, free {self.pool.num_free}")
        pages, ids = got
        if defer_zero:
            self._pending_zero.extend(pages)
        return ids if as_array else pages

    @property
    def stats(self):
        return {"backend": "paged",
                "active_seqs": len(self.seqs),
                "pages_used": self.cfg.max_pages - 1 - self.pool.num_free,
                "pages_free": self.pool.num_free,
                "util": f"{self.pool.utilization:.1%}",
                "radix": self.tree.cached_pages if self.tree else 0}


# --------------------------------------------------------------------------------------
# contiguous backend: the same kernels with one Smax-token "page" per slot
# --------------------------------------------------------------------------------------


class _ContigSeqState:
    __slots__ = ("seq_id", "slot", "num_tokens", "token_ids")

    def __init__(self, seq_id, slot):
        self.seq_id = seq_id
        self.slot = slot
        self.num_tokens = 0
        self.token_ids: List[int] = []


class ContiguousCacheContext(CacheContext):
    """kv_cache.py:247-325. The [L, Bmax, Smax, Hkv, D] pool is a paged pool whose pages
    are whole slots (page_size = Smax) with an identity block table, so the append
    and attention kernels are the paged ones. Rows are addressed by the sequence's
    slot (the reference indexes by batch row; identical while slots are 0..B-1)."""

    def __init__(self, cache: "ContiguousKVCache", seq_ids, new_token_counts, input_offsets):
        self.cache = cache
        self.seq_ids = list(seq_ids)
        self.new_token_counts = list(new_token_counts)
        self.input_offsets = list(input_offsets) if input_offsets else [0] * len(seq_ids)
        self.batch_size = B = len(seq_ids)
        cfg = cache.cfg
        Smax = cfg.max_seq_len
        self.slots = [cache.states[s].slot for s in self.seq_ids]
        self.start_positions = [cache.states[s].num_tokens for s in self.seq_ids]
        self.seq_lens = [self.start_positions[i] + self.new_token_counts[i] for i in range(B)]
        self.max_kv_len = max(self.seq_lens) if self.seq_lens else 0
        self._is_decode = B > 0 and all(n == 1 for n in self.new_token_counts)
        self._iw = max(o + n for o, n in zip(self.input_offsets, self.new_token_counts)) if B else 1
        iw = self._iw
        slot = np.full((B, iw), -1, np.int32)
        for b in range(B):
            o, n, s0 = self.input_offsets[b], self.new_token_counts[b], self.start_positions[b]
            if n > 0:
                slot[b, o:o + n] = self.slots[b] * Smax + np.arange(s0, s0 + n)
        indptr = np.arange(B + 1, dtype=np.int64)
        indices = np.asarray(self.slots or [0], np.int32)
        lpl = np.asarray(self.seq_lens or [0], np.int64)
        # a zero-length sequence gets no page
        if B and any(L == 0 for L in self.seq_lens):
            npg = np.asarray([1 if L > 0 else 0 for L in self.seq_lens])
            indptr = np.zeros(B + 1, np.int64)
            np.cumsum(npg, out=indptr[1:])
            indices = np.asarray([s for s, L in zip(self.slots, self.seq_lens) if L > 0] or [0], np.int32)
        pos, q_rows, qo = _ragged_layout(self.start_positions, self.new_token_counts, self.input_offsets, iw)
        self._max_q = max(self.new_token_counts) if B else 0
        self._uniform_rows = int(qo[-1]) == B * iw
        self._plan = _ForwardPlan(cache.device, B, iw, slot.reshape(-1), pos, indptr, indices, lpl, qo,
                                  q_rows, np.zeros(0, np.int32), np.zeros(0, np.int32))

    def get_position_ids(self, S: int) -> torch.Tensor:
        return _get_positions(self._plan, self.batch_size, self._iw, S)

    def get_start_pos(self, idx: int = 0) -> int:
        return self.start_positions[idx]

    def attend(self, layer_idx, q, k_new, v_new, n_heads, n_kv_heads):
        cache, plan = self.cache, self._plan
        k_layer, v_layer = cache.paged_view(layer_idx)
        B, S = q.shape[0], q.shape[1]
        if not (self._is_decode and S == 1):
            # the write and the attention in one launch (a sequence's slot is its one page)
            uniform = self._uniform_rows and S == self._iw
            o = cache.kernels._paged_prefill_append_layer(
                q.reshape(B * S, q.shape[2], q.shape[3]), plan.qo_indptr, plan.total_q, self._max_q, k_new, v_new,
                k_layer, v_layer, plan.indptr, plan.indices, plan.lpl, cache.workspace,
                q_rows=None if uniform else plan.rows_for(S), grid_width=0 if uniform else S)
            if o is not None:
                return o.view(B, S, -1)
        cache.kernels.append_kv(k_new, v_new, plan.slots_for(S), k_layer, v_layer)
        return self._attend_written(q, k_layer, v_layer)

    def attend_rope(self, layer_idx, q, k_new, v_new, cos, sin, n_heads, n_kv_heads):
        """attend() with the position part of the model's attention forward fused into
        the cache write (models.py:96-105): q and k_new rotated at this forward's
        positions with the model's cos/sin tables, the rotated k and v written into
        the sequence slots of `layer_idx` in one launch. Same result as attend() on
        the eagerly rotated q and k_new, bit for bit."""
        cache, plan = self.cache, self._plan
        if self.max_kv_len > cos.shape[0]:
            raise IndexError(f"position {self.max_kv_len - 1} is outside the rope tables ({cos.shape[0]} rows)")
        S = q.shape[1]
        k_layer, v_layer = cache.paged_view(layer_idx)
        q_rot = cache.kernels.rope_append(q, k_new, v_new, plan.pos_for(S), plan.slots_for(S), cos, sin,
                                          k_layer, v_layer)
        return self._attend_written(q_rot, k_layer, v_layer)

    def _attend_written(self, q, k_layer, v_layer):
        """Attention of the forward's rows over the slots (K/V already written)."""
        cache, plan = self.cache, self._plan
        kern = cache.kernels
        B, S = q.shape[0], q.shape[1]
        if self._is_decode and S == 1:
            out = kern.paged_decode(q[:, 0], k_layer, v_layer, plan.indptr, plan.indices, plan.lpl,
                                    plan.total_pages, workspace=cache.workspace)
            return out.reshape(B, 1, -1)
        Hq, D = q.shape[2], q.shape[3]
        q_grid = q.reshape(B * S, Hq, D)
        if self._uniform_rows and S == self._iw:  # every grid row is a token: the ragged rows themselves
            o = kern.paged_prefill(q_grid, plan.qo_indptr, plan.total_q, self._max_q, k_layer, v_layer,
                                   plan.indptr, plan.indices, plan.lpl, workspace=cache.workspace)
        else:  # padded or ragged: the kernel reads and writes the grid rows (pad rows zero)
            o = kern.paged_prefill(q_grid, plan.qo_indptr, plan.total_q, self._max_q, k_layer, v_layer,
                                   plan.indptr, plan.indices, plan.lpl, workspace=cache.workspace,
                                   q_rows=plan.rows_for(S), grid_width=S)
        return o.view(B, S, Hq * D)


class ContiguousKVCache(KVCacheManager):
    """Pre-allocated [L, Bmax, Smax, Hkv, D] cache, no paging or prefix caching
    (kv_cache.py:328-379)."""

    def __init__(self, cfg: KVCacheConfig, kernels=None):
        self.cfg = cfg
        self.kernels = kernels or _default_kernels()
        _check_head_dim(cfg, self.kernels)
        self.device = torch.device(cfg.device) if cfg.device is not None else torch.device("cpu")
        shape = (cfg.num_layers, cfg.max_batch_size, cfg.max_seq_len, cfg.num_kv_heads, cfg.head_dim)
        self.k = torch.zeros(shape, dtype=cfg.dtype, device=self.device)
        self.v = torch.zeros(shape, dtype=cfg.dtype, device=self.device)
        self.states: Dict[str, _ContigSeqState] = {}
        self._slot = 0
        self.workspace = self.kernels.Workspace(self.device, 16 << 20)

    def paged_view(self, layer_idx):
        return self.k[layer_idx], self.v[layer_idx]

    def allocate_sequence(self, seq_id, token_ids=None, num_tokens=0):
        s = self._slot
        self._slot += 1
        assert s < self.cfg.max_batch_size, "Exceeded max_batch_size"
        (ids,) = _upload_i32([np.asarray([s], np.int32)], self.device)
        self.kernels.zero_pages(self.k, self.v, ids)
        st = _ContigSeqState(seq_id, s)
        if token_ids:
            st.token_ids = list(token_ids)
        self.states[seq_id] = st
        return 0

    def extend_sequence(self, seq_id, num_new=1):
        st = self.states[seq_id]
        assert st.num_tokens + num_new <= self.cfg.max_seq_len

    def begin_forward(self, seq_ids, ntoks, offsets=None):
        for sid, n in zip(seq_ids, ntoks):
            self.extend_sequence(sid, n)
        return ContiguousCacheContext(self, seq_ids, ntoks, offsets)

    def end_forward(self, ctx):
        for b in range(ctx.batch_size):
            self.states[ctx.seq_ids[b]].num_tokens += ctx.new_token_counts[b]

    def release_sequence(self, seq_id):
        if seq_id in self.states:
            del self.states[seq_id]
            if not self.states:
                self._slot = 0

    def append_token_ids(self, seq_id, ids):
        if seq_id in self.states:
            self.states[seq_id].token_ids.extend(ids)

    def reset(self):
        for s in list(self.states):
            self.release_sequence(s)

    @property
    def stats(self):
        return {"backend": "contiguous",
                "active_seqs": len(self.states),
                "slots": f"{self._slot}/{self.cfg.max_batch_size}",
                "max_seq": self.cfg.max_seq_len}


def create_cache_manager(hf_config, parallel_config, device, dtype, model_config,
                         max_batch_size=4) -> KVCacheManager:
    """kv_cache.py:780-805: backend from model_config.kv_backend (auto -> paged)."""
    dev = torch.device(device)
    if dev.type == "cuda":
        torch.cuda.synchronize(dev)
        torch.cuda.empty_cache()
    backend = getattr(model_config, "kv_backend", "auto")
    kv_cfg = KVCacheConfig.from_hf_config(
        hf_config, parallel_config=parallel_config, device=dev,
        page_size=getattr(model_config, "page_size", 16),
        max_pages=getattr(model_config, "max_kv_pages", 0),
        max_batch_size=max_batch_size,
        max_seq_len=getattr(model_config, "max_seq_len", 4096),
        memory_fraction=getattr(model_config, "kv_memory_fraction", 0.30),
        dtype=dtype,
        enable_prefix_caching=getattr(model_config, "enable_prefix_caching", True),
        share_partial_pages=getattr(model_config, "share_partial_pages", True),
        backend=backend,
    )
    if kv_cfg.backend == "paged":
        return PagedKVCache(kv_cfg)
    return ContiguousKVCache(kv_cfg)


# the reference's class names, for callers that import them directly
FlashInferPagedKVCache = PagedKVCache
FlashInferCacheContext = PagedCacheContext


def attention_forward(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, layer_idx: int, n_heads: int,
                      n_kv_heads: int, cos: torch.Tensor, sin: torch.Tensor, cache_ctx: CacheContext) -> torch.Tensor:
    """Drop-in for the model's _attention_forward (models.py:86-105), same arguments
    and result: positions from the context, rotary embedding of q and k_new with the
    model's cos/sin tables, the cache write and attention, with the rotation and the
    write in one kernel launch (the context's attend_rope)."""
    return cache_ctx.attend_rope(layer_idx, q, k_new, v_new, cos, sin, n_heads, n_kv_heads)


# --------------------------------------------------------------------------------------
# decode step replayed from HIP graphs
# --------------------------------------------------------------------------------------


class _GraphPlan:
    """One static set of decode-plan tensors (indices with room for growth)."""

    def __init__(self, device, batch, capacity):
        sizes = [batch + 1, capacity, batch, batch, batch, batch]
        self.buf = torch.zeros(sum(sizes), dtype=torch.int32, device=device)
        (self.indptr, self.indices, self.lpl, self.slot, self.pos, self.new_pages) = self.buf.split(sizes)
        self.batch, self.iw = batch, 1
        self.capacity = capacity
        self.groups = None
        base, o = self.buf.data_ptr(), 0
        self.ptrs = []
        for n in sizes:
            self.ptrs.append(base + 4 * o)
            o += n


class _GraphDecodeContext(CacheContext):
    """The context a captured decode step's attend calls run on: its plan tensors
    are static (the graph's), its host attributes are refreshed every step.

    It refers to its graph weakly: the graph holds its contexts, and a strong
    reference back would make every DecodeGraph a reference cycle, destroyed only
    by Python's cyclic collector at an arbitrary later time, possibly while another
    graph is being captured, when the HIP calls its destruction makes (graph
    teardown, the pinned page-list buffers' stream events) are not allowed."""

    def __init__(self, graph: "DecodeGraph", plan: _GraphPlan, launch):
        self._graph, self._plan_t, self._launch = weakref.ref(graph), plan, launch
        self.seq_ids = list(graph.seq_ids)
        self.batch_size = len(self.seq_ids)
        self.new_token_counts = [1] * self.batch_size
        self.input_offsets = [0] * self.batch_size
        self.seq_lens: List[int] = []
        self.start_positions: List[int] = []

    def get_position_ids(self, S: int) -> torch.Tensor:
        pos = self._plan_t.pos.view(self.batch_size, 1).long()
        return pos if S == 1 else torch.cat([pos, pos.new_zeros(self.batch_size, S - 1)], 1)

    def get_start_pos(self, idx: int = 0) -> int:
        return self.start_positions[idx]

    def attend(self, layer_idx, q, k_new, v_new, n_heads, n_kv_heads):
        B = q.shape[0]
        return self._launch(layer_idx, q[:, 0], k_new, v_new).reshape(B, 1, -1)

    def attend_rope(self, layer_idx, q, k_new, v_new, cos, sin, n_heads, n_kv_heads):
        B = q.shape[0]
        # replays rotate at positions the captured tables must hold (step() checks)
        g = self._graph()
        g.rope_rows = cos.shape[0] if g.rope_rows is None else min(g.rope_rows, cos.shape[0])
        if self.seq_lens and max(self.seq_lens) > cos.shape[0]:
            raise IndexError(f"position {max(self.seq_lens) - 1} is outside the rope tables ({cos.shape[0]} rows)")
        return self._launch(layer_idx, q[:, 0], k_new, v_new, rope=(cos, sin, self._plan_t.pos)).reshape(B, 1, -1)


class DecodeGraph:
    """Steady decode steps of a fixed batch replayed from HIP graphs.

    A step is: a copy of this step's opened-page list in (from pinned host memory),
    the device planner (the next block tables, slots and positions from the previous
    step's, zeroing the opened pages), then `forward(ctx)`, the caller's attend
    calls for every layer (a model forward) on its static input tensors. Two graphs
    alternate between two static plan buffers. Host work per step: the cache
    bookkeeping of the step (pages opened, tokens_used), the page list, one replay.

    forward(ctx) is called once per graph at capture; its return value (static
    tensors) is what step() returns after each replay. The batch must not write a
    shared page (copy-on-write goes through the eager path) and its chunking must
    fit one resident round (the decode's launch is captured once); capacity bounds
    the block-table growth: after max_steps steps, build a new DecodeGraph."""

    def __init__(self, cache: "PagedKVCache", seq_ids: Sequence[str], forward, max_steps: int = 4096):
        kern = cache.kernels
        if not hasattr(kern, "_decode_plan_step_device"):
            raise RuntimeError("DecodeGraph needs the HIP kernels")
        self.cache, self.seq_ids, self.forward = cache, list(seq_ids), forward
        self.rope_rows = None  # rows of the rope tables the captured forward rotates with
        B, ps, pool, cfg = len(self.seq_ids), cache.cfg.page_size, cache.pool, cache.cfg
        self._zero_pending()
        if not 1 <= B <= 512:
            raise ValueError("DecodeGraph: 1..512 sequences")
        self.states = [cache.seqs[s] for s in self.seq_ids]
        lens = np.fromiter((st.num_tokens for st in self.states), np.int64, B)
        if (lens < 1).any():
            raise ValueError("DecodeGraph: every sequence needs at least one cached token")
        npg = (lens + ps - 1) // ps
        have = np.fromiter((st.n_pages for st in self.states), np.int64, B)
        if (have < npg).any():
            raise ValueError("DecodeGraph: a sequence has fewer pages than tokens")
        indptr = np.zeros(B + 1, np.int64)
        np.cumsum(npg, out=indptr[1:])
        indices = np.concatenate([st.bt[:k] for st, k in zip(self.states, npg.tolist())])
        lpl = lens - (npg - 1) * ps
        self.max_steps = int(max_steps)
        cap = int(indptr[-1]) + B * ((self.max_steps + ps - 1) // ps + 1)
        dev = pool.device
        self.plans = [_GraphPlan(dev, B, cap), _GraphPlan(dev, B, cap)]
        (d_ip, d_ix, d_lpl) = _upload_i32([indptr, indices, lpl], dev)
        p0 = self.plans[0]
        p0.indptr.copy_(d_ip)
        p0.indices[:indices.size].copy_(d_ix)
        p0.lpl.copy_(d_lpl)
        groups = cache._prefix_groups(self.states, npg + 1)
        if groups is not None:
            g = kern.DecodeGroups(B, groups[0], groups[1], dev)
            for p in self.plans:
                p.groups = g
        self.new_host = [torch.zeros(B, dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self.new_np = [t.numpy() for t in self.new_host]
        self.new_dev = [torch.zeros(B, dtype=torch.int32, device=dev) for _ in range(2)]
        self.done = [torch.cuda.Event() for _ in range(2)]
        self.dev_index = dev.index if dev.index is not None else torch.cuda.current_device()
        self.used = [False, False]
        L, P = cfg.num_layers, cfg.max_pages
        self.pool_args = (pool.k.data_ptr(), pool.v.data_ptr(), L, P, cfg.num_kv_heads, cfg.head_dim,
                          kern.dtype_code(pool.k.dtype))
        # The launch is captured once, so it is sized for the pool (P pages) rather than
        # this step's page count; the kernel derives its chunk length from the lengths.
        launches = [kern.DecodeLaunch(pool.k, pool.v, p.slot, p.indptr, p.indices, p.lpl, P, cfg.num_qo_heads,
                                      workspace=cache.workspace, groups=p.groups) for p in self.plans]
        self.ctxs = [_GraphDecodeContext(self, self.plans[(i + 1) % 2], launches[(i + 1) % 2]) for i in range(2)]
        self.graphs, self.outputs = [], []
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        torch.cuda.synchronize(dev)
        # No object may be destroyed by the cyclic collector while a graph is being
        # captured: unreachable cycles holding graphs, pinned buffers or events (an
        # earlier DecodeGraph of the caller's, say) are collected now, and the
        # collector stays off until both captures have ended.
        gc.collect()
        gc_was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.stream(side):
                for i in range(2):  # graph i: plan i -> plan 1-i, then the forward on plan 1-i
                    src, dst = self.plans[i], self.plans[1 - i]
                    g = torch.cuda.CUDAGraph()
                    with torch.cuda.graph(g, stream=side):
                        # this step's page list: pinned host memory -> device (a copy node of
                        # the graph; measured faster than the planner reading host memory)
                        self.new_dev[i].copy_(self.new_host[i], non_blocking=True)
                        kern._decode_plan_step_device(src.indptr, src.indices, src.lpl, self.new_dev[i], B, ps,
                                                      dst, self.pool_args)
                        out = forward(self.ctxs[i])
                    self.graphs.append(g)
                    self.outputs.append(out)
        finally:
            if gc_was_enabled:
                gc.enable()
        torch.cuda.current_stream(dev).wait_stream(side)
        self.parity = 0
        self.steps = 0
        cache._dev_plan = None

    def _zero_pending(self) -> None:
        """Zero, now, the pages whose zero-on-alloc the cache still owes (those that
        extend_sequence took, kv_cache.py:411, or that a failed forward left): the
        replayed steps write into them and never run the eager forward that would
        zero them, and that eager forward, run after graph steps, would zero them
        again after tokens were written into them."""
        cache = self.cache
        if cache._pending_zero:
            pending, cache._pending_zero = cache._pending_zero, []
            cache.pool.zero(pending)

    def step(self):
        """One decode step of the batch: bookkeeping, then the graph replay."""
        cache, pool, ps = self.cache, self.cache.pool, self.cache.cfg.page_size
        if self.steps >= self.max_steps:
            raise RuntimeError("DecodeGraph: block-table capacity used up; build a new DecodeGraph")
        i = self.parity
        if self.used[i]:
            self.done[i].synchronize()  # the page list of two steps ago has been copied in
        B = len(self.states)
        start = np.fromiter((st.num_tokens for st in self.states), np.int64, B)
        if self.rope_rows is not None and int(start.max()) >= self.rope_rows:
            raise IndexError(f"position {int(start.max())} is outside the rope tables ({self.rope_rows} rows)")
        # checks first: a page the step writes that the sequence already has must not
        # be shared (a page allocated here never is)
        npg = start // ps + 1
        for b, st in enumerate(self.states):
            if st.n_pages >= npg[b] and pool.ref_count[st.bt[npg[b] - 1]] > 1:
                raise RuntimeError("DecodeGraph: a shared page would be written; use the eager path")
        self._zero_pending()
        opens = start % ps == 0
        new_np = self.new_np[i]
        new_np[:] = -1
        taken: List[int] = []
        try:
            for b in np.flatnonzero(opens).tolist():
                st = self.states[b]
                need = int(start[b]) // ps + 1
                if st.n_pages < need:  # zeroed by the graph's planner, not by a launch of its own
                    k = need - st.n_pages
                    pages = cache._alloc(k, defer_zero=True)
                    del cache._pending_zero[-k:]
                    taken.extend(pages)
                    st.extend(pages)
                # (a page the sequence already had has been zeroed: at its allocation,
                # or by _zero_pending above when its zeroing was deferred)
                new_np[b] = st.bt[need - 1]
        except RuntimeError:
            cache._pending_zero.extend(taken)  # the next forward zeroes them, as allocation would
            raise
        pids = np.fromiter((st.bt[npg[b] - 1] for b, st in enumerate(self.states)), np.int64, B)
        sl = start % ps
        pool.tokens_used[pids] = np.maximum(pool.tokens_used[pids], sl + 1)
        ctx = self.ctxs[i]
        ctx.start_positions = start.tolist()
        ctx.seq_lens = (start + 1).tolist()
        self.graphs[i].replay()
        self.done[i].record(_current_stream(self.dev_index))
        self.used[i] = True
        for st in self.states:
            st.num_tokens += 1
        self.parity ^= 1
        self.steps += 1
        return self.outputs[i]
