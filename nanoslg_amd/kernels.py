"""Tensor-level wrappers over the C ABI of libnslg_kv.so.

Each function validates shapes, dtypes, devices and strides on the host, then
passes raw device pointers and the current HIP stream to the library. Nothing
here computes on the CPU: a missing library or a non-HIP tensor raises.
"""
from __future__ import annotations

import itertools
import math
from typing import Dict, Optional, Tuple

import torch

from . import _lib

_DTYPE_CODE = {torch.float16: _lib.NSLG_F16, torch.bfloat16: _lib.NSLG_BF16, torch.float32: _lib.NSLG_F32}

# Pool dtypes nslg_paged_decode_grouped serves (its work units are 16-bit MFMA tiles);
# decode batches of other pools are decoded per sequence.
GROUPED_DECODE_DTYPES = (torch.float16, torch.bfloat16)
# head dims each pool dtype supports on every entry point a cache uses: decode, RoPE
# append and prefill take 64, 128 and 256 (16-bit pools on the MFMA kernels, fp32
# pools on the VALU attention kernel)
HEAD_DIMS = {torch.float16: (64, 128, 256), torch.bfloat16: (64, 128, 256), torch.float32: (64, 128, 256)}


def dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise TypeError(f"unsupported KV dtype {dt}") from None


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)

# tags of the chunk layouts decode launchers record in their workspaces (one per
# recorded plan; never reused within the process)
_LAYOUT_TAGS = itertools.count(1)


def _stream(t: torch.Tensor) -> int:
    """The current HIP stream of t's device, as an integer handle."""
    if _RAW_STREAM is not None:
        return _RAW_STREAM(t.get_device())
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_gpu(*ts: torch.Tensor) -> None:
    dev = None
    for t in ts:
        if not t.is_cuda:
            raise ValueError("HIP kernels need device tensors (got a CPU tensor); there is no CPU path")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")


def _i32(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.int32 or not t.is_contiguous():
        raise ValueError(f"{name} must be a contiguous int32 tensor (got {t.dtype})")
    return t


def _rows(x: torch.Tensor, name: str) -> Tuple[int, int, int]:
    """(num_rows, row_stride, heads) for a [..., H, D] tensor with a dense [H, D] block
    whose leading dims collapse to a single row stride."""
    if x.dim() < 2:
        raise ValueError(f"{name} must have at least 2 dims")
    H, D = x.shape[-2], x.shape[-1]
    try:
        v = x.view(-1, H, D)
    except RuntimeError:
        raise ValueError(f"{name}: leading dims do not collapse to one row stride") from None
    if v.stride(2) != 1 or (H > 1 and v.stride(1) != D):
        raise ValueError(f"{name}: the trailing [H, D] block must be contiguous")
    n = v.shape[0]
    return n, (v.stride(0) if n > 1 else H * D), H


def append_kv(k_new: torch.Tensor, v_new: torch.Tensor, slot_mapping: torch.Tensor,
              k_pool: torch.Tensor, v_pool: torch.Tensor) -> None:
    """Scatter rows of k_new/v_new ([..., Hkv, D]) into one layer of the pool.

    slot_mapping: int32 with one entry per row (page*page_size + slot; <0 = skip).
    k_pool/v_pool: one layer, [P, page_size, Hkv, D] (or any contiguous [..., Hkv, D]).
    """
    _require_gpu(k_new, v_new, slot_mapping, k_pool, v_pool)
    _i32(slot_mapping, "slot_mapping")
    if k_new.dtype != k_pool.dtype or v_new.dtype != v_pool.dtype or k_pool.dtype != v_pool.dtype:
        raise TypeError("append_kv: k/v dtypes must match the pool dtype")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("append_kv: pool layer must be contiguous")
    Hkv, D = k_pool.shape[-2], k_pool.shape[-1]
    if tuple(k_new.shape[-2:]) != (Hkv, D) or tuple(v_new.shape[-2:]) != (Hkv, D):
        raise ValueError("append_kv: k_new/v_new trailing dims must be [Hkv, D] of the pool")
    nk, ks, _ = _rows(k_new, "k_new")
    nv, vs, _ = _rows(v_new, "v_new")
    T = slot_mapping.numel()
    if nk != T or nv != T:
        raise ValueError(f"append_kv: {T} slots for {nk} k rows / {nv} v rows")
    slots = k_pool.numel() // (Hkv * D)
    rc = _lib.fast().append_kv(k_new.data_ptr(), v_new.data_ptr(), ks, vs, slot_mapping.data_ptr(), T,
                               k_pool.data_ptr(), v_pool.data_ptr(), slots, Hkv, D, dtype_code(k_pool.dtype),
                               _stream(k_pool))
    _lib.check(rc, "nslg_append_kv")


def _append_kv_layer(k_new: torch.Tensor, v_new: torch.Tensor, slot_mapping: torch.Tensor,
                     k_layer: torch.Tensor, v_layer: torch.Tensor) -> None:
    """append_kv for the cache manager: its pool layer (contiguous [P, page_size, Hkv,
    D], K and V alike) and slot mapping (int32 on the pool's device) are taken as they
    are; the caller's k_new and v_new get append_kv's checks (a tensor that fails one
    goes through append_kv, which raises its error)."""
    dev, dt = k_layer.get_device(), k_layer.dtype
    Hkv, D = k_layer.shape[2], k_layer.shape[3]
    if (k_new.get_device() != dev or v_new.get_device() != dev or k_new.dtype != dt or v_new.dtype != dt
            or k_new.dim() < 2 or v_new.dim() < 2 or k_new.shape[-1] != D or v_new.shape[-1] != D
            or k_new.shape[-2] != Hkv or v_new.shape[-2] != Hkv):
        return append_kv(k_new, v_new, slot_mapping, k_layer, v_layer)
    row = Hkv * D
    if k_new.is_contiguous() and v_new.is_contiguous():  # the model's own [B, S, Hkv, D] rows
        nk, ks, nv, vs = k_new.numel() // row, row, v_new.numel() // row, row
    else:
        nk, ks, _ = _rows(k_new, "k_new")
        nv, vs, _ = _rows(v_new, "v_new")
    T = slot_mapping.numel()
    if nk != T or nv != T:
        raise ValueError(f"append_kv: {T} slots for {nk} k rows / {nv} v rows")
    rc = _lib.fast().append_kv(k_new.data_ptr(), v_new.data_ptr(), ks, vs, slot_mapping.data_ptr(), T,
                               k_layer.data_ptr(), v_layer.data_ptr(), k_layer.shape[0] * k_layer.shape[1], Hkv, D,
                               _DTYPE_CODE[dt], _stream(k_layer))
    _lib.check(rc, "nslg_append_kv")


def _rope_tables(cos: torch.Tensor, sin: torch.Tensor, D: int):
    """fp32 [R, >=D] tables with unit inner stride and a common row stride (a
    16-bit table is widened exactly; the kernel rounds it back)."""
    if cos.dtype != torch.float32:
        cos = cos.float()
    if sin.dtype != torch.float32:
        sin = sin.float()
    if cos.dim() != 2 or cos.shape != sin.shape or cos.shape[1] < D:
        raise ValueError(f"rope tables must be [rows, >= {D}] and of one shape")
    if cos.stride(1) != 1 or cos.stride(0) != sin.stride(0) or sin.stride(1) != 1:
        cos, sin = cos.contiguous(), sin.contiguous()
    return cos, sin


def rope_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, positions: torch.Tensor,
                slot_mapping: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, k_pool: torch.Tensor,
                v_pool: torch.Tensor, q_out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Rotary position embedding of q and k_new at `positions`, and the append of the
    rotated k and of v_new into one pool layer at `slot_mapping`, in one launch.

    q [..., Hq, D] rows; k_new/v_new [..., Hkv, D] with as many rows; positions and
    slot_mapping int32, one per row (slot < 0: padding, not written); cos/sin the
    model's [max_positions, D] tables. Returns q rotated, shaped like q (q_out, or a
    new tensor; q_out may be q). A position outside the tables raises IndexError."""
    _require_gpu(q, k_new, v_new, positions, slot_mapping, cos, sin, k_pool, v_pool)
    _i32(positions, "positions")
    _i32(slot_mapping, "slot_mapping")
    if not (q.dtype == k_new.dtype == v_new.dtype == k_pool.dtype == v_pool.dtype):
        raise TypeError("rope_append: q, k/v and the pool must share one dtype")
    if not (k_pool.is_contiguous() and v_pool.is_contiguous()) or k_pool.shape != v_pool.shape:
        raise ValueError("rope_append: pool layers must be contiguous and of one shape")
    Hkv, D = k_pool.shape[-2], k_pool.shape[-1]
    nq, qs, Hq = _rows(q, "q")
    nk, ks, hk = _rows(k_new, "k_new")
    nv, vs, hv = _rows(v_new, "v_new")
    if q.shape[-1] != D or tuple(k_new.shape[-2:]) != (Hkv, D) or tuple(v_new.shape[-2:]) != (Hkv, D):
        raise ValueError("rope_append: trailing dims must be [Hq, D] / [Hkv, D] of the pool")
    T = positions.numel()
    if nq != T or nk != T or nv != T or slot_mapping.numel() != T:
        raise ValueError(f"rope_append: {T} positions for {nq} q / {nk} k / {nv} v rows, "
                         f"{slot_mapping.numel()} slots")
    cos, sin = _rope_tables(cos, sin, D)
    if q_out is None:
        q_out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    if q_out.shape != q.shape or q_out.dtype != q.dtype:
        raise ValueError("rope_append: q_out must be shaped like q")
    no, qos, _ = _rows(q_out, "q_out")
    rc = _lib.load().nslg_rope_append(q.data_ptr(), qs, q_out.data_ptr(), qos, k_new.data_ptr(), ks,
                                      v_new.data_ptr(), vs, positions.data_ptr(), slot_mapping.data_ptr(), T,
                                      cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], Hq, Hkv, D,
                                      k_pool.data_ptr(), v_pool.data_ptr(), k_pool.numel() // (Hkv * D),
                                      dtype_code(q.dtype), _stream(q))
    _lib.check(rc, "nslg_rope_append")
    return q_out


def _pool_geom(k_pool: torch.Tensor, v_pool: torch.Tensor):
    if k_pool.shape != v_pool.shape or k_pool.dtype != v_pool.dtype:
        raise ValueError("k/v pools must have the same shape and dtype")
    if k_pool.dim() != 5 or not (k_pool.is_contiguous() and v_pool.is_contiguous()):
        raise ValueError("pools must be contiguous [L, P, page_size, Hkv, D]")
    return k_pool.shape


def zero_pages(k_pool: torch.Tensor, v_pool: torch.Tensor, page_ids: torch.Tensor) -> None:
    """Zero pages `page_ids` of a [L, P, ps, Hkv, D] pool pair, all layers."""
    _require_gpu(k_pool, v_pool, page_ids)
    _i32(page_ids, "page_ids")
    L, P, ps, Hkv, D = _pool_geom(k_pool, v_pool)
    rc = _lib.fast().zero_pages(k_pool.data_ptr(), v_pool.data_ptr(), L, P, ps, Hkv, D, dtype_code(k_pool.dtype),
                                page_ids.data_ptr(), page_ids.numel(), _stream(k_pool))
    _lib.check(rc, "nslg_zero_pages")


def copy_pages(k_pool: torch.Tensor, v_pool: torch.Tensor, src_ids: torch.Tensor,
               dst_ids: torch.Tensor) -> None:
    """pool[:, dst] <- pool[:, src] for K and V, all layers and slots."""
    _require_gpu(k_pool, v_pool, src_ids, dst_ids)
    _i32(src_ids, "src_ids")
    _i32(dst_ids, "dst_ids")
    if src_ids.numel() != dst_ids.numel():
        raise ValueError("copy_pages: src/dst length mismatch")
    L, P, ps, Hkv, D = _pool_geom(k_pool, v_pool)
    rc = _lib.fast().copy_pages(k_pool.data_ptr(), v_pool.data_ptr(), L, P, ps, Hkv, D, dtype_code(k_pool.dtype),
                                src_ids.data_ptr(), dst_ids.data_ptr(), src_ids.numel(), _stream(k_pool))
    _lib.check(rc, "nslg_copy_pages")


def _layer_geom(k_layer: torch.Tensor, v_layer: torch.Tensor):
    if k_layer.dim() != 4 or k_layer.shape != v_layer.shape or k_layer.dtype != v_layer.dtype:
        raise ValueError("pool layer must be [P, page_size, Hkv, D] for both K and V")
    if not (k_layer.is_contiguous() and v_layer.is_contiguous()):
        raise ValueError("pool layer must be contiguous")
    return k_layer.shape


def gather_kv(k_layer: torch.Tensor, v_layer: torch.Tensor, kv_indptr: torch.Tensor,
              kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, max_len: int
              ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Paged -> contiguous [B, max_len, Hkv, D] K and V (zeros past each length)."""
    _require_gpu(k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        _i32(t, n)
    P, ps, Hkv, D = _layer_geom(k_layer, v_layer)
    B = kv_indptr.numel() - 1
    k_out = torch.empty((B, max_len, Hkv, D), dtype=k_layer.dtype, device=k_layer.device)
    v_out = torch.empty_like(k_out)
    rc = _lib.load().nslg_gather_kv(k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
                                    kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B, max_len, Hkv, D,
                                    dtype_code(k_layer.dtype), k_out.data_ptr(), v_out.data_ptr(),
                                    _stream(k_layer))
    _lib.check(rc, "nslg_gather_kv")
    return k_out, v_out


class Workspace:
    """Caller-owned device scratch for the attention kernels; grows on demand.
    One call at a time may use a workspace (zero-filled when allocated)."""

    def __init__(self, device: torch.device, nbytes: int = 0):
        self.device = torch.device(device)
        self.buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=self.device)

    def get(self, nbytes: int) -> torch.Tensor:
        if self.buf.numel() < nbytes:
            self.buf = torch.zeros(int(nbytes * 1.25) + 256, dtype=torch.uint8, device=self.device)
        return self.buf


class DecodeGroups:
    """Prefix groups of a decode batch: sequences whose first pages are the same pages.

    members: list of lists of batch indices (one list per group, at most 16 / G each),
    prefix_pages: pages each group shares. Builds the device array seq_group_slot
    (16 * group + member per sequence, -1 outside groups) and the host tables the
    grouped decode entry point takes."""

    MAX_GROUPS = 32

    def __init__(self, batch: int, members, prefix_pages, device, seq_group_slot: Optional[torch.Tensor] = None):
        import numpy as np
        if not 1 <= len(members) <= self.MAX_GROUPS or len(prefix_pages) != len(members):
            raise ValueError(f"DecodeGroups: 1..{self.MAX_GROUPS} groups, one prefix length each")
        self.num_groups = len(members)
        self.members = [list(map(int, m)) for m in members]
        self.prefix_pages_np = np.ascontiguousarray(prefix_pages, dtype=np.int32)
        table = np.full((self.num_groups, 16), -1, np.int32)
        slot = np.full(batch, -1, np.int32)
        for g, ms in enumerate(self.members):
            if not 1 <= len(ms) <= 16:
                raise ValueError("DecodeGroups: 1..16 members per group")
            table[g, :len(ms)] = ms
            for m, b in enumerate(ms):
                if not 0 <= b < batch or slot[b] >= 0:
                    raise ValueError(f"DecodeGroups: sequence {b} is not a distinct batch row")
                slot[b] = 16 * g + m
        self.members_np = np.ascontiguousarray(table.reshape(-1))
        self.slot_np = slot
        self.seq_group_slot = (seq_group_slot if seq_group_slot is not None
                               else torch.from_numpy(slot).to(device))


def paged_decode_workspace_size(batch: int, num_qo_heads: int, num_kv_heads: int, head_dim: int,
                                total_pages: int, page_size: int, dtype: torch.dtype) -> int:
    return int(_lib.load().nslg_paged_decode_workspace_size(batch, num_qo_heads, num_kv_heads, head_dim,
                                                            total_pages, page_size, dtype_code(dtype)))


def paged_decode(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                 kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                 total_pages: int, sm_scale: Optional[float] = None,
                 out: Optional[torch.Tensor] = None, workspace: Optional[Workspace] = None,
                 groups: Optional[DecodeGroups] = None, layout: int = 0) -> torch.Tensor:
    """Decode attention. q: [B, Hq, D] (rows may be strided); returns [B, Hq, D].
    With `groups`, the shared prefix pages of each group are read once for all its
    members (nslg_paged_decode_grouped). `layout`: the chunk-layout record of the
    C entry point (0: none; t > 0: record under tag t in the workspace; -t: a later
    layer of the same forward reads it)."""
    return _decode(q, None, None, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                   sm_scale, out, workspace, groups, layout)


def paged_decode_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, k_layer: torch.Tensor,
                        v_layer: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                        kv_last_page_len: torch.Tensor, total_pages: int, sm_scale: Optional[float] = None,
                        out: Optional[torch.Tensor] = None, workspace: Optional[Workspace] = None,
                        groups: Optional[DecodeGroups] = None, layout: int = 0) -> torch.Tensor:
    """One decode step of a layer (nslg_paged_decode_append / _grouped_append): row b
    of k_new / v_new ([B, ..., Hkv, D], one token per sequence, rows may be strided)
    is written into the pool as sequence b's last token (the slot its block table
    gives for token L_b - 1), then decode attention as paged_decode. Same result as
    append_kv of those rows followed by paged_decode. `layout` as in paged_decode."""
    return _decode(q, k_new, v_new, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                   sm_scale, out, workspace, groups, layout)


def paged_decode_rope_append(q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor, positions: torch.Tensor,
                             cos: torch.Tensor, sin: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                             kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                             total_pages: int, sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                             workspace: Optional[Workspace] = None, groups: Optional[DecodeGroups] = None,
                             layout: int = 0) -> torch.Tensor:
    """paged_decode_append with the rotary embedding folded in
    (nslg_paged_decode_rope_append / _grouped_rope_append): q is rotated at each
    sequence's `positions` entry (int32 [B]) as the decode loads it, and row b of k_new
    is written into the pool rotated at the same position; cos/sin are the model's
    [max_positions, >= D] tables. Same result, bit for bit, as rope_append of q, k_new
    and v_new at those positions into the sequences' new slots followed by
    paged_decode of the rotated q. f16/bf16 pools."""
    _require_gpu(positions, cos, sin)
    _i32(positions, "positions")
    if positions.numel() != q.shape[0] or not positions.is_contiguous():
        raise ValueError("paged_decode_rope_append: one position per sequence, contiguous")
    cos, sin = _rope_tables(cos, sin, q.shape[-1])
    return _decode(q, k_new, v_new, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                   sm_scale, out, workspace, groups, layout, rope=(positions, cos, sin))


def _decode(q, k_new, v_new, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, total_pages, sm_scale,
            out, workspace, groups, layout=0, rope=None):
    _require_gpu(q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        _i32(t, n)
    P, ps, Hkv, D = _layer_geom(k_layer, v_layer)
    if q.dim() != 3 or q.shape[2] != D:
        raise ValueError(f"paged_decode: q must be [B, Hq, {D}]")
    if q.dtype != k_layer.dtype:
        raise TypeError("paged_decode: q dtype must match the pool")
    B, Hq, _ = q.shape
    if q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError("paged_decode: q's [Hq, D] block must be contiguous")
    if kv_indptr.numel() != B + 1 or kv_last_page_len.numel() < B:
        raise ValueError("paged_decode: kv_indptr must have B+1 entries and kv_last_page_len B")
    if out is None:
        out = torch.empty((B, Hq, D), dtype=q.dtype, device=q.device)
    if out.shape != (B, Hq, D) or out.stride(2) != 1 or out.stride(1) != D or out.dtype != q.dtype:
        raise ValueError("paged_decode: bad out tensor")
    lib = _lib.load()
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    rows = None
    if k_new is not None:
        _require_gpu(q, k_new, v_new)
        if k_new.dtype != q.dtype or v_new.dtype != q.dtype:
            raise TypeError("paged_decode_append: k_new/v_new dtype must match the pool")
        rows = []
        for t, name in ((k_new, "k_new"), (v_new, "v_new")):
            n, stride, h = _rows(t, name)
            if n != B or h != Hkv or t.shape[-1] != D:
                raise ValueError(f"paged_decode_append: {name} must hold {B} rows of [{Hkv}, {D}]")
            rows += [t.data_ptr(), stride]
    if rope is not None:
        if rows is None:
            raise ValueError("paged_decode_rope_append: needs the step's new rows")
        pos, cos, sin = rope
        rows += [pos.data_ptr(), cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0]]
    if groups is None:
        need = int(lib.nslg_paged_decode_workspace_size(B, Hq, Hkv, D, int(total_pages), ps, dtype_code(q.dtype)))
        ws = (workspace or Workspace(q.device)).get(need)
        if rope is not None:
            rc = lib.nslg_paged_decode_rope_append(q.data_ptr(), q.stride(0), *rows, k_layer.data_ptr(),
                                                   v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
                                                   kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
                                                   int(total_pages), B, Hq, Hkv, D, scale, dtype_code(q.dtype),
                                                   out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), layout,
                                                   _stream(q))
            _lib.check(rc, "nslg_paged_decode_rope_append")
            return out
        if rows is not None:
            rc = lib.nslg_paged_decode_append(q.data_ptr(), q.stride(0), *rows, k_layer.data_ptr(),
                                              v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(), kv_indices.data_ptr(),
                                              kv_last_page_len.data_ptr(), int(total_pages), B, Hq, Hkv, D, scale,
                                              dtype_code(q.dtype), out.data_ptr(), out.stride(0), ws.data_ptr(),
                                              ws.numel(), layout, _stream(q))
            _lib.check(rc, "nslg_paged_decode_append")
            return out
        rc = lib.nslg_paged_decode(q.data_ptr(), q.stride(0), k_layer.data_ptr(), v_layer.data_ptr(), P, ps,
                                   kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
                                   int(total_pages), B, Hq, Hkv, D, scale, dtype_code(q.dtype),
                                   out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), layout, _stream(q))
        _lib.check(rc, "nslg_paged_decode")
        return out
    _require_gpu(q, groups.seq_group_slot)
    _i32(groups.seq_group_slot, "seq_group_slot")
    if groups.seq_group_slot.numel() != B:
        raise ValueError("paged_decode: one group slot per sequence")
    need = int(lib.nslg_paged_decode_grouped_workspace_size(B, Hq, Hkv, D, int(total_pages), ps,
                                                            dtype_code(q.dtype), groups.num_groups))
    if need == 0:
        raise ValueError("paged_decode: unsupported grouped decode shape")
    ws = (workspace or Workspace(q.device)).get(need)
    if rope is not None:
        rc = lib.nslg_paged_decode_grouped_rope_append(
            q.data_ptr(), q.stride(0), *rows, k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
            kv_indices.data_ptr(), kv_last_page_len.data_ptr(), int(total_pages), B, Hq, Hkv, D, scale,
            dtype_code(q.dtype), groups.seq_group_slot.data_ptr(), groups.num_groups,
            groups.prefix_pages_np.ctypes.data, groups.members_np.ctypes.data, out.data_ptr(), out.stride(0),
            ws.data_ptr(), ws.numel(), layout, _stream(q))
        _lib.check(rc, "nslg_paged_decode_grouped_rope_append")
        return out
    if rows is not None:
        rc = lib.nslg_paged_decode_grouped_append(
            q.data_ptr(), q.stride(0), *rows, k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
            kv_indices.data_ptr(), kv_last_page_len.data_ptr(), int(total_pages), B, Hq, Hkv, D, scale,
            dtype_code(q.dtype), groups.seq_group_slot.data_ptr(), groups.num_groups,
            groups.prefix_pages_np.ctypes.data, groups.members_np.ctypes.data, out.data_ptr(), out.stride(0),
            ws.data_ptr(), ws.numel(), layout, _stream(q))
        _lib.check(rc, "nslg_paged_decode_grouped_append")
        return out
    rc = lib.nslg_paged_decode_grouped(q.data_ptr(), q.stride(0), k_layer.data_ptr(), v_layer.data_ptr(), P, ps,
                                       kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
                                       int(total_pages), B, Hq, Hkv, D, scale, dtype_code(q.dtype),
                                       groups.seq_group_slot.data_ptr(), groups.num_groups,
                                       groups.prefix_pages_np.ctypes.data, groups.members_np.ctypes.data,
                                       out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), layout, _stream(q))
    _lib.check(rc, "nslg_paged_decode_grouped")
    return out


def paged_decode_noalloc(q: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                         kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                         total_pages: int, out: torch.Tensor, sm_scale: Optional[float] = None) -> torch.Tensor:
    """paged_decode through nslg_paged_decode_noalloc: no workspace, nothing allocated
    (the library's static per-GPU scratch holds the split-K partials). The caller
    passes `out` ([B, Hq, D], q's dtype). Calls on one GPU must not overlap. A batch
    needing more than NSLG_NOALLOC_SCRATCH_BYTES of scratch raises KernelLibraryError
    (status NSLG_EWORKSPACE) without launching."""
    _require_gpu(q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, out)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        _i32(t, n)
    P, ps, Hkv, D = _layer_geom(k_layer, v_layer)
    if q.dim() != 3 or q.shape[2] != D or q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError(f"paged_decode_noalloc: q must be [B, Hq, {D}] with a contiguous [Hq, D] block")
    if q.dtype != k_layer.dtype:
        raise TypeError("paged_decode_noalloc: q dtype must match the pool")
    B, Hq, _ = q.shape
    if kv_indptr.numel() != B + 1 or kv_last_page_len.numel() < B:
        raise ValueError("paged_decode_noalloc: kv_indptr must have B+1 entries and kv_last_page_len B")
    if out.shape != (B, Hq, D) or out.stride(2) != 1 or out.stride(1) != D or out.dtype != q.dtype:
        raise ValueError("paged_decode_noalloc: bad out tensor")
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    rc = _lib.load().nslg_paged_decode_noalloc(q.data_ptr(), q.stride(0), k_layer.data_ptr(), v_layer.data_ptr(),
                                               P, ps, kv_indptr.data_ptr(), kv_indices.data_ptr(),
                                               kv_last_page_len.data_ptr(), int(total_pages), B, Hq, Hkv, D, scale,
                                               dtype_code(q.dtype), out.data_ptr(), out.stride(0), _stream(q))
    _lib.check(rc, "nslg_paged_decode_noalloc")
    return out


def decode_plan_step(kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                     new_page, page_size: int, num_new: int, k_pool: Optional[torch.Tensor] = None,
                     v_pool: Optional[torch.Tensor] = None):
    """Next decode step's plan on the device (every sequence gains one token).

    new_page: host int32 array [B], the page sequence b opens this step or -1; num_new:
    how many entries are >= 0. With k_pool/v_pool ([L, P, ps, Hkv, D]) the opened pages
    are zeroed in every layer in the same launch. Returns device int32 tensors (indptr
    [B+1], indices, last_page_len [B], slot_mapping [B], positions [B], new_pages
    [num_new])."""
    import numpy as np
    _require_gpu(kv_indptr, kv_indices, kv_last_page_len)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (kv_last_page_len, "kv_last_page_len")):
        _i32(t, n)
    B = kv_indptr.numel() - 1
    new_page = np.ascontiguousarray(new_page, dtype=np.int32)
    if new_page.shape != (B,):
        raise ValueError(f"decode_plan_step: new_page must have {B} entries")
    pool_args = (None, None, 0, 0, 0, 0, 0)
    if k_pool is not None:
        _require_gpu(k_pool, v_pool)
        L, P, ps_, Hkv, D = _pool_geom(k_pool, v_pool)
        if ps_ != page_size:
            raise ValueError("decode_plan_step: pool page size differs")
        pool_args = (k_pool.data_ptr(), v_pool.data_ptr(), L, P, Hkv, D, dtype_code(k_pool.dtype))
    return _decode_plan_step(kv_indptr, kv_indices, kv_last_page_len, new_page, page_size, num_new, pool_args)


def _decode_plan_step(kv_indptr, kv_indices, kv_last_page_len, new_page, page_size, num_new, pool_args, out=None,
                      new_page_ptr=None):
    """decode_plan_step without the argument checks, for callers whose inputs are the
    previous plan's outputs (the cache manager). new_page: contiguous int32 numpy
    (new_page_ptr: its address, when the caller keeps it; the values are read during
    the call); pool_args: (k_pool ptr, v_pool ptr, L, P, Hkv, D, dtype code) or
    all-null. `out`: preallocated outputs (an object with indptr, indices, lpl, slot,
    pos, new_pages tensors, `ptrs` = their six addresses, indices with room for this
    step's pages), else new tensors (indices exactly this step's pages)."""
    B = kv_indptr.numel() - 1
    if out is not None:
        rc = _lib.fast().decode_plan_step(kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B,
                                          int(page_size),
                                          new_page.ctypes.data if new_page_ptr is None else new_page_ptr, *out.ptrs,
                                          *pool_args, _stream(kv_indptr))
        _lib.check(rc, "nslg_decode_plan_step")
        return out.indptr, out.indices, out.lpl, out.slot, out.pos, out.new_pages
    cap = kv_indices.numel() + num_new
    sizes = [B + 1, cap, B, B, B, num_new]
    buf = torch.empty(sum(sizes) + 1, dtype=torch.int32, device=kv_indptr.device)
    indptr, indices, lpl, slot, pos, new, _ = buf.split(sizes + [1])
    base = buf.data_ptr()
    o = [0]
    for n in sizes:
        o.append(o[-1] + 4 * n)  # byte offsets (an empty part still gets a real address)
    rc = _lib.load().nslg_decode_plan_step(kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(),
                                          B, int(page_size), new_page.ctypes.data, base, base + o[1], base + o[2],
                                          base + o[3], base + o[4], base + o[5], *pool_args, _stream(kv_indptr))
    _lib.check(rc, "nslg_decode_plan_step")
    return indptr, indices, lpl, slot, pos, new


def forward_plan(kv_indptr: torch.Tensor, kv_indices: torch.Tensor, start: torch.Tensor, new_tokens: torch.Tensor,
                 input_offsets: torch.Tensor, pages_allocated: torch.Tensor, input_width: int, page_size: int,
                 total_tokens: int):
    """Per-token write plan of a multi-token forward on the device (nslg_forward_plan).

    All inputs int32 on the device ([B+1] CSR pointers, the CSR ids, four [B] per-sequence
    arrays); total_tokens = sum(new_tokens). Returns (slot_mapping [B*iw],
    positions [B*iw], ragged_rows [total_tokens], qo_indptr [B+1]), int32."""
    _require_gpu(kv_indptr, kv_indices, start, new_tokens, input_offsets, pages_allocated)
    for t, n in ((kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"), (start, "start"),
                 (new_tokens, "new_tokens"), (input_offsets, "input_offsets"), (pages_allocated, "pages_allocated")):
        _i32(t, n)
    B = kv_indptr.numel() - 1
    for t in (start, new_tokens, input_offsets, pages_allocated):
        if t.numel() != B:
            raise ValueError(f"forward_plan: per-sequence arrays must have {B} entries")
    return _forward_plan(kv_indptr, kv_indices, start, new_tokens, input_offsets, pages_allocated, B,
                         int(input_width), int(page_size), int(total_tokens))


def block_table_csr(tables: torch.Tensor, row_offset: torch.Tensor, pages_have: torch.Tensor, synced: torch.Tensor,
                    patch_indptr: torch.Tensor, patch: torch.Tensor, kv_indptr: torch.Tensor,
                    kv_indices: torch.Tensor) -> torch.Tensor:
    """CSR indices of a forward from device-resident block-table rows
    (nslg_block_table_csr): kv_indices[kv_indptr[b] + i] = row entry i of sequence b
    (entries [synced_b, pages_have_b) taken from `patch` and written into `tables`),
    0 past pages_have_b. All int32 on the device; rows of the batch must not overlap
    and must lie inside `tables`. Returns kv_indices."""
    _require_gpu(tables, row_offset, pages_have, synced, patch_indptr, patch, kv_indptr, kv_indices)
    for t, n in ((tables, "tables"), (row_offset, "row_offset"), (pages_have, "pages_have"), (synced, "synced"),
                 (patch_indptr, "patch_indptr"), (patch, "patch"), (kv_indptr, "kv_indptr"),
                 (kv_indices, "kv_indices")):
        _i32(t, n)
    B = kv_indptr.numel() - 1
    for t in (row_offset, pages_have, synced):
        if t.numel() != B:
            raise ValueError(f"block_table_csr: per-sequence arrays must have {B} entries")
    if patch_indptr.numel() != B + 1:
        raise ValueError(f"block_table_csr: patch_indptr must have {B + 1} entries")
    _block_table_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch.numel(), kv_indptr,
                     kv_indices, kv_indices.numel(), B)
    return kv_indices


def _block_table_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch_total, kv_indptr,
                     kv_indices, total_pages, B):
    """block_table_csr without the argument checks (the cache manager's own tables)."""
    rc = _lib.fast().block_table_csr(tables.data_ptr(), tables.numel(), row_offset.data_ptr(), pages_have.data_ptr(),
                                     synced.data_ptr(), patch_indptr.data_ptr(), patch.data_ptr(), int(patch_total),
                                     kv_indptr.data_ptr(), kv_indices.data_ptr(), int(total_pages), int(B),
                                     _stream(tables))
    _lib.check(rc, "nslg_block_table_csr")


def _decode_plan_step_device(kv_indptr, kv_indices, kv_last_page_len, new_page, B, page_size, dst, pool_args):
    """The device planner reading the opened-page list from memory at run time (a
    device tensor or a pinned host tensor), for a step captured in a graph: writes the
    next plan into dst's static tensors."""
    rc = _lib.load().nslg_decode_plan_step_device(
        kv_indptr.data_ptr(), kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B, int(page_size),
        new_page.data_ptr(), dst.indptr.data_ptr(), dst.indices.data_ptr(), dst.lpl.data_ptr(),
        dst.slot.data_ptr(), dst.pos.data_ptr(), dst.new_pages.data_ptr(), *pool_args, _stream(kv_indptr))
    _lib.check(rc, "nslg_decode_plan_step_device")


def _forward_plan(kv_indptr, kv_indices, start, new_tokens, input_offsets, pages_allocated, B, iw, page_size, T,
                  out=None):
    """forward_plan without the argument checks (the cache manager's own tables). The
    outputs (slots, positions, rows, qo_indptr) are consecutive views of `out` (int32,
    at least 2*B*iw + T + B + 1 entries on the device) or of a new buffer."""
    sizes = [B * iw, B * iw, T, B + 1]
    buf = torch.empty(sum(sizes) + 1, dtype=torch.int32, device=kv_indptr.device) if out is None else out
    if buf.numel() < sum(sizes) or buf.dtype != torch.int32:
        raise ValueError("forward_plan: the output buffer is too small or not int32")
    slot, pos, rows, qo = buf[:sum(sizes)].split(sizes)
    base = buf.data_ptr()
    o1, o2 = 4 * B * iw, 8 * B * iw
    o3 = o2 + 4 * T
    rc = _lib.fast().forward_plan(kv_indptr.data_ptr(), kv_indices.data_ptr(), start.data_ptr(),
                                  new_tokens.data_ptr(), input_offsets.data_ptr(), pages_allocated.data_ptr(), B, iw,
                                  page_size, base, base + o1, base + o2, base + o3, _stream(kv_indptr))
    _lib.check(rc, "nslg_forward_plan")
    return slot, pos, rows, qo


def _forward_plan_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch_total, kv_indptr, kv_indices,
                      total_pages, start, new_tokens, input_offsets, B, iw, page_size, T, out):
    """_block_table_csr then _forward_plan in one launch (nslg_forward_plan_csr), the
    cache manager's own tables; `out` as for _forward_plan (required)."""
    sizes = [B * iw, B * iw, T, B + 1]
    if out.numel() < sum(sizes) or out.dtype != torch.int32:
        raise ValueError("forward_plan_csr: the output buffer is too small or not int32")
    slot, pos, rows, qo = out[:sum(sizes)].split(sizes)
    base = out.data_ptr()
    o1, o2 = 4 * B * iw, 8 * B * iw
    o3 = o2 + 4 * T
    rc = _lib.fast().forward_plan_csr(tables.data_ptr(), tables.numel(), row_offset.data_ptr(), pages_have.data_ptr(),
                                      synced.data_ptr(), patch_indptr.data_ptr(), patch.data_ptr(), int(patch_total),
                                      kv_indptr.data_ptr(), kv_indices.data_ptr(), int(total_pages), start.data_ptr(),
                                      new_tokens.data_ptr(), input_offsets.data_ptr(), B, iw, page_size, base,
                                      base + o1, base + o2, base + o3, _stream(tables))
    _lib.check(rc, "nslg_forward_plan_csr")
    return slot, pos, rows, qo


def _forward_plan_csr_at(tables, buf, mid, npatch, total_pages, B, iw, page_size, T, out):
    """_forward_plan_csr with its inputs at fixed places of one int32 upload buffer
    (the cache's native plan): from entry `mid` on, start, new tokens, offsets, pages
    held, row offset, pages held, synced (B each), the patch pointers (B + 1) and the
    patch entries (at least one); before them, at 0, the CSR pointers (B + 1); the
    CSR indices follow the patch. Pointers are computed here instead of views (each
    costs the host ~0.5 us)."""
    sizes = [B * iw, B * iw, T, B + 1]
    if out.numel() < sum(sizes) or out.dtype != torch.int32 or buf.dtype != torch.int32:
        raise ValueError("forward_plan_csr: the output buffer is too small or not int32")
    slot, pos, rows, qo = out[:sum(sizes)].split(sizes)
    a = buf.data_ptr()
    m = a + 4 * mid
    patch = m + 4 * (8 * B + 1)
    idx = patch + 4 * max(npatch, 1)
    base = out.data_ptr()
    o1, o2 = 4 * B * iw, 8 * B * iw
    o3 = o2 + 4 * T
    rc = _lib.fast().forward_plan_csr(tables.data_ptr(), tables.numel(), m + 16 * B, m + 20 * B, m + 24 * B,
                                      m + 28 * B, patch, int(npatch), a, idx, int(total_pages), m, m + 4 * B,
                                      m + 8 * B, B, iw, page_size, base, base + o1, base + o2, base + o3,
                                      _stream(tables))
    _lib.check(rc, "nslg_forward_plan_csr")
    return slot, pos, rows, qo


class DecodeLaunch:
    """Append + split-K decode for every layer of one decode forward.

    What is the same for all layers of the forward (pools, block table, slot
    mapping, sizes, the workspace and its size) is checked and computed once, here;
    each call checks that layer's tensors and issues, on the current stream, one
    nslg_paged_decode_append (each sequence's new row written by the decode chunk
    that reads it; rows that are not 16-byte aligned, 4-byte for fp32, take
    nslg_append_kv then the decode), or with RoPE one nslg_paged_decode_rope_append
    (q and the new K rows rotated in the decode launch; fp32 pools and unaligned
    rows or tables: nslg_rope_append then the decode). Same results as append_kv
    (rope_append) followed by paged_decode on the layer's pool slices.

    A launcher can be re-bound to the next forward's plan (rebind) when the pools,
    batch size and head count stay: the pool geometry is then not checked again.

    The first decode call after a (re)bind records the chunk layout of the plan in
    the workspace under a fresh tag; the later calls of the same plan (the other
    layers of the forward) read it instead of cutting the chunks again."""

    def __init__(self, k_pool: torch.Tensor, v_pool: torch.Tensor, slot_mapping: torch.Tensor,
                 kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                 total_pages: int, num_qo_heads: int, workspace: Optional[Workspace] = None,
                 sm_scale: Optional[float] = None, groups: Optional[DecodeGroups] = None):
        _require_gpu(k_pool, v_pool)
        L, P, ps, Hkv, D = _pool_geom(k_pool, v_pool)
        if num_qo_heads % Hkv:
            raise ValueError(f"DecodeLaunch: Hq={num_qo_heads} is not a multiple of Hkv={Hkv}")
        self.lib = _lib.load()
        # the per-layer calls go through the fast-call binding (same entry points)
        fast = _lib.fast()
        self._f_decode_append, self._f_grouped_append = fast.paged_decode_append, fast.paged_decode_grouped_append
        self._f_decode, self._f_grouped, self._f_rope = fast.paged_decode, fast.paged_decode_grouped, fast.rope_append
        self._f_decode_rope, self._f_grouped_rope = fast.paged_decode_rope_append, fast.paged_decode_grouped_rope_append
        self.device, self.dtype = k_pool.device, k_pool.dtype
        self.dev_index = k_pool.get_device()
        self.code = dtype_code(k_pool.dtype)
        # new rows written inside the decode launch: 16-byte rows (4-byte for fp32)
        self.esize = k_pool.element_size()
        self.row_align = 3 if k_pool.dtype == torch.float32 else 15
        self.L, self.P, self.ps, self.Hkv, self.D, self.Hq = L, P, ps, Hkv, D, num_qo_heads
        self.layer_bytes = P * ps * Hkv * D * k_pool.element_size()
        self.kp0, self.vp0 = k_pool.data_ptr(), v_pool.data_ptr()
        self.pools = (k_pool, v_pool)
        self.workspace = workspace or Workspace(self.device)
        self.scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
        self.B = kv_indptr.numel() - 1
        self._kv_grid = torch.Size((self.B, 1, Hkv, D))
        self.groups, self._ws_pages = None, -1
        self.rebind(slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages, groups, check=True)

    def rebind(self, slot_mapping: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
               kv_last_page_len: torch.Tensor, total_pages: int, groups: Optional[DecodeGroups] = None,
               check: bool = True) -> "DecodeLaunch":
        """Point the launcher at another forward's plan of the same batch size."""
        B = self.B
        self._layout = 0  # the next call records the new plan's chunk layout
        if check:
            _require_gpu(self.pools[0], slot_mapping, kv_indptr, kv_indices, kv_last_page_len)
            for t, n in ((slot_mapping, "slot_mapping"), (kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                         (kv_last_page_len, "kv_last_page_len")):
                _i32(t, n)
            if kv_indptr.numel() != B + 1 or slot_mapping.numel() != B or kv_last_page_len.numel() < B:
                raise ValueError(f"DecodeLaunch: a plan of {B} sequences: one slot and one last-page length each")
        self.keep = (slot_mapping, kv_indptr, kv_indices, kv_last_page_len)
        self.slots, self.indptr, self.indices, self.lpl = (slot_mapping.data_ptr(), kv_indptr.data_ptr(),
                                                           kv_indices.data_ptr(), kv_last_page_len.data_ptr())
        self.total_pages = int(total_pages)
        if groups is self.groups and self.total_pages <= self._ws_pages:
            return self  # the workspace was sized for up to _ws_pages pages
        self.groups = groups
        lib = self.lib
        # the size grows with the page count: size it for some headroom, so the steps of
        # a decode batch (a page more now and then) do not query it again
        bound = self.total_pages + max(self.total_pages // 4, 1024)
        if groups is None:
            need = int(lib.nslg_paged_decode_workspace_size(B, self.Hq, self.Hkv, self.D, bound, self.ps, self.code))
        else:
            if check:
                _require_gpu(self.pools[0], groups.seq_group_slot)
                _i32(groups.seq_group_slot, "seq_group_slot")
                if groups.seq_group_slot.numel() != B:
                    raise ValueError("DecodeLaunch: one group slot per sequence")
            need = int(lib.nslg_paged_decode_grouped_workspace_size(B, self.Hq, self.Hkv, self.D, bound, self.ps,
                                                                    self.code, groups.num_groups))
            if need == 0:
                raise ValueError("DecodeLaunch: unsupported grouped decode shape")
            self.keep = self.keep + (groups.seq_group_slot,)
        self.ws = self.workspace.get(need)
        self._ws_pages = bound
        return self

    def _kv_rows(self, t: torch.Tensor, name: str) -> int:
        """Row stride of k_new / v_new: [B, ..., Hkv, D] rows of one token each."""
        sh = t.shape
        if sh == self._kv_grid:  # [B, 1, Hkv, D]
            st = t.stride()
            if st[3] == 1 and st[2] == self.D:
                return st[0]
        n, stride, h = _rows(t, name)
        if n != self.B or h != self.Hkv or sh[-1] != self.D:
            raise ValueError(f"DecodeLaunch: {name} must hold {self.B} rows of [{self.Hkv}, {self.D}]")
        return stride

    def __call__(self, layer: int, q: torch.Tensor, k_new: torch.Tensor, v_new: torch.Tensor,
                 rope: Optional[Tuple[torch.Tensor, torch.Tensor, torch.Tensor]] = None) -> torch.Tensor:
        """q [B, Hq, D] (rows may be strided), k_new/v_new [B, ..., Hkv, D] rows of one
        token each; returns [B, Hq, D] for pool layer `layer` (q [B, 1, Hq, D]: returns
        [B, 1, Hq * D], the layout of a forward's attention output). With rope = (cos, sin,
        positions int32 [B]) q and k_new are first rotated: in the decode launch itself
        (nslg_paged_decode_rope_append; 16-bit pools, rows and table rows 16-byte
        aligned), else by nslg_rope_append ahead of the decode."""
        if not 0 <= layer < self.L:
            raise IndexError(f"layer {layer} out of range [0, {self.L})")
        dt, di = self.dtype, self.dev_index
        if (q.dtype != dt or k_new.dtype != dt or v_new.dtype != dt or q.get_device() != di
                or k_new.get_device() != di or v_new.get_device() != di):
            raise ValueError(f"DecodeLaunch: tensors must be {self.dtype} on {self.device}")
        B, Hq, D = self.B, self.Hq, self.D
        qs, qst = q.shape, q.stride()
        if len(qs) == 4:  # [B, 1, Hq, D], a forward's input grid: the output is [B, 1, Hq * D]
            if qs != (B, 1, Hq, D) or qst[3] != 1 or qst[2] != D:
                raise ValueError(f"DecodeLaunch: q must be [{B}, 1, {Hq}, {D}] with a contiguous [Hq, D] block")
            out_shape = (B, 1, Hq * D)
        elif qs != (B, Hq, D) or qst[2] != 1 or qst[1] != D:
            raise ValueError(f"DecodeLaunch: q must be [{B}, {Hq}, {D}] with a contiguous [Hq, D] block")
        else:
            out_shape = (B, Hq, D)
        ks = self._kv_rows(k_new, "k_new")
        vs = self._kv_rows(v_new, "v_new")
        stream = _RAW_STREAM(di) if _RAW_STREAM is not None else torch.cuda.current_stream(self.device).cuda_stream
        off = layer * self.layer_bytes
        kp, vp = self.kp0 + off, self.vp0 + off
        lib = self.lib
        out = torch.empty(out_shape, dtype=self.dtype, device=self.device)
        grp = self.groups
        lay = self._layout  # < 0: read the layout recorded under tag -lay
        if lay == 0:  # the first call on this plan records its chunk layout
            lay = next(_LAYOUT_TAGS)
            self._layout = -lay
        if rope is None:
            kn, vn = k_new.data_ptr(), v_new.data_ptr()
            if not (kn | vn | (ks | vs) * self.esize) & self.row_align:
                # one launch: each sequence's new row is written by the chunk that reads it
                q_ptr, q_stride = q.data_ptr(), qst[0]
                if grp is None:
                    rc = self._f_decode_append(q_ptr, q_stride, kn, ks, vn, vs, kp, vp, self.P, self.ps, self.indptr,
                                               self.indices, self.lpl, self.total_pages, B, Hq, self.Hkv, D,
                                               self.scale, self.code, out.data_ptr(), Hq * D, self.ws.data_ptr(),
                                               self.ws.numel(), lay, stream)
                    _lib.check(rc, "nslg_paged_decode_append")
                else:
                    rc = self._f_grouped_append(
                        q_ptr, q_stride, kn, ks, vn, vs, kp, vp, self.P, self.ps, self.indptr, self.indices,
                        self.lpl, self.total_pages, B, Hq, self.Hkv, D, self.scale, self.code,
                        grp.seq_group_slot.data_ptr(), grp.num_groups, grp.prefix_pages_np.ctypes.data,
                        grp.members_np.ctypes.data, out.data_ptr(), Hq * D, self.ws.data_ptr(), self.ws.numel(),
                        lay, stream)
                    _lib.check(rc, "nslg_paged_decode_grouped_append")
                return out
            rc = lib.nslg_append_kv(kn, vn, ks, vs, self.slots, B, kp, vp, self.P * self.ps, self.Hkv, D,
                                    self.code, stream)
            _lib.check(rc, "nslg_append_kv")
            q_ptr, q_stride = q.data_ptr(), qst[0]
        else:
            cos, sin, pos = rope
            if pos.get_device() != di or pos.dtype != torch.int32 or pos.numel() != B or not pos.is_contiguous():
                raise ValueError(f"DecodeLaunch: positions must be {B} contiguous int32 on {self.device}")
            cos, sin = _rope_tables(cos, sin, D)
            if cos.get_device() != di:
                raise ValueError(f"DecodeLaunch: rope tables must be on {self.device}")
            kn, vn = k_new.data_ptr(), v_new.data_ptr()
            cp, sp, cst = cos.data_ptr(), sin.data_ptr(), cos.stride(0)
            if (self.code != _DTYPE_CODE[torch.float32] and not (kn | vn | (ks | vs) * self.esize) & self.row_align
                    and not (cp | sp | cst * 4) & 15):
                # one launch: q rotated as the decode loads it, each new K row rotated by
                # the chunk that writes it
                if grp is None:
                    rc = self._f_decode_rope(q.data_ptr(), qst[0], kn, ks, vn, vs, pos.data_ptr(), cp, sp, cst,
                                             cos.shape[0], kp, vp, self.P, self.ps, self.indptr, self.indices,
                                             self.lpl, self.total_pages, B, Hq, self.Hkv, D, self.scale, self.code,
                                             out.data_ptr(), Hq * D, self.ws.data_ptr(), self.ws.numel(), lay, stream)
                    _lib.check(rc, "nslg_paged_decode_rope_append")
                else:
                    rc = self._f_grouped_rope(
                        q.data_ptr(), qst[0], kn, ks, vn, vs, pos.data_ptr(), cp, sp, cst, cos.shape[0], kp, vp,
                        self.P, self.ps, self.indptr, self.indices, self.lpl, self.total_pages, B, Hq, self.Hkv, D,
                        self.scale, self.code, grp.seq_group_slot.data_ptr(), grp.num_groups,
                        grp.prefix_pages_np.ctypes.data, grp.members_np.ctypes.data, out.data_ptr(), Hq * D,
                        self.ws.data_ptr(), self.ws.numel(), lay, stream)
                    _lib.check(rc, "nslg_paged_decode_grouped_rope_append")
                return out
            q_rot = torch.empty((B, Hq, D), dtype=self.dtype, device=self.device)
            rc = self._f_rope(q.data_ptr(), q.stride(0), q_rot.data_ptr(), Hq * D, k_new.data_ptr(), ks,
                              v_new.data_ptr(), vs, pos.data_ptr(), self.slots, B, cos.data_ptr(), sin.data_ptr(),
                              cos.stride(0), cos.shape[0], Hq, self.Hkv, D, kp, vp, self.P * self.ps, self.code,
                              stream)
            _lib.check(rc, "nslg_rope_append")
            q_ptr, q_stride = q_rot.data_ptr(), Hq * D
        if grp is None:
            rc = self._f_decode(q_ptr, q_stride, kp, vp, self.P, self.ps, self.indptr, self.indices, self.lpl,
                                self.total_pages, B, Hq, self.Hkv, D, self.scale, self.code, out.data_ptr(), Hq * D,
                                self.ws.data_ptr(), self.ws.numel(), lay, stream)
            _lib.check(rc, "nslg_paged_decode")
        else:
            rc = self._f_grouped(q_ptr, q_stride, kp, vp, self.P, self.ps, self.indptr, self.indices, self.lpl,
                                 self.total_pages, B, Hq, self.Hkv, D, self.scale, self.code,
                                 grp.seq_group_slot.data_ptr(), grp.num_groups, grp.prefix_pages_np.ctypes.data,
                                 grp.members_np.ctypes.data, out.data_ptr(), Hq * D, self.ws.data_ptr(),
                                 self.ws.numel(), lay, stream)
            _lib.check(rc, "nslg_paged_decode_grouped")
        return out


_PREFILL_WS: Dict[Tuple[int, int, int, int, int], int] = {}  # nslg_paged_prefill_workspace_size by call shape


def _paged_prefill_layer(q: torch.Tensor, qo_indptr: torch.Tensor, total_q: int, max_q: int,
                         k_layer: torch.Tensor, v_layer: torch.Tensor, kv_indptr: torch.Tensor,
                         kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor, workspace: Workspace,
                         q_rows: Optional[torch.Tensor] = None, grid_width: int = 0) -> torch.Tensor:
    """paged_prefill for the cache manager: its pool layer, plan (int32 arrays on the
    pool's device, qo_indptr and kv_indptr of B + 1 entries) and workspace are taken
    as they are; the caller's q gets paged_prefill's checks (a q that fails one goes
    through paged_prefill, which raises its error). Default scale 1/sqrt(D)."""
    dev, dt = k_layer.get_device(), k_layer.dtype
    P, ps, Hkv, D = k_layer.shape
    B = kv_indptr.numel() - 1
    if (q.get_device() != dev or q.dtype != dt or q.dim() != 3 or q.shape[2] != D or q.stride(2) != 1
            or q.stride(1) != D or q.shape[0] < total_q
            or (q_rows is not None and (grid_width < 1 or q.shape[0] != B * grid_width))):
        return paged_prefill(q, qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr, kv_indices,
                             kv_last_page_len, workspace=workspace, q_rows=q_rows, grid_width=grid_width)
    T, Hq = q.shape[0], q.shape[1]
    out = torch.empty((T, Hq, D), dtype=dt, device=q.device)
    fast = _lib.fast()
    key = (B, Hq, D, int(total_q), int(max_q))
    need = _PREFILL_WS.get(key)
    if need is None:  # a pure function of the call shape: asked once per shape
        need = _PREFILL_WS[key] = int(_lib.load().nslg_paged_prefill_workspace_size(*key))
        if len(_PREFILL_WS) > 4096:
            _PREFILL_WS.clear()
    ws = workspace.get(need)
    stream = _stream(k_layer)
    scale = 1.0 / math.sqrt(D)
    if q_rows is not None:
        rc = fast.paged_prefill_grid(q.data_ptr(), q.stride(0), qo_indptr.data_ptr(), q_rows.data_ptr(),
                                     int(grid_width), int(total_q), int(max_q), k_layer.data_ptr(),
                                     v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(), kv_indices.data_ptr(),
                                     kv_last_page_len.data_ptr(), B, Hq, Hkv, D, scale, _DTYPE_CODE[dt],
                                     out.data_ptr(), Hq * D, ws.data_ptr(), ws.numel(), stream)
        _lib.check(rc, "nslg_paged_prefill_grid")
        return out
    rc = fast.paged_prefill(q.data_ptr(), q.stride(0), qo_indptr.data_ptr(), int(total_q), int(max_q),
                            k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
                            kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B, Hq, Hkv, D, scale, _DTYPE_CODE[dt],
                            out.data_ptr(), Hq * D, ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc, "nslg_paged_prefill")
    return out


def _paged_prefill_append_layer(q: torch.Tensor, qo_indptr: torch.Tensor, total_q: int, max_q: int,
                                k_new: torch.Tensor, v_new: torch.Tensor, k_layer: torch.Tensor,
                                v_layer: torch.Tensor, kv_indptr: torch.Tensor, kv_indices: torch.Tensor,
                                kv_last_page_len: torch.Tensor, workspace: Workspace,
                                q_rows: Optional[torch.Tensor] = None, grid_width: int = 0
                                ) -> Optional[torch.Tensor]:
    """nslg_paged_prefill_append for the cache manager (its pool layer, plan and
    workspace taken as they are): the forward's K/V rows written and its queries
    attended in one launch. None, with nothing launched, where the one launch does not
    apply (fp32 pools, q / k_new / v_new not rows of a 16-bit forward at one 16-byte
    stride each): the caller then appends and runs _paged_prefill_layer, whose checks
    raise any error."""
    dev, dt = k_layer.get_device(), k_layer.dtype
    if dt == torch.float32:
        return None
    P, ps, Hkv, D = k_layer.shape
    B = kv_indptr.numel() - 1
    n = q.shape[0] if q.dim() == 3 else -1
    strides = []
    for x in (k_new, v_new):
        if (x.get_device() != dev or x.dtype != dt or x.dim() < 2 or x.shape[-1] != D or x.shape[-2] != Hkv
                or x.numel() != n * Hkv * D or x.data_ptr() % 16):
            return None
        if x.is_contiguous():  # the model's own [B, S, Hkv, D] rows
            strides.append(Hkv * D)
            continue
        try:  # rows at one stride, e.g. the K and V halves of one projection output
            _, st, _ = _rows(x, "k_new/v_new")
        except ValueError:
            return None
        if (st * x.element_size()) % 16:
            return None
        strides.append(st)
    if (q.get_device() != dev or q.dtype != dt or q.stride(2) != 1 or q.stride(1) != D or n < total_q
            or q.shape[2] != D or (q_rows is not None and (grid_width < 1 or n != B * grid_width))):
        return None
    Hq = q.shape[1]
    out = torch.empty((n, Hq, D), dtype=dt, device=q.device)
    key = (B, Hq, D, int(total_q), int(max_q))
    need = _PREFILL_WS.get(key)
    if need is None:
        need = _PREFILL_WS[key] = int(_lib.load().nslg_paged_prefill_workspace_size(*key))
        if len(_PREFILL_WS) > 4096:
            _PREFILL_WS.clear()
    ws = workspace.get(need)
    rc = _lib.fast().paged_prefill_append(
        q.data_ptr(), q.stride(0), qo_indptr.data_ptr(), None if q_rows is None else q_rows.data_ptr(),
        int(grid_width), int(total_q), int(max_q), k_new.data_ptr(), strides[0], v_new.data_ptr(), strides[1],
        k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(), kv_indices.data_ptr(),
        kv_last_page_len.data_ptr(), B, Hq, Hkv, D, 1.0 / math.sqrt(D), _DTYPE_CODE[dt], out.data_ptr(), Hq * D,
        ws.data_ptr(), ws.numel(), _stream(k_layer))
    _lib.check(rc, "nslg_paged_prefill_append")
    return out


def paged_prefill_append(q: torch.Tensor, qo_indptr: torch.Tensor, total_q: int, max_q: int,
                         k_new: torch.Tensor, v_new: torch.Tensor, k_layer: torch.Tensor, v_layer: torch.Tensor,
                         kv_indptr: torch.Tensor, kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                         sm_scale: Optional[float] = None, workspace: Optional[Workspace] = None,
                         q_rows: Optional[torch.Tensor] = None, grid_width: int = 0) -> torch.Tensor:
    """append_kv of the forward's new rows followed by paged_prefill, in one launch
    (nslg_paged_prefill_append; 16-bit pools). k_new / v_new: [..., Hkv, D] with q's
    rows (ragged [T] rows, or the B * grid_width grid rows with q_rows): token t of
    sequence b is written to position L_b - n_b + t through the block table. Returns
    paged_prefill's result; the pool holds the rows, as after append_kv."""
    _require_gpu(q, qo_indptr, k_new, v_new, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len)
    for t, name in ((qo_indptr, "qo_indptr"), (kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                    (kv_last_page_len, "kv_last_page_len")):
        _i32(t, name)
    if q_rows is not None:
        _require_gpu(q, q_rows)
        _i32(q_rows, "q_rows")
        if q_rows.numel() < total_q or grid_width < 1 or q.shape[0] != (kv_indptr.numel() - 1) * grid_width:
            raise ValueError("paged_prefill_append: a grid of B x grid_width rows of q and one q_rows entry per token")
    P, ps, Hkv, D = _layer_geom(k_layer, v_layer)
    if q.dim() != 3 or q.shape[2] != D or q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError(f"paged_prefill_append: q must be [T, Hq, {D}] with a contiguous [Hq, D] block")
    if q.dtype != k_layer.dtype or k_new.dtype != k_layer.dtype or v_new.dtype != k_layer.dtype:
        raise TypeError("paged_prefill_append: q, k_new and v_new dtypes must match the pool")
    if tuple(k_new.shape[-2:]) != (Hkv, D) or tuple(v_new.shape[-2:]) != (Hkv, D):
        raise ValueError("paged_prefill_append: k_new/v_new trailing dims must be [Hkv, D] of the pool")
    nk, ks, _ = _rows(k_new, "k_new")
    nv, vs, _ = _rows(v_new, "v_new")
    T, Hq, _ = q.shape
    if nk != T or nv != T:
        raise ValueError(f"paged_prefill_append: {nk} k rows / {nv} v rows for {T} q rows")
    B = kv_indptr.numel() - 1
    if qo_indptr.numel() != B + 1 or T < total_q:
        raise ValueError("paged_prefill_append: qo_indptr must have B+1 entries and q at least total_q rows")
    out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    lib = _lib.load()
    need = int(lib.nslg_paged_prefill_workspace_size(B, Hq, D, int(total_q), int(max_q)))
    ws = (workspace or Workspace(q.device)).get(need)
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    rc = lib.nslg_paged_prefill_append(q.data_ptr(), q.stride(0), qo_indptr.data_ptr(),
                                       None if q_rows is None else q_rows.data_ptr(), int(grid_width),
                                       int(total_q), int(max_q), k_new.data_ptr(), ks, v_new.data_ptr(), vs,
                                       k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
                                       kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B, Hq, Hkv, D, scale,
                                       dtype_code(q.dtype), out.data_ptr(), out.stride(0), ws.data_ptr(),
                                       ws.numel(), _stream(q))
    _lib.check(rc, "nslg_paged_prefill_append")
    return out


def paged_prefill(q: torch.Tensor, qo_indptr: torch.Tensor, total_q: int, max_q: int,
                  k_layer: torch.Tensor, v_layer: torch.Tensor, kv_indptr: torch.Tensor,
                  kv_indices: torch.Tensor, kv_last_page_len: torch.Tensor,
                  sm_scale: Optional[float] = None, out: Optional[torch.Tensor] = None,
                  workspace: Optional[Workspace] = None, q_rows: Optional[torch.Tensor] = None,
                  grid_width: int = 0) -> torch.Tensor:
    """Causal (bottom-right) prefill attention. q: ragged [T, Hq, D]; returns [T, Hq, D].
    With q_rows (int32 [total_q] on the device) q and the result are the forward's
    padded grid of B * grid_width rows instead (nslg_paged_prefill_grid): ragged row t
    is grid row q_rows[t], sequence b's rows contiguous in its block of grid_width
    rows, and the rows holding no token come out as zeros."""
    _require_gpu(q, qo_indptr, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len)
    if q_rows is not None:
        _require_gpu(q, q_rows)
        _i32(q_rows, "q_rows")
        if q_rows.numel() < total_q or grid_width < 1 or q.shape[0] != (kv_indptr.numel() - 1) * grid_width:
            raise ValueError("paged_prefill: a grid of B x grid_width rows of q and one q_rows entry per token")
    for t, n in ((qo_indptr, "qo_indptr"), (kv_indptr, "kv_indptr"), (kv_indices, "kv_indices"),
                 (kv_last_page_len, "kv_last_page_len")):
        _i32(t, n)
    P, ps, Hkv, D = _layer_geom(k_layer, v_layer)
    if q.dim() != 3 or q.shape[2] != D or q.stride(2) != 1 or q.stride(1) != D:
        raise ValueError(f"paged_prefill: q must be [T, Hq, {D}] with a contiguous [Hq, D] block")
    if q.dtype != k_layer.dtype:
        raise TypeError("paged_prefill: q dtype must match the pool")
    T, Hq, _ = q.shape
    B = kv_indptr.numel() - 1
    if qo_indptr.numel() != B + 1 or T < total_q:
        raise ValueError("paged_prefill: qo_indptr must have B+1 entries and q at least total_q rows")
    if out is None:
        out = torch.empty((T, Hq, D), dtype=q.dtype, device=q.device)
    elif q_rows is not None and (out.shape[0] != T or out.dim() != 3 or out.shape[1:] != (Hq, D)
                                 or out.stride(2) != 1 or out.stride(1) != D or out.dtype != q.dtype):
        raise ValueError("paged_prefill: out must be the grid's [B * grid_width, Hq, D] rows")
    lib = _lib.load()
    need = int(lib.nslg_paged_prefill_workspace_size(B, Hq, D, int(total_q), int(max_q)))
    ws = (workspace or Workspace(q.device)).get(need)
    scale = (1.0 / math.sqrt(D)) if sm_scale is None else float(sm_scale)
    if q_rows is not None:
        rc = lib.nslg_paged_prefill_grid(q.data_ptr(), q.stride(0), qo_indptr.data_ptr(), q_rows.data_ptr(),
                                         int(grid_width), int(total_q), int(max_q), k_layer.data_ptr(),
                                         v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(), kv_indices.data_ptr(),
                                         kv_last_page_len.data_ptr(), B, Hq, Hkv, D, scale, dtype_code(q.dtype),
                                         out.data_ptr(), out.stride(0), ws.data_ptr(), ws.numel(), _stream(q))
        _lib.check(rc, "nslg_paged_prefill_grid")
        return out
    rc = lib.nslg_paged_prefill(q.data_ptr(), q.stride(0), qo_indptr.data_ptr(), int(total_q), int(max_q),
                                k_layer.data_ptr(), v_layer.data_ptr(), P, ps, kv_indptr.data_ptr(),
                                kv_indices.data_ptr(), kv_last_page_len.data_ptr(), B, Hq, Hkv, D, scale,
                                dtype_code(q.dtype), out.data_ptr(), out.stride(0), ws.data_ptr(),
                                ws.numel(), _stream(q))
    _lib.check(rc, "nslg_paged_prefill")
    return out
