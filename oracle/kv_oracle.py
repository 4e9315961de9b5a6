"""CPU oracle of nanoslg's KV-cache hot path — TEST INFRASTRUCTURE ONLY.

This module restates, on the CPU, what the reference computes on the path
(nanoslg/kv_cache.py). It is the checker for the HIP implementation in
``nanoslg_amd``: only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it, and never as the thing that
is measured or shipped. The product path has no CPU fallback.

What each function follows (reference file:line) and what pins it (the pinning
tests live in tests/test_oracle.py):

  sdpa_gqa               kv_cache.py:44-56      pinned by fp64 brute force
                                                (sdpa_brute_f64), L=1 -> out=v,
                                                constant K -> mean(V)
  sdpa_brute_f64         (textbook softmax(qk^T/sqrt(D))v in float64)
                                                pinned by closed forms (L=1,
                                                constant K, one-hot scores)
  build_causal_mask      kv_cache.py:192-224    pinned by closed-form cases and
                                                against is_causal SDPA
  position_ids           kv_cache.py:267-278, 292-295, 567-573, 635-637
                                                pinned by closed form
  rope_inv_freq / rope_tables
                         models.py:37-66        pinned against transformers'
                                                own llama3 inverse frequencies
                                                (a library routine), closed
                                                forms (theta^(-2i/dim), the
                                                three wavelength bands, t = 0
                                                row = (1, 0), angle t * f)
  apply_rotary_ref / rope_forward_ref
                         models.py:69-83, 96-103
                                                pinned by the float64 rotation
                                                (rotate_f64) within 16-bit
                                                rounding, position 0 = identity,
                                                rotation by a quarter turn, and
                                                planted sign / half mistakes
                                                that the checks must catch
  rotate_f64             (the rotation of each (d, d + D/2) pair in float64)
                                                pinned by norm preservation and
                                                composition R(a) R(b) = R(a + b)
  ContiguousRef          kv_cache.py:227-379    the CPU baseline (config 1);
                                                pinned against PagedRef on the
                                                same inputs and against
                                                sdpa_brute_f64
  append_rows / gather_rows / zero_pages / copy_pages
                         kv_cache.py:301-314, 411, 429-436, 661-674
                                                pinned by brute-force per-row
                                                loops on tiny pools
  plan_csr               kv_cache.py:598-615    pinned by closed form
  PagePoolRef            kv_cache.py:382-442    pinned by invariants (page 0
                                                reserved, no double allocation,
                                                conservation, zero on alloc)
  RadixTreeRef           kv_cache.py:445-531    pinned by brute-force longest
                                                common full-page prefix,
                                                invariants, and operation
                                                sequences recorded from the
                                                reference's own RadixTree and
                                                PagePool (tests/golden/
                                                radix_vectors.json); its
                                                stop_at_gap mode (the build's
                                                match, ending at an evicted
                                                page) by a known-answer case
                                                against the default mode
  PagedRef               kv_cache.py:534-777    write plan + CoW order rule,
                                                CSR, attend = SDPA over the
                                                gathered pages; pinned against
                                                ContiguousRef
"""
from __future__ import annotations

import math
import time
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch
import torch.nn.functional as F

# --------------------------------------------------------------------------------------
# attention
# --------------------------------------------------------------------------------------


def sdpa_gqa(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             attn_mask: Optional[torch.Tensor] = None, is_causal: bool = False) -> torch.Tensor:
    """q [B,Hq,Sq,D], k/v [B,Hkv,Skv,D] -> [B,Hq,Sq,D] (kv_cache.py:44-56).

    Query head h reads KV head h // (Hq/Hkv) (enable_gqa); scale 1/sqrt(D)."""
    if q.shape[1] != k.shape[1]:
        return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal,
                                              enable_gqa=True)
    return F.scaled_dot_product_attention(q, k, v, attn_mask=attn_mask, is_causal=is_causal)


def sdpa_brute_f64(q: np.ndarray, k: np.ndarray, v: np.ndarray,
                   visible: Optional[np.ndarray] = None, scale: Optional[float] = None) -> np.ndarray:
    """Textbook attention in float64. q [Hq,Sq,D], k/v [Hkv,Skv,D], visible [Sq,Skv] bool."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    Hq, Sq, D = q.shape
    Hkv = k.shape[0]
    G = Hq // Hkv
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    out = np.zeros((Hq, Sq, D))
    for h in range(Hq):
        s = (q[h] @ k[h // G].T) * scale
        if visible is not None:
            s = np.where(visible, s, -np.inf)
        m = s.max(axis=1, keepdims=True)
        p = np.exp(s - m)
        p /= p.sum(axis=1, keepdims=True)
        out[h] = p @ v[h // G]
    return out


def build_causal_mask(batch_size, input_width, start_positions, new_token_counts, input_offsets,
                      seq_lens, max_kv_len, dtype=torch.float32):
    """[B,1,Q,KV] additive mask or None (kv_cache.py:192-224).

    Key j is visible to input row off_b+t iff j <= start_b+t and j < seq_len_b."""
    B = batch_size
    if B == 1 and start_positions[0] == 0 and input_offsets[0] == 0:
        return None
    if all(n == 1 for n in new_token_counts) and len(set(seq_lens)) == 1:
        return None
    if (all(s == 0 for s in start_positions) and all(o == 0 for o in input_offsets)
            and len(set(new_token_counts)) == 1):
        return None
    neg = -65504.0 if dtype == torch.float16 else float("-inf")
    mask = torch.full((B, 1, input_width, max_kv_len), neg, dtype=dtype)
    for b in range(B):
        off, ntok, base, kv = input_offsets[b], new_token_counts[b], start_positions[b], seq_lens[b]
        if ntok == 0:
            continue
        qp = torch.arange(ntok) + base
        kp = torch.arange(max_kv_len)
        ok = (kp[None, :] <= qp[:, None]) & (kp[None, :] < kv)
        mask[b, 0, off:off + ntok] = torch.where(ok, torch.tensor(0.0, dtype=dtype),
                                                 torch.tensor(neg, dtype=dtype))
    return mask


def position_ids(start_positions, new_token_counts, input_offsets, S: Optional[int] = None):
    """[B, S] int64 positions (kv_cache.py:267-278, 292-295): pos[b, off+t] = start_b + t."""
    B = len(start_positions)
    iw = max(o + n for o, n in zip(input_offsets, new_token_counts)) if B else 1
    pos = torch.zeros(B, iw, dtype=torch.long)
    for b in range(B):
        o, n = input_offsets[b], new_token_counts[b]
        if n > 0:
            pos[b, o:o + n] = torch.arange(start_positions[b], start_positions[b] + n)
    if S is None or S == iw:
        return pos
    if S < iw:
        return pos[:, :S]
    return torch.cat([pos, pos.new_zeros(B, S - iw)], 1)


# --------------------------------------------------------------------------------------
# rotary position embedding (nanoslg/models.py:37-105)
# --------------------------------------------------------------------------------------


def rope_inv_freq(dim: int, theta: float, rope_scaling: Optional[dict] = None) -> torch.Tensor:
    """float32 inverse frequencies [dim/2] of the tables (models.py:40-59).

    f_i = 1 / theta^(2i/dim) in float32. With a "llama3" rope_scaling, each f is
    kept when its wavelength 2*pi/f is below original_max_position_embeddings /
    high_freq_factor, divided by `factor` when it is above original /
    low_freq_factor, and blended linearly in between (s = (original / wavelength
    - low) / (high - low); (1 - s) f / factor + s f), each step a float32 scalar op
    as the reference's per-element loop does."""
    freqs = 1.0 / (theta ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
    if rope_scaling and rope_scaling.get("rope_type") == "llama3":
        factor = rope_scaling.get("factor", 8.0)
        lo = rope_scaling.get("low_freq_factor", 1.0)
        hi = rope_scaling.get("high_freq_factor", 4.0)
        old_ctx = rope_scaling.get("original_max_position_embeddings", 8192)
        lo_wl, hi_wl = old_ctx / lo, old_ctx / hi
        scaled = []
        for i in range(freqs.numel()):
            f = freqs[i]  # a 0-d float32 tensor: every op below is a float32 op
            wl = 2 * math.pi / f
            if wl < hi_wl:
                scaled.append(f)
            elif wl > lo_wl:
                scaled.append(f / factor)
            else:
                s = (old_ctx / wl - lo) / (hi - lo)
                scaled.append((1 - s) * f / factor + s * f)
        freqs = torch.stack(scaled).to(torch.float32)
    return freqs


def rope_tables(dim: int, max_seq_len: int, theta: float, rope_scaling: Optional[dict] = None):
    """fp32 (cos, sin), each [max_seq_len, dim] (models.py:37-66): angles t * f for
    t < max_seq_len (float32 outer product with rope_inv_freq), the dim/2 angles
    repeated to dim, then cos and sin."""
    freqs = rope_inv_freq(dim, theta, rope_scaling)
    t = torch.arange(max_seq_len, dtype=torch.float32)
    ang = torch.outer(t, freqs)
    ang = torch.cat((ang, ang), dim=-1)
    return ang.cos(), ang.sin()


def apply_rotary_ref(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x [B, S, H, D] rotated with per-row cos/sin [B, S, D] (models.py:69-83): the
    tables are cast to x's dtype and the expression x*c + cat(-x2, x1)*s is
    evaluated as eager tensor ops in that dtype (each product and the sum rounded
    to it)."""
    c = cos[:, :, None, :].to(dtype=x.dtype)
    s = sin[:, :, None, :].to(dtype=x.dtype)
    half = x.shape[-1] // 2
    x1, x2 = x[..., :half], x[..., half:]
    return x * c + torch.cat((-x2, x1), dim=-1) * s


def rope_forward_ref(q: torch.Tensor, k_new: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                     pos_ids: torch.Tensor):
    """The position part of _attention_forward (models.py:96-103): gather the table
    rows at pos_ids [B, S], rotate q and k_new. Returns (q_rot, k_rot)."""
    c, s = cos[pos_ids], sin[pos_ids]
    return apply_rotary_ref(q, c, s), apply_rotary_ref(k_new, c, s)


def rotate_f64(x: np.ndarray, pos: np.ndarray, inv_freq: np.ndarray) -> np.ndarray:
    """Closed form of the rotation in float64: element pairs (d, d + D/2) of each row
    turned by the angle pos * inv_freq[d] (x [N, H, D], pos [N])."""
    half = x.shape[-1] // 2
    ang = pos.astype(np.float64)[:, None] * inv_freq.astype(np.float64)[None, :]
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half].astype(np.float64), x[..., half:].astype(np.float64)
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


# --------------------------------------------------------------------------------------
# byte movement on a pool layer [P*ps, Hkv, D] (numpy, bit-exact)
# --------------------------------------------------------------------------------------


def append_rows(pool_rows: np.ndarray, rows: np.ndarray, slot_mapping: np.ndarray) -> None:
    """pool_rows[slot] = rows[i] for slot >= 0 (kv_cache.py:301-303, 661-674), in order."""
    for i, s in enumerate(np.asarray(slot_mapping).tolist()):
        if 0 <= s < pool_rows.shape[0]:
            pool_rows[s] = rows[i]


def seq_lens_from_csr(indptr, last_page_len, page_size):
    indptr = np.asarray(indptr)
    lpl = np.asarray(last_page_len)
    out = []
    for b in range(len(indptr) - 1):
        n = int(indptr[b + 1] - indptr[b])
        out.append((n - 1) * page_size + int(lpl[b]) if n > 0 else 0)
    return out


def gather_rows(pool_rows: np.ndarray, page_size: int, indptr, indices, last_page_len, max_len):
    """[B, max_len, Hkv, D]: token t of seq b from slot indices[indptr[b]+t//ps]*ps + t%ps;
    zeros past the length (kv_cache.py:312-314 slice read, per page)."""
    lens = seq_lens_from_csr(indptr, last_page_len, page_size)
    B = len(lens)
    out = np.zeros((B, max_len) + pool_rows.shape[1:], dtype=pool_rows.dtype)
    for b in range(B):
        for t in range(min(lens[b], max_len)):
            pid = int(indices[int(indptr[b]) + t // page_size])
            out[b, t] = pool_rows[pid * page_size + t % page_size]
    return out


def zero_pages(pool: np.ndarray, page_ids) -> None:
    """pool[:, pid] = 0 for every layer (kv_cache.py:411). pool [L, P, ps, Hkv, D]."""
    for pid in page_ids:
        if 0 <= pid < pool.shape[1]:
            pool[:, pid] = 0


def copy_pages(pool: np.ndarray, src_ids, dst_ids) -> None:
    """pool[:, dst] = pool[:, src] for every layer and slot (kv_cache.py:433-434)."""
    for s, d in zip(src_ids, dst_ids):
        if 0 <= s < pool.shape[1] and 0 <= d < pool.shape[1]:
            pool[:, d] = pool[:, s]


def plan_csr(block_tables: Sequence[Sequence[int]], seq_lens: Sequence[int], page_size: int):
    """CSR block table (kv_cache.py:598-615): indptr, indices (missing -> page 0), last_page_len."""
    indptr, indices, lpl = [0], [], []
    for bt, kv in zip(block_tables, seq_lens):
        n = math.ceil(kv / page_size) if kv > 0 else 0
        for p in range(n):
            indices.append(bt[p] if p < len(bt) else 0)
        indptr.append(indptr[-1] + n)
        lpl.append((kv - (n - 1) * page_size) if n > 0 else 0)
    return (np.array(indptr, np.int32), np.array(indices or [0], np.int32),
            np.array(lpl or [0], np.int32))


def paged_attention_ref(q: torch.Tensor, k_rows: torch.Tensor, v_rows: torch.Tensor,
                        page_size: int, indptr, indices, last_page_len, qo_lens: Sequence[int],
                        sm_scale: Optional[float] = None) -> List[torch.Tensor]:
    """fp32 SDPA over each sequence's gathered pages with bottom-right causal rows.

    q: list-like per sequence [n_b, Hq, D]; k_rows/v_rows: one layer [P*ps, Hkv, D].
    Returns per sequence [n_b, Hq, D] float32 (the FlashInfer paged decode/prefill
    semantics of kv_cache.py:617-632, 648-655 restated as SDPA)."""
    lens = seq_lens_from_csr(indptr, last_page_len, page_size)
    outs = []
    for b, L in enumerate(lens):
        n = qo_lens[b]
        qb = q[b].float()
        if n == 0:
            outs.append(torch.zeros(0, qb.shape[1], qb.shape[2]))
            continue
        rows = [int(indices[int(indptr[b]) + t // page_size]) * page_size + t % page_size for t in range(L)]
        idx = torch.tensor(rows, dtype=torch.long)
        kb = k_rows[idx].float().transpose(0, 1).unsqueeze(0)  # [1,Hkv,L,D]
        vb = v_rows[idx].float().transpose(0, 1).unsqueeze(0)
        qq = qb.transpose(0, 1).unsqueeze(0)  # [1,Hq,n,D]
        start = L - n
        vis = (torch.arange(L)[None, :] <= (start + torch.arange(n))[:, None])
        mask = torch.zeros(n, L).masked_fill(~vis, float("-inf"))
        if sm_scale is None:
            o = sdpa_gqa(qq, kb, vb, attn_mask=mask[None, None])
        else:
            o = F.scaled_dot_product_attention(qq, kb, vb, attn_mask=mask[None, None], scale=sm_scale,
                                               enable_gqa=qq.shape[1] != kb.shape[1])
        outs.append(o[0].transpose(0, 1))
    return outs


# --------------------------------------------------------------------------------------
# contiguous backend (the CPU baseline), kv_cache.py:227-379
# --------------------------------------------------------------------------------------


class ContiguousRef:
    """Op-for-op CPU restatement of ContiguousKVCache + ContiguousCacheContext."""

    def __init__(self, num_layers, max_batch_size, max_seq_len, num_kv_heads, head_dim,
                 dtype=torch.float32):
        shape = (num_layers, max_batch_size, max_seq_len, num_kv_heads, head_dim)
        self.k = torch.zeros(shape, dtype=dtype)
        self.v = torch.zeros(shape, dtype=dtype)
        self.max_batch_size, self.max_seq_len, self.dtype = max_batch_size, max_seq_len, dtype
        self.states: Dict[str, dict] = {}
        self._slot = 0

    def allocate_sequence(self, seq_id, token_ids=None, num_tokens=0):
        s = self._slot
        self._slot += 1
        assert s < self.max_batch_size, "Exceeded max_batch_size"
        self.k[:, s].zero_()
        self.v[:, s].zero_()
        self.states[seq_id] = {"slot": s, "num_tokens": 0, "token_ids": list(token_ids or [])}
        return 0

    def begin_forward(self, seq_ids, ntoks, offsets=None):
        for sid, n in zip(seq_ids, ntoks):
            assert self.states[sid]["num_tokens"] + n <= self.max_seq_len
        return _ContigCtxRef(self, list(seq_ids), list(ntoks), offsets)

    def end_forward(self, ctx):
        for b in range(ctx.batch_size):
            self.states[ctx.seq_ids[b]]["num_tokens"] += ctx.new_token_counts[b]

    def release_sequence(self, seq_id):
        if seq_id in self.states:
            del self.states[seq_id]
            if not self.states:
                self._slot = 0


class _ContigCtxRef:
    def __init__(self, cache: ContiguousRef, seq_ids, new_token_counts, input_offsets):
        self.cache = cache
        self.seq_ids = seq_ids
        self.new_token_counts = new_token_counts
        self.input_offsets = input_offsets or [0] * len(seq_ids)
        self.batch_size = B = len(seq_ids)
        self.slots = [cache.states[s]["slot"] for s in seq_ids]
        self.start_positions = [cache.states[s]["num_tokens"] for s in seq_ids]
        self.seq_lens = [self.start_positions[i] + new_token_counts[i] for i in range(B)]
        self.max_kv_len = max(self.seq_lens) if self.seq_lens else 0
        self._is_decode = all(n == 1 for n in new_token_counts)
        self._iw = max(o + n for o, n in zip(self.input_offsets, new_token_counts)) if B else 1
        self._pos = position_ids(self.start_positions, new_token_counts, self.input_offsets)
        if self._is_decode and B:
            self._d_batch = torch.arange(B)
            self._d_pos = torch.tensor(self.start_positions, dtype=torch.long)
        self._mask = build_causal_mask(B, self._iw, self.start_positions, new_token_counts,
                                       self.input_offsets, self.seq_lens, self.max_kv_len, cache.dtype)

    def get_position_ids(self, S):
        return position_ids(self.start_positions, self.new_token_counts, self.input_offsets, S)

    def get_start_pos(self, idx=0):
        return self.start_positions[idx]

    def attend(self, layer_idx, q, k_new, v_new, n_heads, n_kv_heads):
        """kv_cache.py:297-322; like the reference, the pool is indexed by batch row b,
        not by the sequence's slot (:302, :309)."""
        B, S, _, D = q.shape
        pool = self.cache
        if self._is_decode:
            pool.k[layer_idx, self._d_batch, self._d_pos] = k_new[:, 0]
            pool.v[layer_idx, self._d_batch, self._d_pos] = v_new[:, 0]
        else:
            for b in range(B):
                o, n, s = self.input_offsets[b], self.new_token_counts[b], self.start_positions[b]
                if n > 0:
                    pool.k[layer_idx, b, s:s + n] = k_new[b, o:o + n]
                    pool.v[layer_idx, b, s:s + n] = v_new[b, o:o + n]
        kv = self.max_kv_len
        k_t = pool.k[layer_idx, :B, :kv].transpose(1, 2).contiguous()
        v_t = pool.v[layer_idx, :B, :kv].transpose(1, 2).contiguous()
        q_t = q.transpose(1, 2)
        mask = self._mask
        if mask is not None:
            mask = mask[:, :, :S, :kv].to(dtype=q.dtype)
        out = sdpa_gqa(q_t, k_t, v_t, attn_mask=mask, is_causal=(mask is None and S > 1))
        return out.transpose(1, 2).contiguous().reshape(B, S, -1)


# --------------------------------------------------------------------------------------
# paged backend, kv_cache.py:382-777
# --------------------------------------------------------------------------------------


class PagePoolRef:
    """kv_cache.py:382-442 with a deterministic free list (lowest id first).

    The reference pops from a Python set; which free id it returns is not part of
    the contract, so the oracle picks the lowest."""

    def __init__(self, num_layers, max_pages, page_size, num_kv_heads, head_dim, dtype=torch.float32):
        shape = (num_layers, max_pages, page_size, num_kv_heads, head_dim)
        self.k = torch.zeros(shape, dtype=dtype)
        self.v = torch.zeros(shape, dtype=dtype)
        self.max_pages = max_pages
        self.ref_count = [0] * max_pages
        self.tokens_used = [0] * max_pages
        self.ref_count[0] = 1
        self.free_set = set(range(1, max_pages))

    def alloc(self, n=1):
        if len(self.free_set) < n:
            return None
        out = []
        for _ in range(n):
            pid = min(self.free_set)
            self.free_set.remove(pid)
            self.ref_count[pid] = 1
            self.tokens_used[pid] = 0
            self.k[:, pid].zero_()
            self.v[:, pid].zero_()
            out.append(pid)
        return out

    def release(self, pid):
        if pid <= 0:
            return
        self.ref_count[pid] -= 1
        if self.ref_count[pid] <= 0:
            self.ref_count[pid] = 0
            self.tokens_used[pid] = 0
            self.free_set.add(pid)

    def add_ref(self, pid):
        self.ref_count[pid] += 1

    def is_shared(self, pid):
        return self.ref_count[pid] > 1

    def cow(self, pid):
        new = self.alloc(1)
        if new is None:
            return None
        d = new[0]
        self.k[:, d].copy_(self.k[:, pid])
        self.v[:, d].copy_(self.v[:, pid])
        self.tokens_used[d] = self.tokens_used[pid]
        return d

    @property
    def num_free(self):
        return len(self.free_set)


class _RNodeRef:
    __slots__ = ("children", "page_id", "ref", "last_access", "depth")

    def __init__(self, d=0):
        self.children: Dict[int, "_RNodeRef"] = {}
        self.page_id = -1
        self.ref = 0
        self.last_access = 0.0
        self.depth = d


class RadixTreeRef:
    """Per-token trie of kv_cache.py:453-531, with the reference's behaviour kept: match does not
    stop at an evicted interior page (:467), and LRU ties keep DFS pre-order (:507).

    stop_at_gap=True restates the build's decision instead: match returns pages only up to the
    first evicted page (a gap-free prefix); the walk, its access stamps and its invalidations are
    unchanged. The golden vectors pin the default; tests that compare the product's cache over
    whole serving runs use this mode.

    share_partial=True adds the build's partial-page sharing (not in the reference, whose tree
    holds pages at depths that are multiples of the page size only, :478-486): insert also hangs
    a last page of r < ps tokens on the node at its depth (nf*ps + r), and match returns, after
    its full pages, the page of the deepest such node on the walk that lies right after them
    (no gap before it), for a prefix of nf*ps + r tokens. Such a node with a released page is
    invalidated as the walk passes it, without ending the walk."""

    def __init__(self, ps, pool, stop_at_gap=False, share_partial=False):
        self.root = _RNodeRef()
        self.ps = ps
        self.pool = pool
        self._clock = 0
        self.stop_at_gap = stop_at_gap
        self.share_partial = share_partial

    def _now(self):
        self._clock += 1
        return float(self._clock)

    def match(self, tokens):
        node, pages, now = self.root, [], self._now()
        gap = False
        partial = None  # (page, tokens) of a partial page right after the pages so far
        for i, tok in enumerate(tokens):
            ch = node.children.get(tok)
            if ch is None:
                break
            node = ch
            node.last_access = now
            d = i + 1
            if d % self.ps == 0 and node.page_id < 0:
                gap = True
            if d % self.ps == 0 and node.page_id >= 0:
                if self.pool.ref_count[node.page_id] > 0:
                    if not (self.stop_at_gap and gap):
                        pages.append(node.page_id)
                        partial = None
                else:
                    node.page_id = -1
                    break
            elif d % self.ps and self.share_partial and node.page_id >= 0:
                if self.pool.ref_count[node.page_id] <= 0:
                    node.page_id = -1
                elif not gap and d // self.ps == len(pages):
                    partial = (node.page_id, d - len(pages) * self.ps)
        if partial is not None:
            return len(pages) * self.ps + partial[1], pages + [partial[0]]
        return len(pages) * self.ps, pages

    def insert(self, tokens, page_ids):
        node, pi, now = self.root, 0, self._now()
        for i, tok in enumerate(tokens):
            if tok not in node.children:
                node.children[tok] = _RNodeRef(i + 1)
            node = node.children[tok]
            node.last_access = now
            d = i + 1
            if d % self.ps == 0 and pi < len(page_ids):
                incoming = page_ids[pi]
                pi += 1
                if node.page_id < 0:
                    node.page_id = incoming
                    self.pool.add_ref(incoming)
        nf = len(tokens) // self.ps
        if self.share_partial and len(tokens) % self.ps and nf < len(page_ids) and node.page_id < 0:
            # the last, partial page (node is at depth len(tokens)); it starts unpinned:
            # pins that passed this token position before it held a page do not count
            node.page_id = page_ids[nf]
            node.ref = 0
            self.pool.add_ref(page_ids[nf])

    def add_refs(self, tokens, n=1):
        node = self.root
        for tok in tokens:
            ch = node.children.get(tok)
            if ch is None:
                break
            node = ch
            node.ref += n

    def dec_refs(self, tokens, n=1):
        node = self.root
        for tok in tokens:
            ch = node.children.get(tok)
            if ch is None:
                break
            node = ch
            node.ref = max(0, node.ref - n)

    def evict_lru(self, need):
        cands = []
        self._collect(self.root, cands)
        cands.sort(key=lambda x: x[0])
        freed = 0
        for _, nd, par, edge in cands:
            if freed >= need:
                break
            if nd.ref > 0:
                continue
            if nd.page_id >= 0:
                self.pool.release(nd.page_id)
                nd.page_id = -1
                freed += 1
            if not nd.children and par is not None:
                par.children.pop(edge, None)
        return freed

    def _collect(self, node, out, par=None, edge=-1):
        if node.page_id >= 0 and node.ref == 0:
            out.append((node.last_access, node, par, edge))
        for t, ch in list(node.children.items()):
            self._collect(ch, out, node, t)

    @property
    def cached_pages(self):
        c = [0]

        def _cnt(n):
            if n.page_id >= 0:
                c[0] += 1
            for ch in n.children.values():
                _cnt(ch)

        _cnt(self.root)
        return c[0]


@dataclass
class _SeqRef:
    seq_id: str
    block_table: List[int]
    num_tokens: int
    prefix_len: int
    token_ids: List[int] = field(default_factory=list)


class PagedRef:
    """FlashInferPagedKVCache + FlashInferCacheContext (kv_cache.py:534-777) on the CPU,
    FlashInfer replaced by fp32 SDPA over the gathered pages."""

    def __init__(self, num_layers, max_pages, page_size, num_kv_heads, head_dim,
                 dtype=torch.float32, enable_prefix_caching=True, stop_at_gap=False, share_partial_pages=False):
        """share_partial_pages: the build's partial-page sharing (RadixTreeRef): released
        sequences also cache their last partial page, prompts of any length are matched,
        and a prefix ending inside a page shares that page (its first write copies it)."""
        self.ps = page_size
        self.pool = PagePoolRef(num_layers, max_pages, page_size, num_kv_heads, head_dim, dtype)
        self.tree = (RadixTreeRef(page_size, self.pool, stop_at_gap, share_partial_pages)
                     if enable_prefix_caching else None)
        self.share_partial_pages = share_partial_pages
        self.seqs: Dict[str, _SeqRef] = {}
        self.max_pages = max_pages

    def _alloc(self, n):
        pages = self.pool.alloc(n)
        if pages:
            return pages
        if self.tree:
            if self.tree.evict_lru(n) > 0:
                pages = self.pool.alloc(n)
                if pages:
                    return pages
        raise RuntimeError(f"KV OOM: need {n}, free {self.pool.num_free}")

    def allocate_sequence(self, seq_id, token_ids=None, num_tokens=0):
        tids = token_ids or []
        total = len(tids) if tids else num_tokens
        plen, ppages = 0, []
        if self.tree and len(tids) >= (1 if self.share_partial_pages else self.ps):
            plen, ppages = self.tree.match(tids)
            for p in ppages:
                self.pool.add_ref(p)
            if ppages:
                self.tree.add_refs(tids[:plen])
        st = _SeqRef(seq_id, list(ppages), plen, plen, list(tids))
        need = math.ceil(total / self.ps) - len(ppages)  # = ceil((total - plen) / ps) for whole pages
        if need > 0:
            st.block_table.extend(self._alloc(need))
        self.seqs[seq_id] = st
        return plen

    def extend_sequence(self, seq_id, num_new=1):
        st = self.seqs[seq_id]
        need = math.ceil((st.num_tokens + num_new) / self.ps)
        if need > len(st.block_table):
            st.block_table.extend(self._alloc(need - len(st.block_table)))

    def begin_forward(self, seq_ids, ntoks, offsets=None):
        for s, n in zip(seq_ids, ntoks):
            self.extend_sequence(s, n)
        return _PagedCtxRef(self, list(seq_ids), list(ntoks), offsets)

    def end_forward(self, ctx):
        for b in range(ctx.batch_size):
            self.seqs[ctx.seq_ids[b]].num_tokens += ctx.new_token_counts[b]

    def release_sequence(self, seq_id):
        if seq_id not in self.seqs:
            return
        st = self.seqs[seq_id]
        if self.tree and st.token_ids:
            if self.share_partial_pages:  # the full pages and the last, partial one
                n = min(st.num_tokens, len(st.token_ids))
                if n:
                    self.tree.insert(st.token_ids[:n], st.block_table[:math.ceil(n / self.ps)])
            else:
                nf = st.num_tokens // self.ps
                if nf:
                    self.tree.insert(st.token_ids[:nf * self.ps], st.block_table[:nf])
            if st.prefix_len:
                self.tree.dec_refs(st.token_ids[:st.prefix_len])
        for p in st.block_table:
            self.pool.release(p)
        del self.seqs[seq_id]

    def append_token_ids(self, seq_id, ids):
        if seq_id in self.seqs:
            self.seqs[seq_id].token_ids.extend(ids)

    def logical_kv(self, seq_id, layer):
        """[num_tokens, Hkv, D] K and V of a sequence, read through its block table."""
        st = self.seqs[seq_id]
        n = st.num_tokens
        rows_k = [self.pool.k[layer, st.block_table[t // self.ps], t % self.ps] for t in range(n)]
        rows_v = [self.pool.v[layer, st.block_table[t // self.ps], t % self.ps] for t in range(n)]
        if not rows_k:
            shp = self.pool.k.shape[3:]
            return torch.zeros((0,) + tuple(shp)), torch.zeros((0,) + tuple(shp))
        return torch.stack(rows_k), torch.stack(rows_v)


class _PagedCtxRef:
    def __init__(self, cache: PagedRef, seq_ids, new_token_counts, input_offsets):
        self.cache = cache
        self.seq_ids = seq_ids
        self.new_token_counts = new_token_counts
        self.input_offsets = input_offsets or [0] * len(seq_ids)
        self.batch_size = B = len(seq_ids)
        pool, ps = cache.pool, cache.ps
        self.start_positions = [cache.seqs[s].num_tokens for s in seq_ids]
        self.seq_lens = [self.start_positions[i] + new_token_counts[i] for i in range(B)]
        self._is_decode = all(n == 1 for n in new_token_counts)
        self.cow_events: List[Tuple[int, int]] = []
        self._write_info: List[List[Tuple[int, int]]] = []
        for b in range(B):
            st = cache.seqs[seq_ids[b]]
            info = []
            for t in range(new_token_counts[b]):
                ap = st.num_tokens + t
                pi, sl = ap // ps, ap % ps
                if pi >= len(st.block_table):
                    info.append((0, 0))
                    continue
                pid = st.block_table[pi]
                if pool.is_shared(pid):
                    np_ = pool.cow(pid)
                    if np_ is None and cache.share_partial_pages and cache.tree and cache.tree.evict_lru(1) > 0:
                        # the build's extended mode: a copy may evict a cached page, like any
                        # allocation (kv_cache.py:760-768); if that released the page's other
                        # reference, the page is written in place
                        np_ = pool.cow(pid) if pool.is_shared(pid) else -1
                    if np_ is None:
                        raise RuntimeError("KV OOM during CoW")
                    if np_ >= 0:
                        self.cow_events.append((pid, np_))
                        st.block_table[pi] = np_
                        pool.release(pid)
                        pid = np_
                info.append((pid, sl))
                pool.tokens_used[pid] = max(pool.tokens_used[pid], sl + 1)
            self._write_info.append(info)
        self.indptr, self.indices, self.lpl = plan_csr(
            [cache.seqs[s].block_table for s in seq_ids], self.seq_lens, ps)

    def get_position_ids(self, S):
        return position_ids(self.start_positions, self.new_token_counts, self.input_offsets, S)

    def get_start_pos(self, idx=0):
        return self.start_positions[idx]

    def slot_mapping(self, S):
        """[B*S] slot ids for the input grid (pad rows -1): the write plan as one array."""
        sm = np.full((self.batch_size, S), -1, np.int64)
        for b in range(self.batch_size):
            o = self.input_offsets[b]
            for t, (pid, sl) in enumerate(self._write_info[b]):
                sm[b, o + t] = pid * self.cache.ps + sl
        return sm.reshape(-1)

    def attend(self, layer_idx, q, k_new, v_new, n_heads, n_kv_heads):
        B, S = q.shape[0], q.shape[1]
        pool, ps = self.cache.pool, self.cache.ps
        for b in range(B):
            o, n = self.input_offsets[b], self.new_token_counts[b]
            for t in range(n):
                pid, sl = self._write_info[b][t]
                pool.k[layer_idx, pid, sl] = k_new[b, o + t]
                pool.v[layer_idx, pid, sl] = v_new[b, o + t]
        k_rows = pool.k[layer_idx].reshape(-1, *pool.k.shape[3:])
        v_rows = pool.v[layer_idx].reshape(-1, *pool.v.shape[3:])
        qs = [q[b, self.input_offsets[b]:self.input_offsets[b] + self.new_token_counts[b]] for b in range(B)]
        outs = paged_attention_ref(qs, k_rows, v_rows, ps, self.indptr, self.indices, self.lpl,
                                   self.new_token_counts)
        out = torch.zeros(B, S, q.shape[2] * q.shape[3], dtype=torch.float32)
        for b in range(B):
            o, n = self.input_offsets[b], self.new_token_counts[b]
            if n:
                out[b, o:o + n] = outs[b].reshape(n, -1)
        return out


def timed_contiguous_decode(num_steps=64, prefill=512, Hq=32, Hkv=8, D=128, seed=0, warmup=8,
                            repeats=5, threads=None):
    """The config-1 CPU baseline: fp32, B=1, prefill `prefill` tokens of N(0,1) K/V, then
    `num_steps` decode steps through ContiguousRef, timed at contexts prefill+1 ..
    prefill+num_steps (the `warmup` steps run first on a separate cache of the same
    shape). Returns (median seconds per step over `repeats`, threads used)."""
    if threads is not None:
        torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(seed)
    cache = ContiguousRef(1, 1, prefill + num_steps, Hkv, D)
    warm = ContiguousRef(1, 1, prefill + warmup, Hkv, D)
    times = []
    for _ in range(repeats):
        for c in (warm, cache):
            c.release_sequence("s")
            c.allocate_sequence("s")
            c.k[0, 0, :prefill] = torch.randn(prefill, Hkv, D, generator=g)
            c.v[0, 0, :prefill] = torch.randn(prefill, Hkv, D, generator=g)
            c.states["s"]["num_tokens"] = prefill
        qs = torch.randn(warmup + num_steps, 1, 1, Hq, D, generator=g) / math.sqrt(D)
        ks = torch.randn(warmup + num_steps, 1, 1, Hkv, D, generator=g)
        vs = torch.randn(warmup + num_steps, 1, 1, Hkv, D, generator=g)
        for i in range(warmup + num_steps):
            c = warm if i < warmup else cache
            if i == warmup:
                t0 = time.perf_counter()
            ctx = c.begin_forward(["s"], [1])
            ctx.attend(0, qs[i], ks[i], vs[i], Hq, Hkv)
            c.end_forward(ctx)
        assert cache.states["s"]["num_tokens"] == prefill + num_steps
        times.append((time.perf_counter() - t0) / num_steps)
    return float(np.median(times)), torch.get_num_threads()
