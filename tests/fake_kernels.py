"""CPU stand-in for nanoslg_amd.kernels, used only to test the host layer
(bookkeeping, plans, copy-on-write order) without a GPU. It implements the
same functions with plain torch indexing and the oracle's fp32 attention.
The product never uses it: nanoslg_amd.kv_cache gets it only when a test
passes it in explicitly."""
from __future__ import annotations

import math

import torch

from oracle import kv_oracle

CALLS = []  # (name, summary) log of launches, for tests that count them


class Workspace:
    def __init__(self, device, nbytes=0):
        self.device = device

    def get(self, nbytes):
        return None


def append_kv(k_new, v_new, slot_mapping, k_pool, v_pool):
    CALLS.append(("append_kv", int(slot_mapping.numel())))
    Hkv, D = k_pool.shape[-2], k_pool.shape[-1]
    kr = k_new.reshape(-1, Hkv, D)
    vr = v_new.reshape(-1, Hkv, D)
    kp = k_pool.view(-1, Hkv, D)
    vp = v_pool.view(-1, Hkv, D)
    for i, s in enumerate(slot_mapping.tolist()):
        if 0 <= s < kp.shape[0]:
            kp[s] = kr[i]
            vp[s] = vr[i]


def zero_pages(k_pool, v_pool, page_ids):
    CALLS.append(("zero_pages", int(page_ids.numel())))
    for p in page_ids.tolist():
        if 0 <= p < k_pool.shape[1]:
            k_pool[:, p] = 0
            v_pool[:, p] = 0


def copy_pages(k_pool, v_pool, src_ids, dst_ids):
    CALLS.append(("copy_pages", int(src_ids.numel())))
    for s, d in zip(src_ids.tolist(), dst_ids.tolist()):
        k_pool[:, d] = k_pool[:, s]
        v_pool[:, d] = v_pool[:, s]


def gather_kv(k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, max_len):
    ps = k_layer.shape[1]
    kr = k_layer.reshape(-1, *k_layer.shape[2:]).numpy()
    vr = v_layer.reshape(-1, *v_layer.shape[2:]).numpy()
    k = kv_oracle.gather_rows(kr, ps, kv_indptr.numpy(), kv_indices.numpy(), kv_last_page_len.numpy(), max_len)
    v = kv_oracle.gather_rows(vr, ps, kv_indptr.numpy(), kv_indices.numpy(), kv_last_page_len.numpy(), max_len)
    return torch.from_numpy(k), torch.from_numpy(v)


def _attend(q_list, qo_lens, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, sm_scale):
    ps = k_layer.shape[1]
    kr = k_layer.reshape(-1, *k_layer.shape[2:])
    vr = v_layer.reshape(-1, *v_layer.shape[2:])
    return kv_oracle.paged_attention_ref(q_list, kr, vr, ps, kv_indptr.tolist(), kv_indices.tolist(),
                                         kv_last_page_len.tolist(), qo_lens, sm_scale)


def paged_decode(q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                 sm_scale=None, out=None, workspace=None, groups=None):
    CALLS.append(("paged_decode", int(q.shape[0])))
    B = q.shape[0]
    outs = _attend([q[b:b + 1] for b in range(B)], [1] * B, k_layer, v_layer, kv_indptr, kv_indices,
                   kv_last_page_len, sm_scale)
    res = torch.stack([o[0] for o in outs]).to(q.dtype)
    if out is not None:
        out.copy_(res)
        return out
    return res


def paged_prefill(q, qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len,
                  sm_scale=None, out=None, workspace=None, q_rows=None, grid_width=0):
    CALLS.append(("paged_prefill", int(total_q)))
    qo = qo_indptr.tolist()
    B = len(qo) - 1
    if q_rows is not None:  # the padded grid: rows of each sequence contiguous in its block, pads zero
        rows = q_rows[:int(total_q)].long()
        assert q.shape[0] == B * grid_width
        for b in range(B):
            r = rows[qo[b]:qo[b + 1]].tolist()
            assert r == list(range(r[0], r[0] + len(r))) if r else True
            assert all(b * grid_width <= x < (b + 1) * grid_width for x in r)
        res = paged_prefill(q.index_select(0, rows), qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr,
                            kv_indices, kv_last_page_len, sm_scale)
        grid = q.new_zeros(q.shape)
        grid.index_copy_(0, rows, res)
        if out is not None:
            out.copy_(grid)
            return out
        return grid
    qs = [q[qo[b]:qo[b + 1]] for b in range(B)]
    outs = _attend(qs, [qo[b + 1] - qo[b] for b in range(B)], k_layer, v_layer, kv_indptr, kv_indices,
                   kv_last_page_len, sm_scale)
    res = torch.cat(outs, 0).to(q.dtype) if outs else q.new_zeros(0, q.shape[1], q.shape[2])
    if out is not None:
        out[:res.shape[0]].copy_(res)
        return out
    return res


def _append_kv_layer(k_new, v_new, slot_mapping, k_layer, v_layer):
    append_kv(k_new, v_new, slot_mapping, k_layer, v_layer)


FUSED_PREFILL_APPEND = True  # False: decline the one-launch write + attention, as for fp32 pools on the GPU


def _paged_prefill_append_layer(q, qo_indptr, total_q, max_q, k_new, v_new, k_layer, v_layer, kv_indptr,
                                kv_indices, kv_last_page_len, workspace, q_rows=None, grid_width=0):
    """The contract of nslg_paged_prefill_append, by its own rule (no slot mapping):
    token t of sequence b, row qo_indptr[b] + t (or q_rows[qo_indptr[b]] + t) of
    k_new / v_new, goes to position L_b - n_b + t through the block table (slot 0 of
    page 0 past the table); then paged_prefill."""
    if not FUSED_PREFILL_APPEND:
        return None
    CALLS.append(("paged_prefill_append", int(total_q)))
    ps, Hkv, D = k_layer.shape[1], k_layer.shape[2], k_layer.shape[3]
    kr, vr = k_new.reshape(-1, Hkv, D), v_new.reshape(-1, Hkv, D)
    kp, vp = k_layer.view(-1, Hkv, D), v_layer.view(-1, Hkv, D)
    qo, ip, idx, lpl = (t.tolist() for t in (qo_indptr, kv_indptr, kv_indices, kv_last_page_len))
    rows = None if q_rows is None else q_rows.tolist()
    for b in range(len(ip) - 1):
        n, npg = qo[b + 1] - qo[b], ip[b + 1] - ip[b]
        L = (npg - 1) * ps + lpl[b] if npg > 0 else 0
        r0 = qo[b] if rows is None else (rows[qo[b]] if n > 0 else 0)
        for t in range(n):
            pos = L - n + t
            pi = pos // ps
            pid = idx[ip[b] + pi] if pi < npg else 0
            if not 0 <= pid < k_layer.shape[0]:
                continue
            slot = pid * ps + pos % ps if pi < npg else 0
            kp[slot] = kr[r0 + t]
            vp[slot] = vr[r0 + t]
    return _paged_prefill_layer(q, qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr, kv_indices,
                                kv_last_page_len, workspace, q_rows=q_rows, grid_width=grid_width)


def _paged_prefill_layer(q, qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len,
                         workspace, q_rows=None, grid_width=0):
    return paged_prefill(q, qo_indptr, total_q, max_q, k_layer, v_layer, kv_indptr, kv_indices, kv_last_page_len,
                         workspace=workspace, q_rows=q_rows, grid_width=grid_width)


class DecodeLaunch:
    """Per-forward append + decode, as nanoslg_amd.kernels.DecodeLaunch, from the
    functions above."""

    def __init__(self, k_pool, v_pool, slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages,
                 num_qo_heads, workspace=None, sm_scale=None, groups=None):
        CALLS.append(("DecodeLaunch", groups))
        self.k_pool, self.v_pool = k_pool, v_pool
        self.args = (slot_mapping, kv_indptr, kv_indices, kv_last_page_len, total_pages)
        self.sm_scale = sm_scale

    def __call__(self, layer, q, k_new, v_new, rope=None):
        if q.dim() == 4:  # [B, 1, Hq, D] -> [B, 1, Hq * D]
            return self(layer, q[:, 0], k_new, v_new, rope).reshape(q.shape[0], 1, -1)
        slots, indptr, indices, lpl, total = self.args
        k_layer, v_layer = self.k_pool[layer], self.v_pool[layer]
        if rope is None:
            # the product's launch writes row b at the slot of sequence b's last token
            # through its block table (nslg_paged_decode_append): it must be the
            # plan's slot for that row
            ps = k_layer.shape[1]
            ip, ix, lp = (t.tolist() for t in (indptr, indices, lpl))
            table_slots = []
            for b in range(len(ip) - 1):
                n = ip[b + 1] - ip[b]
                L = (n - 1) * ps + min(max(lp[b], 1), ps) if n > 0 else 0
                table_slots.append(ix[ip[b] + (L - 1) // ps] * ps + (L - 1) % ps if L > 0 else -1)
            assert table_slots == slots.tolist(), (table_slots, slots.tolist())
            append_kv(k_new, v_new, slots, k_layer, v_layer)
        else:
            cos, sin, pos = rope
            q = rope_append(q, k_new, v_new, pos, slots, cos, sin, k_layer, v_layer)
        return paged_decode(q, k_layer, v_layer, indptr, indices, lpl, total, sm_scale=self.sm_scale)


def rope_append(q, k_new, v_new, positions, slot_mapping, cos, sin, k_pool, v_pool, q_out=None):
    """As nanoslg_amd.kernels.rope_append: the oracle's eager rotation, then append."""
    CALLS.append(("rope_append", int(positions.numel())))
    Hq, D = q.shape[-2], q.shape[-1]
    Hkv = k_pool.shape[-2]
    T = positions.numel()
    pos = positions.reshape(1, T).long()
    qr, kr = kv_oracle.rope_forward_ref(q.reshape(1, T, Hq, D), k_new.reshape(1, T, Hkv, D), cos.float(),
                                        sin.float(), pos)
    append_kv(kr.reshape(T, Hkv, D), v_new.reshape(T, Hkv, D), slot_mapping, k_pool, v_pool)
    out = qr.reshape(q.shape)
    if q_out is not None:
        q_out.copy_(out)
        return q_out
    return out


def decode_plan_step(kv_indptr, kv_indices, kv_last_page_len, new_page, page_size, num_new, k_pool=None,
                     v_pool=None):
    """As nanoslg_amd.kernels.decode_plan_step, in plain Python on the CPU."""
    CALLS.append(("decode_plan_step", int(kv_indptr.numel() - 1)))
    ip, idx, lpl = kv_indptr.tolist(), kv_indices.tolist(), kv_last_page_len.tolist()
    out_ip, out_idx, out_lpl, slots, pos, new = [0], [], [], [], [], []
    for b in range(len(ip) - 1):
        seg = idx[ip[b]:ip[b + 1]]
        last = min(max(lpl[b] if seg else page_size, 1), page_size)
        if last == page_size:
            page = int(new_page[b]) if new_page[b] >= 0 else 0
            seg = seg + [page]
            new.append(page)
            last = 1
        else:
            page = seg[-1]
            last += 1
        out_idx += seg
        out_ip.append(len(out_idx))
        out_lpl.append(last)
        slots.append(page * page_size + last - 1)
        pos.append((len(seg) - 1) * page_size + last - 1)
    if k_pool is not None and new:
        ids = torch.tensor(new, dtype=torch.long)
        k_pool[:, ids] = 0
        v_pool[:, ids] = 0
    t = lambda x: torch.tensor(x, dtype=torch.int32)  # noqa: E731
    return t(out_ip), t(out_idx), t(out_lpl), t(slots), t(pos), t(new)


# the stand-in groups decode rows of any pool dtype (grouping does not change results)
GROUPED_DECODE_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


class DecodeGroups:
    """As nanoslg_amd.kernels.DecodeGroups (the grouping does not change results)."""

    def __init__(self, batch, members, prefix_pages, device, seq_group_slot=None):
        self.num_groups = len(members)
        self.members = [list(map(int, m)) for m in members]
        self.prefix_pages = list(map(int, prefix_pages))
        self.seq_group_slot = seq_group_slot


def _block_table_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch_total, kv_indptr,
                     kv_indices, total_pages, B):
    """As nanoslg_amd.kernels._block_table_csr, in plain Python on the CPU."""
    CALLS.append(("block_table_csr", int(B)))
    row, have, syn = row_offset.tolist(), pages_have.tolist(), synced.tolist()
    pip, pat, ip = patch_indptr.tolist(), patch.tolist(), kv_indptr.tolist()
    cap = tables.numel()
    for b in range(B):
        for i in range(max(have[b], ip[b + 1] - ip[b])):
            pid = 0
            if i < have[b]:
                at = row[b] + i
                inside = 0 <= row[b] and at < cap
                if i >= syn[b]:
                    k = pip[b] + i - syn[b]
                    pid = pat[k] if 0 <= k < patch_total else 0
                    if inside:
                        tables[at] = pid
                elif inside:
                    pid = int(tables[at])
            if i < ip[b + 1] - ip[b] and ip[b] + i < total_pages:
                kv_indices[ip[b] + i] = pid


def _forward_plan(kv_indptr, kv_indices, start, new_tokens, input_offsets, pages_allocated, B, iw, page_size, T,
                  out=None):
    """As nanoslg_amd.kernels._forward_plan, in plain Python on the CPU."""
    CALLS.append(("forward_plan", T))
    ip, idx = kv_indptr.tolist(), kv_indices.tolist()
    st, n, off, have = start.tolist(), new_tokens.tolist(), input_offsets.tolist(), pages_allocated.tolist()
    slot, pos, rows, qo = [-1] * (B * iw), [0] * (B * iw), [0] * T, [0]
    for b in range(B):
        for t in range(max(n[b], 0)):
            ap = st[b] + t
            pi = ap // page_size
            r = b * iw + off[b] + t
            slot[r] = idx[ip[b] + pi] * page_size + ap - pi * page_size if pi < have[b] else 0
            pos[r] = ap
            rows[qo[-1] + t] = r
        qo.append(qo[-1] + max(n[b], 0))
    flat = torch.tensor(slot + pos + rows + qo, dtype=torch.int32)
    if out is not None:  # the outputs are consecutive views of the caller's buffer
        assert out.dtype == torch.int32 and out.numel() >= flat.numel()
        out[:flat.numel()].copy_(flat)
        flat = out[:flat.numel()]
    return tuple(flat.split([B * iw, B * iw, T, B + 1]))


def _forward_plan_csr_at(tables, buf, mid, npatch, total_pages, B, iw, page_size, T, out):
    """As nanoslg_amd.kernels._forward_plan_csr_at: the inputs found at the same places
    of the upload buffer, then _forward_plan_csr."""
    m = buf[mid:]
    start, n, off, _, row, have, syn = (m[i * B:(i + 1) * B] for i in range(7))
    pip = m[7 * B:8 * B + 1]
    patch = m[8 * B + 1:8 * B + 1 + max(npatch, 1)]
    idx_at = mid + 8 * B + 1 + max(npatch, 1)
    idx = buf[idx_at:idx_at + max(total_pages, 1)]
    return _forward_plan_csr(tables, row, have, syn, pip, patch, npatch, buf[:B + 1], idx, total_pages, start, n, off,
                             B, iw, page_size, T, out)


def _forward_plan_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch_total, kv_indptr, kv_indices,
                      total_pages, start, new_tokens, input_offsets, B, iw, page_size, T, out):
    """As nanoslg_amd.kernels._forward_plan_csr: the two launches it fuses, in order."""
    _block_table_csr(tables, row_offset, pages_have, synced, patch_indptr, patch, patch_total, kv_indptr, kv_indices,
                     total_pages, B)
    return _forward_plan(kv_indptr, kv_indices, start, new_tokens, input_offsets, pages_have, B, iw, page_size, T,
                         out=out)
