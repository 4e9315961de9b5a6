"""Fused rotary embedding + K/V append on the GPU (nslg_rope_append) against the
oracle's restatement of the model's eager rotation (nanoslg/models.py:69-103):
rotated q and the pool's K rows bit-exact, V rows copied, padding and
out-of-range slots not written. At the cache API, attention_forward (the fused
path) gives the same outputs and pool bytes as the model's own sequence
(positions, eager rotation, attend), bit for bit."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _oracle_rows(q, k, cos, sin, pos):
    """Oracle rotation of row-major [T, H, D] q and k at int positions [T] (CPU)."""
    T = pos.numel()
    qr, kr = O.rope_forward_ref(q.reshape(1, T, *q.shape[-2:]), k.reshape(1, T, *k.shape[-2:]), cos, sin,
                                pos.reshape(1, T).long())
    return qr.reshape(q.shape), kr.reshape(k.shape)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("Hq,Hkv,D", [(32, 8, 128), (8, 8, 64), (16, 2, 256), (4, 1, 128)])
def test_rope_append_bit_exact(dtype, Hq, Hkv, D):
    _log(f"rope_append dtype={dtype} Hq={Hq} Hkv={Hkv} D={D}")
    from nanoslg_amd import kernels as K
    g = torch.Generator().manual_seed(D + Hq)
    T, P, ps, R = 300, 64, 16, 40000
    cos, sin = O.rope_tables(D, R, 500000.0, LLAMA3)
    q = torch.randn(T, Hq, D, generator=g).to(dtype)
    kv = torch.randn(T, 3, Hkv, D, generator=g).to(dtype)  # k and v as strided views of one buffer
    k, v = kv[:, 0], kv[:, 2]
    pos = torch.randint(0, R, (T,), generator=g, dtype=torch.int32)
    pos[:4] = torch.tensor([0, 1, R - 1, R - 2], dtype=torch.int32)
    slots = torch.from_numpy(np.random.default_rng(D).permutation(P * ps)[:T].astype(np.int32))
    slots[5:9] = -1                    # padding rows
    slots[9] = P * ps + 3              # past the pool: rejected on the device
    k_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    v_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    qr, kr = _oracle_rows(q, k, cos, sin, pos)
    k_exp, v_exp = k_pool.clone().view(-1, Hkv, D), v_pool.clone().view(-1, Hkv, D)
    ok = (slots >= 0) & (slots < P * ps)
    k_exp[slots[ok].long()] = kr[ok]
    v_exp[slots[ok].long()] = v[ok]

    kd, vd = k_pool.to(DEV), v_pool.to(DEV)
    kvd = kv.to(DEV)
    out = K.rope_append(q.to(DEV), kvd[:, 0], kvd[:, 2], pos.to(DEV), slots.to(DEV), cos.to(DEV), sin.to(DEV),
                        kd, vd)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), qr)
    assert torch.equal(kd.cpu().view(-1, Hkv, D), k_exp)
    assert torch.equal(vd.cpu().view(-1, Hkv, D), v_exp)

    # in place on q (q_out = q), and q rows at a stride wider than Hq*D
    qwide = torch.zeros(T, Hq + 2, D, dtype=dtype)
    qwide[:, :Hq] = q
    qd = qwide.to(DEV)[:, :Hq]
    res = K.rope_append(qd, kvd[:, 0], kvd[:, 2], pos.to(DEV), slots.to(DEV), cos.to(DEV), sin.to(DEV), kd, vd,
                        q_out=qd)
    torch.cuda.synchronize()
    assert res.data_ptr() == qd.data_ptr()
    assert torch.equal(qd.cpu(), qr)
    assert torch.equal(qwide.to(DEV)[:, Hq:].cpu(), torch.zeros(T, 2, D, dtype=dtype))


def test_rope_append_argument_errors():
    from nanoslg_amd import kernels as K
    cos, sin = O.rope_tables(128, 16, 10000.0)
    q = torch.zeros(4, 32, 128, dtype=torch.float16, device=DEV)
    k = torch.zeros(4, 8, 128, dtype=torch.float16, device=DEV)
    pool = torch.zeros(8, 16, 8, 128, dtype=torch.float16, device=DEV)
    pos = torch.zeros(4, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        K.rope_append(q, k, k, pos[:3], pos, cos.to(DEV), sin.to(DEV), pool, pool.clone())
    with pytest.raises(TypeError):
        K.rope_append(q.float(), k, k, pos, pos, cos.to(DEV), sin.to(DEV), pool, pool.clone())
    with pytest.raises(ValueError):
        K.rope_append(q, k, k, pos, pos, cos.to(DEV)[:, :64], sin.to(DEV)[:, :64], pool, pool.clone())
    with pytest.raises(ValueError):
        K.rope_append(q, k, k, pos.cpu(), pos, cos.to(DEV), sin.to(DEV), pool, pool.clone())


@pytest.mark.parametrize("backend", ["paged", "contiguous"])
def test_attention_forward_fused_equals_model_sequence(backend):
    """attention_forward (rotation fused into the cache write) against the model's
    sequence on a second cache: get_position_ids, eager rotation, attend. Ragged
    prefill with offsets, then decode steps (device-planned ones included): outputs
    and pool bytes identical."""
    _log(f"attention_forward fused vs eager, backend={backend}")
    from nanoslg_amd import kv_cache as KC
    L, HQ, HKV, D = 2, 32, 8, 128
    g = torch.Generator().manual_seed(5)
    cos, sin = O.rope_tables(D, 4096, 500000.0, LLAMA3)
    cos_d, sin_d = cos.to(DEV), sin.to(DEV)
    cfg = dict(num_layers=L, num_kv_heads=HKV, num_qo_heads=HQ, head_dim=D, page_size=16, max_pages=512,
               dtype=torch.float16, device=DEV, backend=backend, max_batch_size=4, max_seq_len=1024)
    cls = KC.PagedKVCache if backend == "paged" else KC.ContiguousKVCache
    a, b = cls(KC.KVCacheConfig(**cfg)), cls(KC.KVCacheConfig(**cfg))
    ids = ["x", "y", "z", "w"]
    lens = [300, 517, 64, 129]
    for m in (a, b):
        for s, n in zip(ids, lens):
            m.allocate_sequence(s, num_tokens=n)
    steps = [(lens, [0, 3, 1, 0])] + [([1, 1, 1, 1], None)] * 20
    for ntok, offs in steps:
        offs = offs or [0] * 4
        S = max(o + n for o, n in zip(offs, ntok))
        q = torch.randn(4, S, HQ, D, generator=g).half().to(DEV)
        k = torch.randn(4, S, HKV, D, generator=g).half().to(DEV)
        v = torch.randn(4, S, HKV, D, generator=g).half().to(DEV)
        ca, cb = a.begin_forward(ids, ntok, offs), b.begin_forward(ids, ntok, offs)
        for layer in range(L):
            oa = KC.attention_forward(q, k, v, layer, HQ, HKV, cos_d, sin_d, ca)
            pos = cb.get_position_ids(S).cpu()
            qr, kr = O.rope_forward_ref(q.cpu(), k.cpu(), cos, sin, pos)
            ob = cb.attend(layer, qr.to(DEV), kr.to(DEV), v, HQ, HKV)
            torch.cuda.synchronize()
            for bi in range(4):
                rows = slice(offs[bi], offs[bi] + ntok[bi])
                assert torch.equal(oa[bi, rows], ob[bi, rows])
        a.end_forward(ca)
        b.end_forward(cb)
    if backend == "paged":
        assert torch.equal(a.pool.k, b.pool.k) and torch.equal(a.pool.v, b.pool.v)
    else:
        assert torch.equal(a.k, b.k) and torch.equal(a.v, b.v)


@pytest.mark.parametrize("grouped", [False, True])
@pytest.mark.parametrize("Hq,Hkv,D,ps", [(32, 8, 128, 16), (8, 8, 64, 16), (16, 2, 256, 16), (16, 4, 128, 5),
                                         (4, 1, 64, 1)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_decode_rope_append_equals_rope_append_then_decode(dtype, Hq, Hkv, D, ps, grouped):
    """nslg_paged_decode_rope_append (q rotated as the decode loads it, the new K rows
    rotated by the chunks that write them) against nslg_rope_append into the new
    slots followed by nslg_paged_decode of the rotated q, on copies of one pool:
    outputs and pool bytes bit-identical. Positions anywhere in the tables (one past
    the end, clamped); with `grouped`, sequences 0..3 share their first pages as a
    prefix group (each member's q rotated at its own position)."""
    _log(f"decode rope append dtype={dtype} Hq={Hq} Hkv={Hkv} D={D} ps={ps} grouped={grouped}")
    from nanoslg_amd import kernels as K
    G = Hq // Hkv
    B, R, prefix = 6, 4096, 8
    members = list(range(min(4, 16 // G))) if grouped else []
    rng = np.random.default_rng(1000 * D + 10 * Hq + ps + grouped)
    g = torch.Generator().manual_seed(int(rng.integers(1 << 30)))
    lens = [int(rng.integers((prefix + 2) * ps + 1, (prefix + 2) * ps + 400)) for _ in range(B)]
    npg = [-(-n // ps) for n in lens]
    P = sum(npg) + prefix + 8
    ids = rng.permutation(np.arange(1, P)).astype(np.int32)
    tables, o = [], 0
    shared = ids[:prefix]
    o = prefix
    for b in range(B):
        own = npg[b] - (prefix if b in members else 0)
        t = np.concatenate([shared, ids[o:o + own]]) if b in members else ids[o:o + own]
        o += own
        tables.append(t)
    assert o <= P - 1
    indptr = np.zeros(B + 1, np.int32)
    np.cumsum(npg, out=indptr[1:])
    lpl = np.array([n - (k - 1) * ps for n, k in zip(lens, npg)], np.int32)
    slots = np.array([int(t[(n - 1) // ps]) * ps + (n - 1) % ps for t, n in zip(tables, lens)], np.int32)
    pos = rng.integers(0, R, size=B).astype(np.int32)
    pos[0], pos[1] = R, 0  # one past the tables (clamped to the last row), the first row
    cos, sin = O.rope_tables(D, R, 500000.0, LLAMA3)
    cos, sin = cos.to(DEV), sin.to(DEV)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(DEV)  # noqa: E731
    d_indptr, d_idx, d_lpl, d_slots, d_pos = t(indptr), t(np.concatenate(tables)), t(lpl), t(slots), t(pos)
    k_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    v_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    q = torch.randn(B, Hq, D, generator=g).to(dtype).to(DEV)
    kv = torch.randn(B, 2, Hkv, D, generator=g).to(dtype).to(DEV)  # k and v as strided views
    k_new, v_new = kv[:, 0], kv[:, 1]
    grp = K.DecodeGroups(B, [members], [prefix], DEV) if grouped else None
    kp_a, vp_a, kp_b, vp_b = k_pool.clone(), v_pool.clone(), k_pool.clone(), v_pool.clone()
    q_rot = K.rope_append(q, k_new, v_new, d_pos, d_slots, cos, sin, kp_a, vp_a)
    out_a = K.paged_decode(q_rot, kp_a, vp_a, d_indptr, d_idx, d_lpl, sum(npg), groups=grp)
    out_b = K.paged_decode_rope_append(q, k_new, v_new, d_pos, cos, sin, kp_b, vp_b, d_indptr, d_idx, d_lpl,
                                       sum(npg), groups=grp)
    torch.cuda.synchronize()
    assert torch.equal(kp_a, kp_b) and torch.equal(vp_a, vp_b)
    assert torch.equal(out_a, out_b)
    assert not torch.equal(kp_b, k_pool)  # the rows were written
