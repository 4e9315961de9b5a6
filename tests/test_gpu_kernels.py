"""Kernel parity on the GPU: every entry point of libnslg_kv.so against the CPU
oracle on identical seeded inputs. Byte movement (append, zero, copy, gather)
must be bit-exact; attention must be within 2e-3 abs + 1e-2 rel of fp32 SDPA
over the gathered pages."""
import math
import sys

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
DEV = "cuda"


def _k():
    from nanoslg_amd import kernels
    return kernels


def _log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _csr_random(lens, ps, num_pages, seed):
    rng = np.random.default_rng(seed)
    npg = [math.ceil(L / ps) if L > 0 else 0 for L in lens]
    assert sum(npg) <= num_pages - 1
    perm = rng.permutation(np.arange(1, num_pages))
    tables, off = [], 0
    for n in npg:
        tables.append(perm[off:off + n].tolist())
        off += n
    return tables, O.plan_csr(tables, lens, ps)


def _bits(t):
    return t.view(torch.int16) if t.element_size() == 2 else t.view(torch.int32)


# ------------------------------------------------------------------ byte movement


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_append_bit_exact(dtype):
    _log(f"append dtype={dtype}")
    g = torch.Generator().manual_seed(11)
    P, ps, H, D, T = 64, 16, 8, 128, 37
    pool_k = torch.randn(P, ps, H, D, generator=g).to(dtype)
    pool_v = torch.randn(P, ps, H, D, generator=g).to(dtype)
    rows_k = torch.randn(T, H, D, generator=g).to(dtype)
    rows_v = torch.randn(T, H, D, generator=g).to(dtype)
    rng = np.random.default_rng(0)
    slots = rng.choice(P * ps, size=T, replace=False).astype(np.int32)
    slots[[3, 10]] = -1  # padding rows are skipped
    ref_k = pool_k.clone().view(-1, H, D)
    ref_v = pool_v.clone().view(-1, H, D)
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            ref_k[s] = rows_k[i]
            ref_v[s] = rows_v[i]
    dk, dv = pool_k.to(DEV), pool_v.to(DEV)
    _k().append_kv(rows_k.to(DEV), rows_v.to(DEV), torch.from_numpy(slots).to(DEV), dk, dv)
    torch.cuda.synchronize()
    assert torch.equal(_bits(dk.cpu().view(-1, H, D)), _bits(ref_k))
    assert torch.equal(_bits(dv.cpu().view(-1, H, D)), _bits(ref_v))


def test_append_strided_source_bit_exact():
    """k_new as a [B,S,Hkv,D] view with S>1 and v_new as a view of a wider projection."""
    _log("append strided")
    g = torch.Generator().manual_seed(12)
    B, S, H, D, P, ps = 3, 5, 8, 128, 16, 16
    k_new = torch.randn(B, S, H, D, generator=g).half()
    proj = torch.randn(B, S, 3 * H * D, generator=g).half()
    v_new = proj[:, :, H * D:2 * H * D].reshape(B, S, H, D)  # strided rows
    slots = torch.full((B * S,), -1, dtype=torch.int32)
    slots[[0, 4, 7, 14]] = torch.tensor([3, 40, 41, 200], dtype=torch.int32)
    pk = torch.zeros(P, ps, H, D).half()
    pv = torch.zeros(P, ps, H, D).half()
    dk, dv = pk.to(DEV), pv.to(DEV)
    _k().append_kv(k_new.to(DEV), proj.to(DEV)[:, :, H * D:2 * H * D].reshape(B, S, H, D), slots.to(DEV), dk, dv)
    torch.cuda.synchronize()
    rk, rv = pk.view(-1, H, D), pv.view(-1, H, D)
    for i, s in enumerate(slots.tolist()):
        if s >= 0:
            rk[s] = k_new.reshape(-1, H, D)[i]
            rv[s] = v_new.reshape(-1, H, D)[i]
    assert torch.equal(_bits(dk.cpu()), _bits(pk)) and torch.equal(_bits(dv.cpu()), _bits(pv))


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_zero_and_copy_pages_bit_exact(dtype):
    _log(f"zero/copy dtype={dtype}")
    g = torch.Generator().manual_seed(13)
    L, P, ps, H, D = 3, 40, 16, 8, 64
    k = torch.randn(L, P, ps, H, D, generator=g).to(dtype)
    v = torch.randn(L, P, ps, H, D, generator=g).to(dtype)
    dk, dv = k.to(DEV), v.to(DEV)
    src, dst = [1, 5, 7, 9], [20, 21, 30, 39]
    _k().copy_pages(dk, dv, torch.tensor(src, dtype=torch.int32, device=DEV),
                    torch.tensor(dst, dtype=torch.int32, device=DEV))
    zero = [2, 21, 33, -4, 1000]  # out-of-range ids are skipped
    _k().zero_pages(dk, dv, torch.tensor(zero, dtype=torch.int32, device=DEV))
    torch.cuda.synchronize()
    rk, rv = k.numpy().copy(), v.numpy().copy()
    O.copy_pages(rk, src, dst)
    O.copy_pages(rv, src, dst)
    O.zero_pages(rk, zero)
    O.zero_pages(rv, zero)
    assert np.array_equal(dk.cpu().numpy().view(np.uint8), rk.view(np.uint8))
    assert np.array_equal(dv.cpu().numpy().view(np.uint8), rv.view(np.uint8))


@pytest.mark.parametrize("ps", [16, 8, 1])
def test_gather_bit_exact(ps):
    _log(f"gather ps={ps}")
    g = torch.Generator().manual_seed(14)
    lens = [1, ps, 3 * ps + 1, 0, 50]
    P = 160
    H, D = 8, 128
    k = torch.randn(P, ps, H, D, generator=g).half()
    v = torch.randn(P, ps, H, D, generator=g).half()
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, 1)
    max_len = max(lens) + 3
    gk, gv = _k().gather_kv(k.to(DEV), v.to(DEV), torch.from_numpy(indptr).to(DEV),
                            torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV), max_len)
    rk = O.gather_rows(k.view(-1, H, D).numpy(), ps, indptr, indices, lpl, max_len)
    rv = O.gather_rows(v.view(-1, H, D).numpy(), ps, indptr, indices, lpl, max_len)
    assert np.array_equal(gk.cpu().numpy().view(np.uint16), rk.view(np.uint16))
    assert np.array_equal(gv.cpu().numpy().view(np.uint16), rv.view(np.uint16))


# ------------------------------------------------------------------ decode attention


def _decode_case(lens, Hq, Hkv, D, ps, dtype, seed, num_pages=None, scale=None):
    g = torch.Generator().manual_seed(seed)
    npg = sum(math.ceil(L / ps) for L in lens)
    P = num_pages or (npg + 8)
    k = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    v = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    q = torch.randn(len(lens), Hq, D, generator=g).to(dtype)
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, seed)
    out = _k().paged_decode(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(indptr).to(DEV),
                            torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV),
                            int(indptr[-1]), sm_scale=scale)
    torch.cuda.synchronize()
    ref = O.paged_attention_ref([q[b:b + 1] for b in range(len(lens))], k.view(-1, Hkv, D),
                                v.view(-1, Hkv, D), ps, indptr, indices, lpl, [1] * len(lens), scale)
    ref = torch.stack([r[0] if r.shape[0] else torch.zeros(Hq, D) for r in ref])
    return out.cpu().float(), ref


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_decode_dtypes_and_head_dims(dtype, D):
    _log(f"decode dtype={dtype} D={D}")
    out, ref = _decode_case([1, 17, 300, 1024], 32, 8, D, 16, dtype, seed=D)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("Hq,Hkv", [(8, 8), (32, 8), (64, 8), (16, 1), (48, 3)])
def test_decode_gqa_groups(Hq, Hkv):
    _log(f"decode gqa Hq={Hq} Hkv={Hkv}")
    out, ref = _decode_case([5, 64, 129, 700], Hq, Hkv, 128, 16, torch.float16, seed=Hq + Hkv)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("ps", [1, 8, 16, 32, 64, 48])
def test_decode_page_sizes(ps):
    _log(f"decode ps={ps}")
    out, ref = _decode_case([1, ps, ps + 1, 333, 2000], 32, 8, 128, ps, torch.float16, seed=ps)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_decode_long_and_many_splits():
    _log("decode long")
    out, ref = _decode_case([32768, 2048, 9000, 16], 32, 8, 128, 16, torch.float16, seed=21)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_decode_empty_sequence_is_zero_and_scale():
    _log("decode empty + scale")
    out, ref = _decode_case([0, 40, 0, 3], 32, 8, 128, 16, torch.float16, seed=22, scale=0.05)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0


def test_decode_closed_forms():
    """L=1 -> out = v; identical keys -> out = mean(V)."""
    _log("decode closed forms")
    Hq, Hkv, D, ps = 32, 8, 128, 16
    g = torch.Generator().manual_seed(23)
    P = 8
    k = torch.randn(P, ps, Hkv, D, generator=g).half()
    v = torch.randn(P, ps, Hkv, D, generator=g).half()
    k[2] = k[2, :1].expand(ps, Hkv, D)  # page 2: identical keys
    k[3] = k[2, :1].expand(ps, Hkv, D)
    q = torch.randn(2, Hq, D, generator=g).half()
    indptr = torch.tensor([0, 1, 3], dtype=torch.int32)
    indices = torch.tensor([5, 2, 3], dtype=torch.int32)
    lpl = torch.tensor([1, 16], dtype=torch.int32)
    out = _k().paged_decode(q.to(DEV), k.to(DEV), v.to(DEV), indptr.to(DEV), indices.to(DEV), lpl.to(DEV), 3)
    out = out.cpu().float()
    G = Hq // Hkv
    for h in range(Hq):
        torch.testing.assert_close(out[0, h], v[5, 0, h // G].float(), atol=1e-3, rtol=0)
        mean = torch.cat([v[2, :, h // G], v[3, :, h // G]]).float().mean(0)
        torch.testing.assert_close(out[1, h], mean, atol=2e-3, rtol=1e-2)


def test_decode_rejects_bad_arguments():
    kern = _k()
    from nanoslg_amd._lib import KernelLibraryError
    q = torch.zeros(2, 32, 100, dtype=torch.float16, device=DEV)
    kv = torch.zeros(4, 16, 8, 100, dtype=torch.float16, device=DEV)
    ip = torch.tensor([0, 1, 2], dtype=torch.int32, device=DEV)
    with pytest.raises(KernelLibraryError):
        kern.paged_decode(q, kv, kv, ip, ip[:2].contiguous(), ip[:2].contiguous(), 2)


# ------------------------------------------------------------------ prefill attention


def _prefill_case(lens, news, Hq, Hkv, D, ps, dtype, seed, scale=None, max_q=None):
    g = torch.Generator().manual_seed(seed)
    npg = sum(math.ceil(L / ps) for L in lens)
    P = npg + 4
    k = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    v = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    T = sum(news)
    q = torch.randn(T, Hq, D, generator=g).to(dtype)
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, seed)
    qo = np.zeros(len(lens) + 1, np.int32)
    qo[1:] = np.cumsum(news)
    out = _k().paged_prefill(q.to(DEV), torch.from_numpy(qo).to(DEV), T, max(news) if max_q is None else max_q,
                             k.to(DEV), v.to(DEV),
                             torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV),
                             torch.from_numpy(lpl).to(DEV), sm_scale=scale)
    torch.cuda.synchronize()
    qs = [q[qo[b]:qo[b + 1]] for b in range(len(lens))]
    ref = O.paged_attention_ref(qs, k.view(-1, Hkv, D), v.view(-1, Hkv, D), ps, indptr, indices, lpl, news, scale)
    return out.cpu().float(), torch.cat(ref, 0)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_prefill_from_zero(dtype, D):
    _log(f"prefill from zero dtype={dtype} D={D}")
    out, ref = _prefill_case([37, 100, 1], [37, 100, 1], 32, 8, D, 16, dtype, seed=31 + D)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("Hq,Hkv", [(32, 8), (8, 8), (16, 1), (48, 3), (16, 8)])
def test_prefill_chunk_over_cached_context(Hq, Hkv):
    _log(f"prefill chunked Hq={Hq} Hkv={Hkv}")
    out, ref = _prefill_case([300, 1000, 64, 17], [64, 200, 64, 3], Hq, Hkv, 128, 16, torch.float16,
                             seed=Hq * 7 + Hkv)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("ps", [1, 8, 32, 48])
def test_prefill_page_sizes(ps):
    _log(f"prefill ps={ps}")
    out, ref = _prefill_case([130, 77, 400], [130, 20, 129], 32, 8, 128, ps, torch.float16, seed=40 + ps)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_prefill_long_chunk_and_page_window():
    """A 512-token chunk over 3584 cached tokens, and a sequence whose page ids span
    more than one 2048-entry window (page size 1)."""
    _log("prefill long + window")
    out, ref = _prefill_case([4096, 2500], [512, 300], 32, 8, 128, 16, torch.float16, seed=50)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    out, ref = _prefill_case([4500], [70], 32, 8, 128, 1, torch.float16, seed=51)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_prefill_row_tile_orders():
    """Near-uniform batches run their row tiles longest first (rounds sized by the
    host's max_q); a max_q below a sequence's new tokens, or a ragged batch, takes the
    packed order. Same results either way."""
    _log("prefill tile orders")
    lens, news = [1500, 1400, 1300, 1200], [512, 512, 500, 480]
    # exact: rounds; understated: the kernel finds a sequence with more tiles than the
    # rounds cover and packs; far overstated: too many empty slots, packed by the host
    for max_q in (None, 1, 4096):
        out, ref = _prefill_case(lens, news, 32, 8, 128, 16, torch.float16, seed=53, max_q=max_q)
        torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_prefill_head_dim_256_chunk_over_cached_context(dtype):
    """16-bit pools at head_dim 256 (the MFMA kernel's shape for it: one 16-row column
    block per wave, 64-key tiles, 128 rows per workgroup): chunks over cached context,
    GQA 4, 1 and 8, a 512-token chunk over 3584 cached tokens, page sizes 16 and 1 (a
    sequence whose page ids span more than one 2048-entry window), against the oracle."""
    _log(f"prefill D=256 {dtype}")
    out, ref = _prefill_case([300, 1000, 64, 17], [64, 200, 64, 3], 32, 8, 256, 16, dtype, seed=61)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    out, ref = _prefill_case([90, 40], [30, 40], 16, 4, 256, 1, dtype, seed=62)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    out, ref = _prefill_case([4096, 2500], [512, 300], 16, 4, 256, 16, dtype, seed=63)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    out, ref = _prefill_case([4500, 33], [70, 33], 8, 8, 256, 1, dtype, seed=64)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    out, ref = _prefill_case([1500, 1400, 1300], [512, 500, 480], 64, 8, 256, 16, dtype, seed=65)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_prefill_sequence_without_new_tokens():
    _log("prefill n=0 rows")
    out, ref = _prefill_case([50, 20, 33], [5, 0, 33], 32, 8, 128, 16, torch.float16, seed=52, scale=0.1)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("dtype,D", [(torch.float16, 128), (torch.bfloat16, 64), (torch.float32, 128),
                                     (torch.float32, 256), (torch.bfloat16, 256)])
def test_prefill_grid_rows_bit_exact(dtype, D):
    """nslg_paged_prefill_grid on a padded [B, S] grid (left and right padding, a
    sequence without new tokens, a full row) against nslg_paged_prefill on the ragged
    rows gathered from it: the token rows bit-identical, every pad row zero (the output
    starts as NaN), and the ragged result against the oracle."""
    _log(f"prefill grid rows {dtype} D={D}")
    K = _k()
    ps, Hq, Hkv = 16, 32, 8
    lens, news, offs = [300, 77, 40, 129, 9], [64, 20, 0, 129, 9], [3, 0, 5, 0, 100]
    S = max(o + n for o, n in zip(offs, news))
    B = len(lens)
    g = torch.Generator().manual_seed(D + len(lens))
    P = sum(math.ceil(L / ps) for L in lens) + 5
    k = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, D)
    qo = np.zeros(B + 1, np.int32)
    np.cumsum(news, out=qo[1:])
    rows = np.concatenate([b * S + o + np.arange(n) for b, (o, n) in enumerate(zip(offs, news))]).astype(np.int32)
    grid = torch.randn(B * S, Hq, D, generator=g).to(dtype).to(DEV)
    ip, ix, lp, qo_d, rows_d = (torch.from_numpy(a).to(DEV) for a in (indptr, indices, lpl, qo, rows))
    T = int(qo[-1])
    out = torch.full((B * S, Hq, D), float("nan"), dtype=dtype, device=DEV)
    K.paged_prefill(grid, qo_d, T, max(news), k, v, ip, ix, lp, out=out, q_rows=rows_d, grid_width=S)
    rag = K.paged_prefill(grid.index_select(0, rows_d.long()).contiguous(), qo_d, T, max(news), k, v, ip, ix, lp)
    torch.cuda.synchronize()
    assert torch.equal(_bits(out[rows_d.long()]), _bits(rag))
    pad = torch.ones(B * S, dtype=torch.bool)
    pad[torch.from_numpy(rows).long()] = False
    assert torch.count_nonzero(out[pad.to(DEV)]) == 0
    q_list = [grid[torch.from_numpy(rows[qo[b]:qo[b + 1]]).long().to(DEV)].cpu() for b in range(B)]
    ref = O.paged_attention_ref(q_list, k.cpu().view(-1, Hkv, D), v.cpu().view(-1, Hkv, D), ps, indptr, indices,
                                lpl, news)
    ref = torch.cat([r for r in ref if r.shape[0]], 0)
    tol = F32_TOL if dtype == torch.float32 else dict(atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(rag.cpu().float(), ref, **tol)


# ------------------------------------------------------------------ fp32 pools

F32_TOL = dict(atol=2e-5, rtol=1e-4)  # fp32 kernel against fp32 SDPA: summation-order differences only


@pytest.mark.parametrize("D", [64, 128, 256])
def test_f32_decode_and_prefill(D):
    """fp32 pools (the contiguous backend of an fp32 model) go through the fp32
    attention kernel: decode rows and ragged causal prefill rows."""
    _log(f"f32 decode/prefill D={D}")
    out, ref = _decode_case([1, 17, 300, 1024, 0], 32, 8, D, 16, torch.float32, seed=60 + D)
    torch.testing.assert_close(out, ref, **F32_TOL)
    assert torch.count_nonzero(out[4]) == 0
    out, ref = _prefill_case([37, 300, 1, 50], [37, 64, 1, 0], 32, 8, D, 16, torch.float32, seed=61 + D)
    torch.testing.assert_close(out, ref, **F32_TOL)


@pytest.mark.parametrize("Hq,Hkv,ps", [(48, 3, 16), (16, 1, 1), (8, 8, 48), (64, 8, 32)])
def test_f32_groups_and_page_sizes(Hq, Hkv, ps):
    _log(f"f32 Hq={Hq} Hkv={Hkv} ps={ps}")
    out, ref = _decode_case([5, ps + 1, 700], Hq, Hkv, 128, ps, torch.float32, seed=Hq + ps, scale=0.07)
    torch.testing.assert_close(out, ref, **F32_TOL)
    out, ref = _prefill_case([130, 77, 400], [130, 20, 129], Hq, Hkv, 128, ps, torch.float32, seed=Hq * ps)
    torch.testing.assert_close(out, ref, **F32_TOL)


@pytest.mark.parametrize("lens", [[32768], [9000, 3000, 1, 0], [20000] * 8])
def test_f32_decode_split_over_keys(lens):
    """Long fp32 decodes are split over keys (partials in the workspace, then an fp32
    merge): 64, 7 and 8 splits here."""
    _log(f"f32 decode splits lens={lens[:4]}")
    out, ref = _decode_case(lens, 32, 8, 128, 16, torch.float32, seed=len(lens) + lens[0] % 97)
    torch.testing.assert_close(out, ref, **F32_TOL)
    for b, L in enumerate(lens):
        if L == 0:
            assert torch.count_nonzero(out[b]) == 0


def test_f32_grouped_decode_is_rejected():
    """Grouped (shared-prefix) decode runs on the 16-bit MFMA path only."""
    from nanoslg_amd import _lib
    lib = _lib.load()
    assert lib.nslg_paged_decode_grouped_workspace_size(4, 32, 8, 128, 100, 16, _lib.NSLG_F32, 1) == 0


def test_decode_large_batches():
    """Batches larger than half the device's resident chunk slots take the
    several-rounds launch; more than 256 sequences go past the lengths a wave
    keeps in registers. Mixed lengths (empty ones included) and many short ones."""
    rng = np.random.default_rng(70)
    lens = rng.integers(0, 3000, size=400).tolist()
    lens[:3] = [0, 1, 16]
    _log(f"decode large batch B={len(lens)}")
    out, ref = _decode_case(lens, 32, 8, 128, 16, torch.float16, seed=70)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)
    lens = rng.integers(1, 65, size=2000).tolist()
    _log(f"decode large batch B={len(lens)}")
    out, ref = _decode_case(lens, 32, 8, 128, 16, torch.bfloat16, seed=71)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_prefill_large_ragged_batch():
    """100 sequences with 0..64 new tokens over cached contexts of up to 2000 tokens."""
    rng = np.random.default_rng(72)
    news = rng.integers(0, 65, size=100).tolist()
    lens = [n + int(c) for n, c in zip(news, rng.integers(0, 2000, size=100))]
    lens[0], news[0] = 0, 0
    _log(f"prefill large ragged batch B={len(lens)} T={sum(news)}")
    out, ref = _prefill_case(lens, news, 32, 8, 128, 16, torch.float16, seed=72)
    torch.testing.assert_close(out, ref, atol=ATOL, rtol=RTOL)


def test_decode_workspace_reuse_across_calls():
    """One workspace serves a sequence of different batches (split-K partials of a
    call never leak into the next)."""
    _log("decode workspace reuse")
    from nanoslg_amd.kernels import Workspace
    ws = Workspace(torch.device(DEV))
    cases = [([32768, 2048, 9000, 16], 60), ([5, 64, 129, 700], 61), ([20000] * 8, 62), ([1, 3000], 63),
             ([32768, 2048, 9000, 16], 60)]
    for lens, seed in cases:
        g = torch.Generator().manual_seed(seed)
        ps, Hq, Hkv, D = 16, 32, 8, 128
        npg = sum(math.ceil(L / ps) for L in lens)
        P = npg + 8
        k = torch.randn(P, ps, Hkv, D, generator=g).half()
        v = torch.randn(P, ps, Hkv, D, generator=g).half()
        q = torch.randn(len(lens), Hq, D, generator=g).half()
        tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, seed)
        out = _k().paged_decode(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(indptr).to(DEV),
                                torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV),
                                int(indptr[-1]), workspace=ws)
        ref = O.paged_attention_ref([q[b:b + 1] for b in range(len(lens))], k.view(-1, Hkv, D),
                                    v.view(-1, Hkv, D), ps, indptr, indices, lpl, [1] * len(lens))
        torch.testing.assert_close(out.cpu().float(), torch.stack([r[0] for r in ref]), atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("lens,Hq,Hkv,D,ps", [
    ([91, 51, 18], 32, 8, 128, 16),
    ([32768, 2048, 9000, 16, 300], 32, 8, 128, 16),
    ([5000, 17, 2048], 8, 2, 64, 32),
    ([4000, 129], 16, 1, 256, 8),
    ([20000] * 8, 28, 4, 128, 16),
])
def test_decode_writes_stay_inside_workspace_and_out(lens, Hq, Hkv, D, ps):
    """Every byte the decode call writes lies inside `out` and the sized workspace:
    guard regions after both keep their fill pattern, and the result is correct."""
    _log(f"decode guards {lens} Hq={Hq} Hkv={Hkv} D={D} ps={ps}")
    import ctypes
    from nanoslg_amd import _lib
    lib = _lib.load()
    g = torch.Generator().manual_seed(70)
    npg = sum(math.ceil(L / ps) for L in lens)
    P = npg + 8
    k = torch.randn(P, ps, Hkv, D, generator=g).half()
    v = torch.randn(P, ps, Hkv, D, generator=g).half()
    B = len(lens)
    q = torch.randn(B, Hq, D, generator=g).half()
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, 70)
    need = int(lib.nslg_paged_decode_workspace_size(B, Hq, Hkv, D, int(indptr[-1]), ps, 0))
    guard = 1 << 20
    ws = torch.full((need + guard,), 0xA5, dtype=torch.uint8, device=DEV)
    out = torch.full((B + 4, Hq, D), -7.0, dtype=torch.float16, device=DEV)
    kd, vd, qd = k.to(DEV), v.to(DEV), q.to(DEV)
    ip, ix, lp = (torch.from_numpy(a).to(DEV) for a in (indptr, indices, lpl))
    rc = lib.nslg_paged_decode(qd.data_ptr(), Hq * D, kd.data_ptr(), vd.data_ptr(), P, ps, ip.data_ptr(),
                               ix.data_ptr(), lp.data_ptr(), int(indptr[-1]), B, Hq, Hkv, D,
                               1.0 / math.sqrt(D), 0, out.data_ptr(), Hq * D, ws.data_ptr(), need, 0,
                               ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == 0, _lib.last_error()
    torch.cuda.synchronize()
    assert bool((ws[need:] == 0xA5).all()), "decode wrote past its workspace"
    assert bool((out[B:] == -7.0).all()), "decode wrote past its output rows"
    ref = O.paged_attention_ref([q[b:b + 1] for b in range(B)], k.view(-1, Hkv, D), v.view(-1, Hkv, D), ps,
                                indptr, indices, lpl, [1] * B)
    torch.testing.assert_close(out[:B].cpu().float(), torch.stack([r[0] for r in ref]), atol=ATOL, rtol=RTOL)


def test_decode_chunks_longer_than_the_page_window():
    """Two 400k-token sequences whose block tables draw (with repeats) from a
    64-page pool: the chunks run past 128 pages, so the per-lane page-id window is
    refilled mid-chunk. Reference: attention over the distinct rows weighted by
    how often each appears, in float64."""
    _log("decode long chunks / page-id window refill")
    ps, Hq, Hkv, D, P = 16, 32, 8, 128, 64
    lens = [400_000, 399_993]
    g = torch.Generator().manual_seed(71)
    rng = np.random.default_rng(71)
    k = torch.randn(P, ps, Hkv, D, generator=g).half()
    v = torch.randn(P, ps, Hkv, D, generator=g).half()
    q = torch.randn(len(lens), Hq, D, generator=g).half()
    tables = [rng.integers(1, P, size=math.ceil(L / ps)).tolist() for L in lens]
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    out = _k().paged_decode(q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(indptr).to(DEV),
                            torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV), int(indptr[-1]))
    torch.cuda.synchronize()
    kf = k.double().reshape(P * ps, Hkv, D)
    vf = v.double().reshape(P * ps, Hkv, D)
    G = Hq // Hkv
    for b, L in enumerate(lens):
        rows = (np.asarray(tables[b])[:, None] * ps + np.arange(ps)[None, :]).reshape(-1)[:L]
        mult = torch.from_numpy(np.bincount(rows, minlength=P * ps)).double()
        used = mult > 0
        ks, vs, w = kf[used], vf[used], mult[used]
        qb = q[b].double().reshape(Hkv, G, D)
        s = torch.einsum("hgd,nhd->hgn", qb, ks) / math.sqrt(D)
        s = s - s.amax(-1, keepdim=True)
        p = torch.exp(s) * w
        ref = torch.einsum("hgn,nhd->hgd", p, vs) / p.sum(-1, keepdim=True)
        torch.testing.assert_close(out[b].cpu().float(), ref.reshape(Hq, D).float(), atol=ATOL, rtol=RTOL)


def test_decode_launch_matches_separate_calls():
    """The per-forward launcher (append + decode per layer, one launch when the new rows
    are 16-byte aligned) gives the same pool bytes and the same outputs as append_kv
    followed by paged_decode on each layer, with q as [B, Hq, D] rows or as a forward's
    [B, 1, Hq, D] grid (output [B, 1, Hq * D]), and with unaligned new rows."""
    _log("decode launcher vs separate calls")
    from nanoslg_amd import kernels as K
    g = torch.Generator().manual_seed(72)
    L, P, ps, Hq, Hkv, D = 3, 200, 16, 32, 8, 128
    lens = [700, 33, 1500, 1]
    k_pool = torch.randn(L, P, ps, Hkv, D, generator=g).half().to(DEV)
    v_pool = torch.randn(L, P, ps, Hkv, D, generator=g).half().to(DEV)
    k2, v2 = k_pool.clone(), v_pool.clone()
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, 72)
    slots = torch.tensor([tables[b][(n - 1) // ps] * ps + (n - 1) % ps for b, n in enumerate(lens)],
                         dtype=torch.int32, device=DEV)
    ip, ix, lp = (torch.from_numpy(a).to(DEV) for a in (indptr, indices, lpl))
    launch = K.DecodeLaunch(k_pool, v_pool, slots, ip, ix, lp, int(indptr[-1]), Hq)
    for layer in range(L):
        q = torch.randn(len(lens), Hq, D, generator=g).half().to(DEV)
        kn = torch.randn(len(lens), 1, Hkv, D, generator=g).half().to(DEV)
        vn = torch.randn(len(lens), 1, Hkv, D, generator=g).half().to(DEV)
        if layer == 2:  # rows 2 bytes off 16-byte alignment: the append runs as its own launch
            kn = torch.cat([torch.zeros(1, dtype=kn.dtype, device=DEV), kn.reshape(-1)])[1:].view(kn.shape)
            assert kn.data_ptr() % 16 == 2
        grid = layer % 2 == 1  # odd layers: the forward's [B, 1, Hq, D] grid
        o1 = launch(layer, q.unsqueeze(1) if grid else q, kn, vn)
        K.append_kv(kn, vn, slots, k2[layer], v2[layer])
        o2 = K.paged_decode(q, k2[layer], v2[layer], ip, ix, lp, int(indptr[-1]))
        torch.cuda.synchronize()
        if grid:
            assert o1.shape == (len(lens), 1, Hq * D)
            o1 = o1.view(len(lens), Hq, D)
        assert torch.equal(o1, o2)
    assert torch.equal(k_pool, k2) and torch.equal(v_pool, v2)
    with pytest.raises(ValueError):
        launch(0, q[:2], kn, vn)
    with pytest.raises(ValueError):  # two tokens per sequence: not a decode grid
        launch(0, q.unsqueeze(1).expand(-1, 2, -1, -1), kn, vn)
    with pytest.raises(IndexError):
        launch(L, q, kn, vn)


@pytest.mark.parametrize("dtype,D,ps,Hq,Hkv,lens", [
    (torch.float16, 128, 16, 32, 8, [700, 33, 1500, 1, 16, 17]),
    (torch.bfloat16, 128, 16, 32, 8, [4096, 2, 31]),
    (torch.float16, 64, 8, 16, 2, [300, 1, 65]),
    (torch.bfloat16, 256, 24, 8, 8, [100, 999]),
    (torch.float16, 128, 1, 16, 1, [40, 3]),
    (torch.float16, 128, 64, 48, 3, [5000, 64, 65]),
    (torch.float32, 128, 16, 32, 8, [700, 33, 1]),
    (torch.float32, 64, 5, 8, 2, [2100, 9]),
])
def test_decode_append_bit_exact(dtype, D, ps, Hq, Hkv, lens):
    """nslg_paged_decode_append (the new rows written by the decode chunk that reads
    them) against nslg_append_kv at the block table's slots followed by
    nslg_paged_decode: pools and outputs bit-identical, k_new/v_new as strided views of
    one projection buffer (the model's layout); and the outputs against the oracle."""
    _log(f"decode_append {dtype} D={D} ps={ps} Hq={Hq} Hkv={Hkv} lens={lens}")
    K = _k()
    g = torch.Generator().manual_seed(D + ps + len(lens))
    B = len(lens)
    P = sum(math.ceil(L / ps) for L in lens) + 9
    k_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    v_pool = torch.randn(P, ps, Hkv, D, generator=g).to(dtype).to(DEV)
    k2, v2 = k_pool.clone(), v_pool.clone()
    tables, (indptr, indices, lpl) = _csr_random(lens, ps, P, D + ps)
    slots = torch.tensor([tables[b][(n - 1) // ps] * ps + (n - 1) % ps for b, n in enumerate(lens)],
                         dtype=torch.int32, device=DEV)
    ip, ix, lp = (torch.from_numpy(a).to(DEV) for a in (indptr, indices, lpl))
    qkv = torch.randn(B, 1, (Hq + 2 * Hkv) * D, generator=g).to(dtype).to(DEV)
    q = qkv[:, 0, :Hq * D].view(B, Hq, D)
    kn = qkv[:, :, Hq * D:(Hq + Hkv) * D].view(B, 1, Hkv, D)
    vn = qkv[:, :, (Hq + Hkv) * D:].view(B, 1, Hkv, D)
    o1 = K.paged_decode_append(q, kn, vn, k_pool, v_pool, ip, ix, lp, int(indptr[-1]))
    K.append_kv(kn, vn, slots, k2, v2)
    o2 = K.paged_decode(q, k2, v2, ip, ix, lp, int(indptr[-1]))
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_pool), _bits(k2)) and torch.equal(_bits(v_pool), _bits(v2))
    assert torch.equal(_bits(o1), _bits(o2))
    ref = O.paged_attention_ref([q[b:b + 1].cpu() for b in range(B)], k2.cpu().view(-1, Hkv, D),
                                v2.cpu().view(-1, Hkv, D), ps, indptr, indices, lpl, [1] * B)
    ref = torch.stack([r[0] for r in ref])
    tol = (2e-5, 1e-4) if dtype == torch.float32 else (ATOL, RTOL)
    torch.testing.assert_close(o1.cpu().float(), ref, atol=tol[0], rtol=tol[1])


def test_decode_append_grouped_bit_exact():
    """nslg_paged_decode_grouped_append against append + the grouped decode: groups of
    sequences sharing prefix pages, each writing its new row past the prefix."""
    _log("decode_append grouped")
    K = _k()
    rng = np.random.default_rng(5)
    ps, Hq, Hkv, D = 16, 32, 8, 128
    members = [[0, 3, 5], [1, 4]]
    prefix = [20, 7]
    pages = iter(rng.permutation(np.arange(1, 3000)).tolist())
    tables, lens = [None] * 7, [0] * 7
    for ms, pp in zip(members, prefix):
        shared = [next(pages) for _ in range(pp)]
        for b in ms:
            own = int(rng.integers(1, 200))
            lens[b] = pp * ps + own
            tables[b] = shared + [next(pages) for _ in range(math.ceil(own / ps))]
    for b in (2, 6):
        lens[b] = int(rng.integers(1, 900))
        tables[b] = [next(pages) for _ in range(math.ceil(lens[b] / ps))]
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    g = torch.Generator().manual_seed(5)
    k_pool = torch.randn(3000, ps, Hkv, D, generator=g).half().to(DEV)
    v_pool = torch.randn(3000, ps, Hkv, D, generator=g).half().to(DEV)
    k2, v2 = k_pool.clone(), v_pool.clone()
    q = torch.randn(7, Hq, D, generator=g).half().to(DEV)
    kn = torch.randn(7, Hkv, D, generator=g).half().to(DEV)
    vn = torch.randn(7, Hkv, D, generator=g).half().to(DEV)
    slots = torch.tensor([tables[b][(n - 1) // ps] * ps + (n - 1) % ps for b, n in enumerate(lens)],
                         dtype=torch.int32, device=DEV)
    ip, ix, lp = (torch.from_numpy(a).to(DEV) for a in (indptr, indices, lpl))
    groups = K.DecodeGroups(7, members, prefix, DEV)
    o1 = K.paged_decode_append(q, kn, vn, k_pool, v_pool, ip, ix, lp, int(indptr[-1]), groups=groups)
    K.append_kv(kn, vn, slots, k2, v2)
    o2 = K.paged_decode(q, k2, v2, ip, ix, lp, int(indptr[-1]), groups=groups)
    torch.cuda.synchronize()
    assert torch.equal(_bits(k_pool), _bits(k2)) and torch.equal(_bits(v_pool), _bits(v2))
    assert torch.equal(_bits(o1), _bits(o2))


@pytest.mark.parametrize("B,ps", [(64, 16), (65, 16), (1, 16), (37, 32), (512, 8)])
def test_decode_plan_step_bit_exact(B, ps):
    """The device-built next-step plan equals the CSR the oracle builds from the
    extended block tables (kv_cache.py:598-615), with slots and positions of the new
    tokens; sequences with a full last page or no page open the page they are given,
    or the null page when given none."""
    _log(f"decode plan step B={B} ps={ps}")
    from nanoslg_amd import kernels as K
    rng = np.random.default_rng(73 + B)
    lens = [int(x) for x in rng.integers(0, 3000, size=B)]
    for b in range(0, B, 5):
        lens[b] = ps * (b % 7)  # full last page (or empty)
    npg = [math.ceil(L / ps) for L in lens]
    perm = rng.permutation(np.arange(1, sum(npg) + B + 10)).tolist()
    tables, off = [], 0
    for n in npg:
        tables.append(perm[off:off + n])
        off += n
    spare = perm[off:]
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    opens = [L % ps == 0 for L in lens]
    new_page = np.full(B, -1, np.int32)
    for b in range(B):
        if opens[b] and b % 11 != 3:  # a few openers get no page: the null page
            new_page[b] = spare.pop()
    exp_tables = [t + ([int(new_page[b]) if new_page[b] >= 0 else 0] if opens[b] else []) for b, t in enumerate(tables)]
    exp_lens = [L + 1 for L in lens]
    e_indptr, e_indices, e_lpl = O.plan_csr(exp_tables, exp_lens, ps)
    e_slot = [exp_tables[b][L // ps] * ps + L % ps for b, L in enumerate(lens)]
    e_new = [t[-1] for b, t in enumerate(exp_tables) if opens[b]]
    out = K.decode_plan_step(torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV),
                             torch.from_numpy(lpl).to(DEV), new_page, ps, int(sum(opens)))
    torch.cuda.synchronize()
    ip, ix, lp, sl, pos, new = (t.cpu().numpy() for t in out)
    assert np.array_equal(ip, e_indptr)
    assert np.array_equal(ix[:e_indptr[-1]], e_indices[:e_indptr[-1]])
    assert np.array_equal(lp, e_lpl)
    assert np.array_equal(sl, np.array(e_slot, np.int32))
    assert np.array_equal(pos, np.array(lens, np.int32))
    assert np.array_equal(new, np.array(e_new, np.int32))


@pytest.mark.parametrize("L,ps,Hkv,D,B", [(2, 16, 8, 128, 64), (3, 8, 2, 64, 37), (1, 32, 16, 128, 5)])
def test_decode_plan_step_zeroes_opened_pages(L, ps, Hkv, D, B):
    """Given the pools, the planner launch also zeroes every opened page in every
    layer, K and V (the zero-on-alloc, kv_cache.py:411), 16 KiB per workgroup, and
    touches no other page; the plan itself is the one built without the pools."""
    _log(f"decode plan step zeroing L={L} ps={ps} Hkv={Hkv} D={D} B={B}")
    from nanoslg_amd import kernels as K
    rng = np.random.default_rng(91 + B)
    lens = [int(x) for x in rng.integers(1, 200, size=B)]
    for b in range(0, B, 3):
        lens[b] = ps * (1 + b % 4)  # full last page: opens one
    npg = [math.ceil(n / ps) for n in lens]
    P = sum(npg) + B + 4
    perm = rng.permutation(np.arange(1, P)).tolist()
    tables, off = [], 0
    for n in npg:
        tables.append(perm[off:off + n])
        off += n
    spare = perm[off:]
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    opens = [n % ps == 0 for n in lens]
    new_page = np.full(B, -1, np.int32)
    for b in range(B):
        if opens[b]:
            new_page[b] = spare.pop()
    g = torch.Generator().manual_seed(5)
    k_pool = torch.randn(L, P, ps, Hkv, D, generator=g).half().to(DEV)
    v_pool = torch.randn(L, P, ps, Hkv, D, generator=g).half().to(DEV)
    k_exp, v_exp = k_pool.clone(), v_pool.clone()
    opened = torch.tensor([int(p) for p in new_page if p >= 0], dtype=torch.long, device=DEV)
    k_exp[:, opened] = 0
    v_exp[:, opened] = 0
    args = (torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV),
            new_page, ps, int(sum(opens)))
    plain = K.decode_plan_step(*args)
    fused = K.decode_plan_step(*args, k_pool, v_pool)
    torch.cuda.synchronize()
    for a, b in zip(plain, fused):
        assert torch.equal(a, b)
    assert torch.equal(k_pool, k_exp)
    assert torch.equal(v_pool, v_exp)


def _grouped_case(Hq, Hkv, ps, dtype, seed, group_sizes, prefix_pages, n_alone, own_max=300, D=128):
    """A batch in which groups of sequences share their first pages (same page ids),
    plus sequences of their own, in shuffled batch order. Returns the grouped and the
    plain decode outputs and the oracle's."""
    K = _k()
    rng = np.random.default_rng(seed)
    B = sum(group_sizes) + n_alone
    order = rng.permutation(B).tolist()
    members, lens, tables = [], [0] * B, [None] * B
    next_page = iter(rng.permutation(np.arange(1, 20000)).tolist())
    pos = 0
    for gsz, pp in zip(group_sizes, prefix_pages):
        shared = [next(next_page) for _ in range(pp)]
        ms = order[pos:pos + gsz]
        pos += gsz
        members.append(ms)
        for i, b in enumerate(ms):
            own = 0 if i == 1 else int(rng.integers(1, own_max))  # member 1 has nothing past the prefix
            lens[b] = pp * ps + own
            tables[b] = shared + [next(next_page) for _ in range(math.ceil(own / ps))]
    for b in order[pos:]:
        lens[b] = int(rng.integers(1, 3000))
        tables[b] = [next(next_page) for _ in range(math.ceil(lens[b] / ps))]
    P = 20000
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    v = torch.randn(P, ps, Hkv, D, generator=g).to(dtype)
    q = torch.randn(B, Hq, D, generator=g).to(dtype)
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    args = (q.to(DEV), k.to(DEV), v.to(DEV), torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV),
            torch.from_numpy(lpl).to(DEV), int(indptr[-1]))
    groups = K.DecodeGroups(B, members, prefix_pages, DEV)
    out_g = K.paged_decode(*args, groups=groups)
    out_p = K.paged_decode(*args)
    torch.cuda.synchronize()
    ref = O.paged_attention_ref([q[b:b + 1] for b in range(B)], k.view(-1, Hkv, D), v.view(-1, Hkv, D), ps,
                                indptr, indices, lpl, [1] * B)
    ref = torch.stack([r[0] for r in ref])
    return out_g.cpu().float(), out_p.cpu().float(), ref


@pytest.mark.parametrize("Hq,Hkv,ps,dtype,sizes,prefix,D", [
    (32, 8, 16, torch.float16, [4, 4, 3], [127, 10, 1], 128),
    (32, 8, 16, torch.bfloat16, [4, 2], [12, 3], 64),
    (32, 8, 16, torch.float16, [4, 3], [20, 2], 256),
    (16, 8, 16, torch.bfloat16, [8, 5], [30, 4], 128),   # G = 2: 8 members
    (8, 8, 16, torch.float16, [16, 2], [40, 3], 128),
    (64, 8, 16, torch.bfloat16, [2, 2], [64, 5], 128),
    (32, 8, 8, torch.float16, [4, 2], [50, 7], 128),
    (16, 1, 16, torch.float16, [1, 1], [20, 2], 128),
])
def test_decode_grouped_prefix(Hq, Hkv, ps, dtype, sizes, prefix, D):
    """Groups of sequences sharing their first pages: the grouped decode (prefix read
    once per group, members in the MFMA columns) against the oracle, and against the
    plain decode of the same batch; a member with no token past the prefix included."""
    _log(f"decode grouped Hq={Hq} Hkv={Hkv} ps={ps} {dtype} groups={sizes} prefix={prefix} D={D}")
    out_g, out_p, ref = _grouped_case(Hq, Hkv, ps, dtype, 7 + Hq + ps, sizes, prefix, n_alone=5, D=D)
    torch.testing.assert_close(out_g, ref, atol=ATOL, rtol=RTOL)
    torch.testing.assert_close(out_p, ref, atol=ATOL, rtol=RTOL)


@pytest.mark.parametrize("grouped,n_alone,own_max", [(False, 3, 4000), (True, 2, 600), (False, 40, 2500),
                                                      (True, 30, 900)])
def test_decode_layout_record_and_reuse_bit_exact(grouped, n_alone, own_max):
    """The later layers of a forward read the chunk layout the first layer's call
    recorded in the workspace (layout -t) instead of cutting the chunks again; a call
    whose tag the workspace no longer holds (another call recorded in between) cuts
    them itself. Outputs bit-identical to calls that always cut the chunks (layout 0),
    plain and grouped, at a small batch (many chunks per sequence) and a larger one;
    the first layer also against the oracle."""
    _log(f"decode layout record/reuse grouped={grouped} alone={n_alone}")
    K = _k()
    rng = np.random.default_rng(90 + n_alone)
    L, ps, Hq, Hkv, D = 3, 16, 32, 8, 128
    sizes, prefix = ([4, 3], [40, 9]) if grouped else ([], [])
    B = sum(sizes) + n_alone
    order = rng.permutation(B).tolist()
    next_page = iter(rng.permutation(np.arange(1, 12000)).tolist())
    lens, tables, members, pos = [0] * B, [None] * B, [], 0
    for gsz, pp in zip(sizes, prefix):
        shared = [next(next_page) for _ in range(pp)]
        ms = order[pos:pos + gsz]
        pos += gsz
        members.append(ms)
        for b in ms:
            own = int(rng.integers(1, own_max))
            lens[b] = pp * ps + own
            tables[b] = shared + [next(next_page) for _ in range(math.ceil(own / ps))]
    for b in order[pos:]:
        lens[b] = int(rng.integers(1, own_max))
        tables[b] = [next(next_page) for _ in range(math.ceil(lens[b] / ps))]
    P = 12000
    g = torch.Generator().manual_seed(91)
    gd = torch.Generator(device=DEV).manual_seed(91)
    kd = torch.randn(L, P, ps, Hkv, D, generator=gd, device=DEV, dtype=torch.float16)
    vd = torch.randn(L, P, ps, Hkv, D, generator=gd, device=DEV, dtype=torch.float16)
    k0, v0 = kd[0].cpu(), vd[0].cpu()
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    plan = (torch.from_numpy(indptr).to(DEV), torch.from_numpy(indices).to(DEV), torch.from_numpy(lpl).to(DEV),
            int(indptr[-1]))
    groups = K.DecodeGroups(B, members, prefix, DEV) if grouped else None
    ws_fresh, ws_rec = K.Workspace(DEV), K.Workspace(DEV)
    # another forward's plan: the first half of the batch, no groups
    h = max(1, B // 2)
    ip2, ix2, lp2 = O.plan_csr(tables[:h], lens[:h], ps)
    plan2 = (torch.from_numpy(ip2).to(DEV), torch.from_numpy(ix2).to(DEV), torch.from_numpy(lp2).to(DEV),
             int(ip2[-1]))
    tag = 1000 + n_alone
    for step in range(2):
        for layer in range(L):
            q = torch.randn(B, Hq, D, generator=g).half().to(DEV)
            want = K.paged_decode(q, kd[layer], vd[layer], *plan, workspace=ws_fresh, groups=groups, layout=0)
            lay = tag if layer == 0 else -tag
            got = K.paged_decode(q, kd[layer], vd[layer], *plan, workspace=ws_rec, groups=groups, layout=lay)
            torch.cuda.synchronize()
            assert torch.equal(_bits(got), _bits(want)), (step, layer)
            if step == 0 and layer == 0:
                ref = O.paged_attention_ref([q[b:b + 1].cpu() for b in range(B)], k0.view(-1, Hkv, D),
                                            v0.view(-1, Hkv, D), ps, indptr, indices, lpl, [1] * B)
                torch.testing.assert_close(got.cpu().float(), torch.stack([r[0] for r in ref]), atol=ATOL,
                                           rtol=RTOL)
        tag += 1
    # a record of another plan in between: the reusing call no longer finds its tag
    q = torch.randn(B, Hq, D, generator=g).half().to(DEV)
    K.paged_decode(q, kd[0], vd[0], *plan, workspace=ws_rec, groups=groups, layout=tag)
    K.paged_decode(q[:h], kd[0], vd[0], *plan2, workspace=ws_rec, layout=tag + 1)
    got = K.paged_decode(q, kd[1], vd[1], *plan, workspace=ws_rec, groups=groups, layout=-tag)
    want = K.paged_decode(q, kd[1], vd[1], *plan, workspace=ws_fresh, groups=groups, layout=0)
    torch.cuda.synchronize()
    assert torch.equal(_bits(got), _bits(want))


def test_decode_grouped_rejects_bad_groups():
    K = _k()
    lib = __import__("nanoslg_amd._lib", fromlist=["load"]).load()
    import ctypes
    B, Hq, Hkv, D, ps = 6, 32, 8, 128, 16
    q = torch.zeros(B, Hq, D, dtype=torch.float16, device=DEV)
    pool = torch.zeros(8, ps, Hkv, D, dtype=torch.float16, device=DEV)
    ip = torch.arange(B + 1, dtype=torch.int32, device=DEV)
    ix = torch.ones(B, dtype=torch.int32, device=DEV)
    lp = torch.full((B,), ps, dtype=torch.int32, device=DEV)
    slot = torch.full((B,), -1, dtype=torch.int32, device=DEV)
    ws = torch.zeros(1 << 24, dtype=torch.uint8, device=DEV)

    def call(num_groups, prefix, members):
        pp = (ctypes.c_int32 * max(1, len(prefix)))(*prefix)
        mm = (ctypes.c_int32 * (16 * max(1, num_groups)))(*([-1] * 16 * max(1, num_groups)))
        for i, x in enumerate(members):
            mm[i] = x
        return lib.nslg_paged_decode_grouped(q.data_ptr(), Hq * D, pool.data_ptr(), pool.data_ptr(), 8, ps,
                                             ip.data_ptr(), ix.data_ptr(), lp.data_ptr(), B, B, Hq, Hkv, D, 0.1, 0,
                                             slot.data_ptr(), num_groups, pp, mm, q.data_ptr(), Hq * D,
                                             ws.data_ptr(), ws.numel(), 0, None)
    assert call(0, [], []) == -2               # no group
    assert call(33, [1] * 33, [0]) == -2       # too many groups
    assert call(1, [0], [0, 1]) == -1          # empty prefix
    assert call(1, [1], [0, 1, 2, 3, 4]) == -1  # 5 members > 16 / G = 4
    assert call(1, [1], [0, 0]) == -1          # a sequence twice
    assert call(1, [1], [-1, 2]) == -1         # members not listed first
    assert call(1, [1], [0, 9]) == -1          # not a batch row
    assert call(2, [1, 1], [0, 1] + [-1] * 14 + [1]) == -1  # a sequence in two groups
    torch.cuda.synchronize()


@pytest.mark.parametrize("B,ps,seed", [(37, 16, 1), (5, 1, 2), (300, 16, 3)])
def test_block_table_csr_bit_exact(B, ps, seed):
    """The forward's CSR built from device-resident block-table rows
    (nslg_block_table_csr) equals the oracle's CSR of the same tables
    (kv_cache.py:598-615, missing pages -> the null page :606-607): rows partly
    synced (the rest from the upload), sequences needing more pages than they have,
    empty sequences; the uploaded entries land in the rows and no other arena entry
    changes."""
    _log(f"block table csr B={B} ps={ps}")
    from nanoslg_amd import kernels as K
    rng = np.random.default_rng(seed)
    have = [int(x) for x in rng.integers(0, 300, size=B)]
    have[0] = 0
    tables = [rng.integers(1, 1 << 20, size=h).tolist() for h in have]
    # tokens the forward sees: within the pages the sequence has, or past them
    lens = []
    for b, h in enumerate(have):
        if b % 7 == 3:
            lens.append((h + 2) * ps)          # two pages past the table: null pages
        elif h == 0:
            lens.append(0)
        else:
            lens.append(int(rng.integers((h - 1) * ps + 1, h * ps + 1)) if b % 5 else max(0, (h - 3) * ps))
    synced = [int(rng.integers(0, h + 1)) if h else 0 for h in have]
    # disjoint rows at random offsets of an arena filled with junk
    caps = [max(16, h + int(rng.integers(0, 40))) for h in have]
    order = rng.permutation(B)
    offs = np.zeros(B, np.int64)
    o = 0
    for b in order:
        offs[b] = o
        o += caps[b] + int(rng.integers(0, 9))
    arena = rng.integers(-5, 1 << 20, size=o + 64).astype(np.int32)
    for b in range(B):
        arena[offs[b]:offs[b] + synced[b]] = tables[b][:synced[b]]
    patch = [x for b in range(B) for x in tables[b][synced[b]:]] or [0]
    pip = np.zeros(B + 1, np.int32)
    np.cumsum([h - s for h, s in zip(have, synced)], out=pip[1:])
    indptr, indices, _ = O.plan_csr(tables, lens, ps)
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(DEV)  # noqa: E731
    d_arena = t(arena)
    d_idx = torch.full((max(int(indptr[-1]), 1),), -7, dtype=torch.int32, device=DEV)
    K.block_table_csr(d_arena, t(offs), t(have), t(synced), t(pip), t(patch), t(indptr), d_idx)
    torch.cuda.synchronize()
    n = int(indptr[-1])
    assert np.array_equal(d_idx.cpu().numpy()[:n], indices[:n])
    want = arena.copy()
    for b in range(B):
        want[offs[b]:offs[b] + have[b]] = tables[b]
    assert np.array_equal(d_arena.cpu().numpy(), want)


@pytest.mark.parametrize("B,ps,seed", [(37, 16, 11), (5, 1, 12), (300, 16, 13), (8, 16, 14)])
def test_forward_plan_csr_matches_the_two_launches(B, ps, seed):
    """nslg_forward_plan_csr (the CSR and the plan of a device-planned forward in one
    launch) against nslg_block_table_csr then nslg_forward_plan on copies of the same
    arena: the CSR, the arena rows, slots, positions, ragged rows and qo_indptr
    bit-identical; rows partly synced, sequences needing pages past their table,
    empty sequences, input offsets. The two launches are tied to the oracle by
    test_block_table_csr_bit_exact and the cache tests."""
    _log(f"forward plan csr B={B} ps={ps}")
    from nanoslg_amd import kernels as K
    rng = np.random.default_rng(seed)
    have = [int(x) for x in rng.integers(0, 80, size=B)]
    have[0] = 0
    tables = [rng.integers(1, 1 << 20, size=h).tolist() for h in have]
    lens, ntok = [], []
    for b, h in enumerate(have):
        L = (h + 2) * ps if b % 7 == 3 else (0 if h == 0 else int(rng.integers((h - 1) * ps + 1, h * ps + 1)))
        lens.append(L)
        ntok.append(int(rng.integers(0, min(L, 600) + 1)))
    start = [L - n for L, n in zip(lens, ntok)]
    offs_in = [int(rng.integers(0, 4)) for _ in range(B)]
    iw = max(o + n for o, n in zip(offs_in, ntok))
    T = sum(ntok)
    synced = [int(rng.integers(0, h + 1)) if h else 0 for h in have]
    caps = [max(16, h + int(rng.integers(0, 40))) for h in have]
    rows = np.zeros(B, np.int64)
    o = 0
    for b in rng.permutation(B):
        rows[b] = o
        o += caps[b] + int(rng.integers(0, 9))
    arena = rng.integers(-5, 1 << 20, size=o + 64).astype(np.int32)
    for b in range(B):
        arena[rows[b]:rows[b] + synced[b]] = tables[b][:synced[b]]
    patch = [x for b in range(B) for x in tables[b][synced[b]:]] or [0]
    pip = np.zeros(B + 1, np.int32)
    np.cumsum([h - s for h, s in zip(have, synced)], out=pip[1:])
    indptr = np.zeros(B + 1, np.int32)
    np.cumsum([(L + ps - 1) // ps for L in lens], out=indptr[1:])
    total = int(indptr[-1])
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(DEV)  # noqa: E731
    args = [t(rows), t(have), t(synced), t(pip), t(patch)]
    d_indptr, d_start, d_n, d_off = t(indptr), t(start), t(ntok), t(offs_in)
    outs, idxs, arenas = [], [], []
    for fused in (False, True):
        d_arena = t(arena)
        d_idx = torch.full((max(total, 1),), -7, dtype=torch.int32, device=DEV)
        out = torch.full((2 * B * iw + T + B + 1,), -9, dtype=torch.int32, device=DEV)
        if fused:
            res = K._forward_plan_csr(d_arena, *args, len(patch), d_indptr, d_idx, total, d_start, d_n, d_off, B, iw,
                                      ps, T, out)
        else:
            K._block_table_csr(d_arena, *args, len(patch), d_indptr, d_idx, total, B)
            res = K._forward_plan(d_indptr, d_idx, d_start, d_n, d_off, args[1], B, iw, ps, T, out=out)
        torch.cuda.synchronize()
        outs.append([r.cpu() for r in res])
        idxs.append(d_idx.cpu())
        arenas.append(d_arena.cpu())
    assert torch.equal(idxs[0], idxs[1]) and torch.equal(arenas[0], arenas[1])
    for a, b in zip(*outs):
        assert torch.equal(a, b)
    assert int(outs[1][3][-1]) == T and (outs[1][0] >= -1).all()


@pytest.mark.parametrize("B,ps,where", [(64, 16, "device"), (37, 4, "pinned"), (5, 16, "pinned")])
def test_decode_plan_step_device_list_bit_exact(B, ps, where):
    """nslg_decode_plan_step_device (the planner of a step replayed from a HIP graph:
    the opened-page list read from memory at run time, device or pinned host) equals
    the CSR the oracle builds from the extended block tables (kv_cache.py:598-615),
    with the new tokens' slots and positions and the opened pages in batch order;
    sequences whose last page is full or that have none open the page given, or the
    null page when given none."""
    _log(f"decode plan step (list in {where} memory) B={B} ps={ps}")
    import types
    from nanoslg_amd import kernels as K
    rng = np.random.default_rng(300 + B)
    lens = [int(x) for x in rng.integers(0, 3000, size=B)]
    for b in range(0, B, 4):
        lens[b] = ps * (b % 9)  # full last page (or empty): opens one
    npg = [math.ceil(L / ps) for L in lens]
    perm = rng.permutation(np.arange(1, sum(npg) + B + 10)).tolist()
    tables, off = [], 0
    for n in npg:
        tables.append(perm[off:off + n])
        off += n
    spare = perm[off:]
    indptr, indices, lpl = O.plan_csr(tables, lens, ps)
    opens = [L % ps == 0 for L in lens]
    new_page = np.full(B, -1, np.int32)
    for b in range(B):
        if opens[b] and b % 7 != 3:  # a few openers get no page: the null page
            new_page[b] = spare.pop()
    exp_tables = [t + ([int(new_page[b]) if new_page[b] >= 0 else 0] if opens[b] else []) for b, t in
                  enumerate(tables)]
    exp_lens = [L + 1 for L in lens]
    e_indptr, e_indices, e_lpl = O.plan_csr(exp_tables, exp_lens, ps)
    e_slot = [exp_tables[b][L // ps] * ps + L % ps for b, L in enumerate(lens)]
    e_new = [exp_tables[b][-1] for b in range(B) if opens[b]]
    cap = int(e_indptr[-1]) + 8
    z = lambda n: torch.full((n,), -9, dtype=torch.int32, device=DEV)  # noqa: E731
    dst = types.SimpleNamespace(indptr=z(B + 1), indices=z(cap), lpl=z(B), slot=z(B), pos=z(B), new_pages=z(B))
    if where == "device":
        new = torch.from_numpy(new_page).to(DEV)
    else:
        new = torch.from_numpy(new_page).pin_memory()
    t = lambda a: torch.from_numpy(np.asarray(a, np.int32)).to(DEV)  # noqa: E731
    K._decode_plan_step_device(t(indptr), t(indices), t(lpl), new, B, ps, dst, (None, None, 0, 0, 0, 0, 0))
    torch.cuda.synchronize()
    n = int(e_indptr[-1])
    assert np.array_equal(dst.indptr.cpu().numpy(), e_indptr)
    assert np.array_equal(dst.indices.cpu().numpy()[:n], e_indices[:n])
    assert np.array_equal(dst.lpl.cpu().numpy(), e_lpl)
    assert np.array_equal(dst.slot.cpu().numpy(), np.array(e_slot, np.int32))
    assert np.array_equal(dst.pos.cpu().numpy(), np.array(lens, np.int32))
    assert np.array_equal(dst.new_pages.cpu().numpy()[:len(e_new)], np.array(e_new, np.int32))
