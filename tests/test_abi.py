"""The C ABI library: it builds, loads, exports every symbol include/nslg_kv.h
declares, and rejects bad arguments on the host (no device work needed)."""
import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "nslg_kv.h"


def declared_symbols():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nslg_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    syms = declared_symbols()
    for name in ["nslg_append_kv", "nslg_zero_pages", "nslg_copy_pages", "nslg_gather_kv",
                 "nslg_paged_decode", "nslg_paged_decode_workspace_size", "nslg_paged_prefill",
                 "nslg_paged_prefill_workspace_size", "nslg_decode_plan_step", "nslg_rope_append",
                 "nslg_version",
                 "nslg_last_error"]:
        assert name in syms


def test_library_exports_every_declared_symbol():
    from nanoslg_amd import _lib
    lib = _lib.load()
    for name in declared_symbols():
        assert hasattr(lib, name), name
    assert set(declared_symbols()) == set(_lib.SIGNATURES)
    assert lib.nslg_version() >= 100


def test_host_side_argument_checks():
    from nanoslg_amd import _lib
    lib = _lib.load()
    # bad dtype, negative sizes, null pointers: rejected before any device work
    assert lib.nslg_append_kv(None, None, 0, 0, None, 4, None, None, 16, 8, 128, 9, None) == -1
    assert lib.nslg_append_kv(None, None, 0, 0, None, 0, None, None, 16, 8, 128, 0, None) == 0
    assert lib.nslg_zero_pages(None, None, 1, 4, 16, 8, 128, 0, None, 3, None) == -1
    assert lib.nslg_copy_pages(None, None, 0, 4, 16, 8, 128, 0, None, None, 1, None) == -1
    assert "copy_pages" in _lib.last_error()
    rc = lib.nslg_paged_decode(1, 4096, 1, 1, 100, 16, 1, 1, 1, 10, 2, 32, 8, 100, 0.1, 0, 1, 4096,
                               None, 0, 0, None)
    assert rc == -2  # head_dim 100 unsupported
    rc = lib.nslg_paged_decode(256, 4096, 256, 256, 100, 16, 1, 1, 1, 10, 2, 32, 8, 128, 0.1, 0, 256, 4096,
                               None, 0, 0, None)
    assert rc == -4  # no workspace
    rc = lib.nslg_paged_decode(256, 4096, 256, 256, 100, 16, 1, 1, 1, 10, 2, 34, 8, 128, 0.1, 0, 256, 4096,
                               None, 0, 0, None)
    assert rc == -1  # Hq not a multiple of Hkv
    # an fp32 decode long enough to be split over keys needs its workspace
    assert lib.nslg_paged_decode_workspace_size(1, 32, 8, 128, 2048, 16, 2) > (1 << 20)
    rc = lib.nslg_paged_decode(256, 4096, 256, 256, 4096, 16, 256, 256, 256, 2048, 1, 32, 8, 128, 0.1, 2, 256,
                               4096, None, 0, 0, None)
    assert rc == -4 and "workspace" in _lib.last_error()
    # prefill: the softmax scale must be positive and finite (the lazy running max
    # compares raw scores against a threshold divided by the scale)
    for bad in (0.0, -0.1, float("inf"), float("nan")):
        rc = lib.nslg_paged_prefill(256, 4096, 256, 8, 8, 256, 256, 100, 16, 256, 256, 256, 1, 32, 8, 128,
                                    bad, 0, 256, 4096, 256, 256, None)
        assert rc == -1 and "sm_scale" in _lib.last_error(), bad
    # device decode planner: too large a batch, null pointers, aliased outputs
    z = (None, None, 0, 0, 0, 0, 0)
    assert lib.nslg_decode_plan_step(1, 1, 1, 513, 16, 1, 2, 2, 2, 2, 2, 2, *z, None) == -2
    assert lib.nslg_decode_plan_step(None, 1, 1, 4, 16, 1, 2, 2, 2, 2, 2, 2, *z, None) == -1
    assert lib.nslg_decode_plan_step(1, 1, 1, 4, 16, 1, 2, 1, 2, 2, 2, 2, *z, None) == -1
    assert lib.nslg_decode_plan_step(None, None, None, 0, 16, None, None, None, None, None, None, None,
                                     *z, None) == 0
    nopage = (ctypes.c_int32 * 4)(-1, -1, -1, -1)
    assert lib.nslg_decode_plan_step(1, 1, 1, 4, 16, nopage, 2, 2, 2, 2, 2, 2, 256, None, 1, 10, 8, 128, 0,
                                     None) == -1  # half a pool


def test_decode_append_argument_checks():
    """nslg_paged_decode_append / _grouped_append: the new rows are checked on the host
    (present, not overlapping, aligned for the folded 16-byte writes) before any launch."""
    from nanoslg_amd import _lib
    lib = _lib.load()
    geo = (256, 256, 100, 16, 256, 256, 256, 10, 2, 32, 8, 128, 0.1)  # pools .. sm_scale
    tail = (256, 4096, None, 0, 0, None)  # out, out_stride, workspace, bytes, layout, stream
    # f16: k_new missing; rows overlapping (stride < Hkv*D); unaligned row stride / pointer
    assert lib.nslg_paged_decode_append(256, 4096, None, 1024, 256, 1024, *geo, 0, *tail) == -1
    assert "k_new" in _lib.last_error()
    assert lib.nslg_paged_decode_append(256, 4096, 256, 1000, 256, 1024, *geo, 0, *tail) == -1
    assert "overlap" in _lib.last_error()
    assert lib.nslg_paged_decode_append(256, 4096, 256, 1028, 256, 1024, *geo, 0, *tail) == -1
    assert "aligned" in _lib.last_error()
    assert lib.nslg_paged_decode_append(256, 4096, 258, 1024, 256, 1024, *geo, 0, *tail) == -1
    # fp32 rows only need 4-byte alignment: this one gets as far as the workspace check
    rc = lib.nslg_paged_decode_append(256, 4096, 260, 1028, 256, 1024, 256, 256, 4096, 16, 256, 256, 256, 2048, 1,
                                      32, 8, 128, 0.1, 2, *tail)
    assert rc == -4, _lib.last_error()
    # batch 0 is a no-op
    assert lib.nslg_paged_decode_append(None, 0, None, 0, None, 0, *geo[:8], 0, *geo[9:], 0, *tail) == 0
    members = (ctypes.c_int32 * 16)(0, 1, *([-1] * 14))
    prefix = (ctypes.c_int32 * 1)(4)
    rc = lib.nslg_paged_decode_grouped_append(256, 4096, None, 1024, 256, 1024, *geo, 0, 256, 1, prefix, members,
                                              *tail)
    assert rc == -1 and "k_new" in _lib.last_error()


def test_prefill_grid_argument_checks():
    """nslg_paged_prefill_grid: the grid rows map and the grid's shape are checked on
    the host before any launch."""
    from nanoslg_amd import _lib
    lib = _lib.load()
    tail = (256, 256, 100, 16, 256, 256, 256, 2, 32, 8, 128, 0.1, 0, 256, 4096, None, 0, None)
    assert lib.nslg_paged_prefill_grid(256, 4096, 256, None, 8, 10, 8, *tail) == -1
    assert "q_rows" in _lib.last_error()
    assert lib.nslg_paged_prefill_grid(256, 4096, 256, 256, 0, 10, 8, *tail) == -1  # no width
    assert lib.nslg_paged_prefill_grid(256, 4096, 256, 256, 4, 10, 8, *tail) == -1  # 10 tokens, 2 x 4 rows
    assert "grid" in _lib.last_error()


def test_prefill_append_argument_checks():
    """nslg_paged_prefill_append: the new rows' pointers, strides and alignment, and the
    pool dtype, are checked on the host before any launch; the fast-call binding
    returns the same statuses."""
    from nanoslg_amd import _lib
    lib, fast = _lib.load(), _lib.fast()
    A = 4096

    def call(k=A, ks=1024, v=A, vs=1024, dt=0, q_rows=None, width=0, D=128):
        args = (A, 4096, A, q_rows, width, 10, 8, k, ks, v, vs, A, A, 100, 16, A, A, A, 2, 32, 8, D, 0.1, dt,
                A, 4096, None, 0, None)
        rc = lib.nslg_paged_prefill_append(*args)
        assert fast.paged_prefill_append(*args) == rc
        return rc

    assert call(k=None) == -1 and "k_new" in _lib.last_error()
    assert call(v=None) == -1 and "k_new" in _lib.last_error()
    assert call(ks=1000) == -1 and "stride" in _lib.last_error()      # < Hkv * D
    assert call(vs=1028) == -1 and "16-byte" in _lib.last_error()     # rows not 16-byte aligned
    assert call(k=A + 8) == -1 and "16-byte" in _lib.last_error()
    assert call(dt=2) == -2 and "f16 or bf16" in _lib.last_error()   # fp32 pools: append, then prefill
    assert call(D=96) == -2 and "head_dim" in _lib.last_error()
    # rows spanning 4 GiB: 10 ragged rows at a 2^28-element stride
    assert call(ks=1 << 28) == -2 and "4 GiB" in _lib.last_error()
    assert call(q_rows=A, width=0) == -1 and "grid" in _lib.last_error()
    zero = (A, 4096, A, None, 0, 0, 0, None, 0, None, 0, A, A, 100, 16, A, A, A, 2, 32, 8, 128, 0.1, 0,
            A, 4096, None, 0, None)
    assert lib.nslg_paged_prefill_append(*zero) == 0  # no token: nothing to read, write or launch


def test_rope_append_argument_checks():
    from nanoslg_amd import _lib
    lib = _lib.load()
    # fused RoPE + append: unsupported head_dim, null pointers, misaligned stride, overlapping q_out
    A = 4096  # a 16-byte aligned stand-in address (never dereferenced: rejected first)
    ok = dict(q=A, qs=4096, qo=A, qos=4096, k=A, ks=1024, v=A, vs=1024, pos=A, slot=A, n=4, cos=A, sin=A,
              ts=128, tr=100, hq=32, hkv=8, d=128, kp=A, vp=A, slots=64, dt=0)

    def rope(**kw):
        a = dict(ok, **kw)
        return lib.nslg_rope_append(a["q"], a["qs"], a["qo"], a["qos"], a["k"], a["ks"], a["v"], a["vs"], a["pos"],
                                    a["slot"], a["n"], a["cos"], a["sin"], a["ts"], a["tr"], a["hq"], a["hkv"],
                                    a["d"], a["kp"], a["vp"], a["slots"], a["dt"], None)
    assert rope(d=96, ts=96) == -2
    assert rope(dt=7) == -2  # no such dtype (f16, bf16 and f32 are supported)
    assert rope(pos=None) == -1
    assert rope(qs=4092) == -1  # row stride smaller than Hq*D
    assert rope(ks=1028) == -1  # not a multiple of 8 elements
    assert rope(qo=A + 64) == -1  # q_out overlaps q
    assert rope(ts=64) == -1  # table rows shorter than D
    assert rope(n=0) == 0


def test_block_table_csr_argument_checks():
    from nanoslg_amd import _lib
    lib = _lib.load()
    A = 4096
    assert lib.nslg_block_table_csr(None, 0, None, None, None, None, None, 0, None, None, 0, 0, None) == 0
    assert lib.nslg_block_table_csr(A, 64, A, A, A, A, A, 1, A, A, 4, -1, None) == -1  # negative batch
    assert lib.nslg_block_table_csr(None, 64, A, A, A, A, A, 1, A, A, 4, 2, None) == -1  # no arena
    assert lib.nslg_block_table_csr(A, 64, A, A, A, A, None, 3, A, A, 4, 2, None) == -1  # patch missing
    assert "block_table_csr" in _lib.last_error()


def test_decode_rope_append_argument_checks():
    """nslg_paged_decode_rope_append / _grouped_rope_append: the rotary tables and
    positions are checked on the host (present, rows 16-byte aligned and at least
    head_dim wide, 16-bit pools only) before any launch; ctypes and the fast binding
    return the same statuses."""
    from nanoslg_amd import _lib
    lib, fast = _lib.load(), _lib.fast()
    A = 4096
    # q, k_new, v_new (rows aligned) | positions, cos, sin, stride, rows | pools .. sm_scale, dtype | out .. stream
    head = (A, 4096, A, 1024, A, 1024)
    geo = (A, A, 100, 16, A, A, A, 10, 2, 32, 8, 128, 0.1, 0)
    tail = (A, 4096, None, 0, 0, None)

    def both(rope, dtype=0):
        args = head + rope + geo[:-1] + (dtype,) + tail
        a, b = lib.nslg_paged_decode_rope_append(*args), fast.paged_decode_rope_append(*args)
        assert a == b
        return a

    assert both((A, None, A, 128, 100)) == -1                  # no cos table
    assert "tables" in _lib.last_error()
    assert both((None, A, A, 128, 100)) == -1                  # no positions
    assert both((A, A, A, 64, 100)) == -1                      # rows narrower than head_dim
    assert "stride" in _lib.last_error()
    assert both((A, A, A, 128, 0)) == -1                       # no rows
    assert both((A, A + 4, A, 128, 100)) == -1                 # table not 16-byte aligned
    assert "aligned" in _lib.last_error()
    assert both((A, A, A, 130, 100)) == -1                     # row stride not 16-byte aligned
    assert both((A, A, A, 128, 100), dtype=2) == -2            # fp32 pools: rope_append, then decode
    assert "f16/bf16" in _lib.last_error()
    # past the rope checks: the workspace is missing
    assert both((A, A, A, 128, 100)) == -4
    members = (ctypes.c_int32 * 16)(0, 1, *([-1] * 14))
    prefix = (ctypes.c_int32 * 1)(4)
    grp = (A, 1, ctypes.addressof(prefix), ctypes.addressof(members))
    args = head + (A, None, A, 128, 100) + geo + grp + tail
    assert lib.nslg_paged_decode_grouped_rope_append(*args) == fast.paged_decode_grouped_rope_append(*args) == -1
    zero_batch = head + (A, A, A, 128, 100) + geo[:8] + (0,) + geo[9:] + tail
    assert lib.nslg_paged_decode_rope_append(*zero_batch) == 0


def test_forward_plan_csr_argument_checks():
    """nslg_forward_plan_csr: the checks of both launches it fuses, on the host (the
    fast binding returns the same statuses)."""
    from nanoslg_amd import _lib
    lib, fast = _lib.load(), _lib.fast()
    A = 4096
    ok = (A, 64, A, A, A, A, A, 1, A, A, 4, A, A, A, 2, 8, 16, A, A, A, A, None)
    zero_batch = ok[:14] + (0,) + ok[15:]
    assert lib.nslg_forward_plan_csr(*zero_batch) == fast.forward_plan_csr(*zero_batch) == 0
    for k, bad, what in ((14, -1, "sizes"), (16, 0, "sizes"), (15, -1, "sizes"), (1, -1, "sizes"),
                         (0, None, "null"), (6, None, "null"), (11, None, "null"), (20, None, "null")):
        args = ok[:k] + (bad,) + ok[k + 1:]
        assert lib.nslg_forward_plan_csr(*args) == fast.forward_plan_csr(*args) == -1, k
        assert "forward_plan_csr" in _lib.last_error() and what in _lib.last_error(), k
    big = ok[:14] + (1 << 16,) + (1 << 16,) + ok[16:]
    assert lib.nslg_forward_plan_csr(*big) == -1 and "too large" in _lib.last_error()


def test_noalloc_decode_rejects_oversize_on_host():
    """nslg_paged_decode_noalloc refuses a call whose scratch need exceeds its static
    array before any device work (no device is touched here)."""
    from nanoslg_amd import _lib
    lib = _lib.load()
    # 1000 sequences over 2^20 pages: several hundred chunks of partials, > 16 MiB
    need = lib.nslg_paged_decode_workspace_size(1000, 32, 8, 128, 1 << 20, 16, 0)
    assert need > _lib.NSLG_NOALLOC_SCRATCH_BYTES
    A = 4096
    rc = lib.nslg_paged_decode_noalloc(A, 4096, A, A, 1 << 20, 16, A, A, A, 1 << 20, 1000, 32, 8, 128, 0.1, 0,
                                       A, 4096, None)
    assert rc == _lib.NSLG_EWORKSPACE and "static scratch" in _lib.last_error()


def test_decode_workspace_size_monotone():
    from nanoslg_amd import _lib
    lib = _lib.load()
    a = lib.nslg_paged_decode_workspace_size(4, 32, 8, 128, 640, 16, 0)
    b = lib.nslg_paged_decode_workspace_size(64, 64, 8, 128, 44000, 16, 0)  # group 8 vs 4
    assert 0 < a < b < (64 << 20)
    assert lib.nslg_paged_decode_workspace_size(4, 32, 8, 100, 640, 16, 0) == 0  # unsupported D


def test_missing_library_fails_loudly(tmp_path, monkeypatch):
    from nanoslg_amd import _lib
    monkeypatch.setattr(_lib, "_lib", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "nope.so")
    with pytest.raises(_lib.KernelLibraryError):
        _lib.load()


def test_attention_kernel_rejects_rows_not_16_byte_aligned():
    """Prefill on a padded grid takes only row strides of whole 16-byte units for q and
    out, on the MFMA kernel (16-bit pools, here at head_dim 256) and on the VALU kernel
    (fp32 pools) alike: their vector accesses and the pad-row zeroing store 16 bytes at
    a time."""
    from nanoslg_amd import _lib
    lib = _lib.load()
    A = 4096
    for dt, D, q_stride, out_stride in ((0, 256, 512, 516), (0, 256, 516, 512), (2, 128, 256, 258)):
        rc = lib.nslg_paged_prefill_grid(A, q_stride, A, A, 8, 10, 8, A, A, 100, 16, A, A, A, 2, 2, 1, D, 0.1,
                                         dt, A, out_stride, None, 0, None)
        assert rc == -1 and "16-byte" in _lib.last_error(), (dt, q_stride, out_stride, _lib.last_error())
    assert _lib.NSLG_ECAPTURE == -5


def test_fast_binding_calls_the_same_entry_points():
    """The fast-call binding of the per-step entry points (_nslg_fast) calls the same C
    functions as ctypes: the same statuses and error text from the host-side checks
    (no device work), and it refuses a wrong argument count or an int32 out of range."""
    from nanoslg_amd import _lib
    lib, fast = _lib.load(), _lib.fast()
    A = 4096
    dec = (A, 4096, A, A, 100, 16, A, A, A, 10, 2, 32, 8, 100, 0.1, 0, A, 4096, None, 0, 0, None)
    assert fast.paged_decode(*dec) == lib.nslg_paged_decode(*dec) == -2
    assert "head_dim" in _lib.last_error()
    app = (A, 4096, None, 1024, A, 1024, A, A, 100, 16, A, A, A, 10, 2, 32, 8, 128, 0.1, 0, A, 4096, None, 0, 0, None)
    assert fast.paged_decode_append(*app) == lib.nslg_paged_decode_append(*app) == -1
    assert "k_new" in _lib.last_error()
    zero = (None, 0, None, 0, None, 0, A, A, 100, 16, A, A, A, 0, 0, 32, 8, 128, 0.1, 0, None, 4096, None, 0, 0, None)
    assert fast.paged_decode_append(*zero) == 0
    members = (ctypes.c_int32 * 16)(0, 1, *([-1] * 14))
    prefix = (ctypes.c_int32 * 1)(4)
    mp, pp = ctypes.addressof(members), ctypes.addressof(prefix)
    grp = (A, 4096, A, A, 100, 16, A, A, A, 10, 2, 32, 8, 128, 0.1, 0, A, 0, pp, mp, A, 4096, None, 0, 0, None)
    assert fast.paged_decode_grouped(*grp) == lib.nslg_paged_decode_grouped(*grp) == -2  # no group
    gap = (A, 4096, None, 1024, A, 1024, A, A, 100, 16, A, A, A, 10, 2, 32, 8, 128, 0.1, 0, A, 1, pp, mp, A, 4096,
           None, 0, 0, None)
    assert fast.paged_decode_grouped_append(*gap) == lib.nslg_paged_decode_grouped_append(*gap) == -1
    z = (None, None, 0, 0, 0, 0, 0)
    plan = (1, 1, 1, 513, 16, 1, 2, 2, 2, 2, 2, 2, *z, None)
    assert fast.decode_plan_step(*plan) == lib.nslg_decode_plan_step(*plan) == -2
    rope = (A, 4096, A, 4096, A, 1024, A, 1024, A, A, 4, A, A, 96, 100, 32, 8, 96, A, A, 64, 0, None)
    assert fast.rope_append(*rope) == lib.nslg_rope_append(*rope) == -2
    with pytest.raises(TypeError):
        fast.paged_decode(*dec[:-1])
    with pytest.raises(OverflowError):
        fast.paged_decode(*dec[:10], 1 << 40, *dec[11:])  # batch is an int32


def test_fast_binding_signatures_match_the_header():
    """Each function of the fast-call binding converts its arguments by the same types
    as the ctypes declaration of its entry point (which test_library_exports_every_
    declared_symbol ties to include/nslg_kv.h)."""
    import re
    from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p
    from nanoslg_amd import _lib
    code = {c_void_p: "p", c_int64: "q", c_int32: "i", c_size_t: "z", c_float: "f"}
    src = (ROOT / "nanoslg_amd" / "csrc" / "fastcall.c").read_text()
    found = re.findall(r'parse\("(\w+)", "(\w+)"', src)
    assert len(found) == 17
    for fn, sig in found:
        assert sig == "".join(code[t] for t in _lib.SIGNATURES["nslg_" + fn][1]), fn
