"""Pins of the oracle's rotary position embedding (nanoslg/models.py:37-105): the
tables against transformers' own inverse frequencies and closed forms, the
rotation against a float64 restatement, and planted mistakes that these checks
must catch. CPU only."""
import math

import numpy as np
import pytest
import torch

from oracle import kv_oracle as O

LLAMA3 = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0, "high_freq_factor": 4.0,
          "original_max_position_embeddings": 8192}


def test_inv_freq_matches_transformers_llama3():
    """Llama-3.1's scaled frequencies, from transformers' own routine (a library)."""
    from transformers import LlamaConfig
    from transformers import modeling_rope_utils as mru
    params = dict(LLAMA3, rope_theta=500000.0)
    params.pop("rope_type")
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32, head_dim=128, max_position_embeddings=131072,
                      rope_parameters=dict(params, rope_type="llama3"))
    lib, _ = mru._compute_llama3_parameters(cfg)
    mine = O.rope_inv_freq(128, 500000.0, LLAMA3)
    assert mine.dtype == torch.float32 and mine.shape == (64,)
    assert torch.equal(lib, mine)


def test_inv_freq_closed_forms():
    """Unscaled: theta^(-2i/dim). Scaled: the three wavelength bands of the llama3 rule."""
    dim, theta = 128, 500000.0
    plain = O.rope_inv_freq(dim, theta).double().numpy()
    exact = theta ** (-np.arange(0, dim, 2) / dim)
    assert np.allclose(plain, exact, rtol=2e-6, atol=0)
    scaled = O.rope_inv_freq(dim, theta, LLAMA3).double().numpy()
    wl = 2 * math.pi / plain
    hi_band = wl < 8192 / 4.0
    lo_band = wl > 8192 / 1.0
    mid = ~hi_band & ~lo_band
    assert hi_band.any() and lo_band.any() and mid.any()
    assert np.array_equal(scaled[hi_band], plain[hi_band])
    assert np.allclose(scaled[lo_band], plain[lo_band] / 8.0, rtol=1e-7, atol=0)
    s = (8192 / wl[mid] - 1.0) / (4.0 - 1.0)
    assert np.allclose(scaled[mid], (1 - s) * plain[mid] / 8.0 + s * plain[mid], rtol=2e-6, atol=0)


def test_tables_closed_forms():
    cos, sin = O.rope_tables(64, 3000, 10000.0)
    assert cos.shape == sin.shape == (3000, 64) and cos.dtype == torch.float32
    assert torch.equal(cos[0], torch.ones(64)) and torch.equal(sin[0], torch.zeros(64))
    f = O.rope_inv_freq(64, 10000.0)
    t = torch.arange(3000, dtype=torch.float32)
    ang32 = torch.outer(t, f).double().numpy()  # the float32 angles the tables use
    assert np.allclose(cos[:, :32].double().numpy(), np.cos(ang32), atol=2e-6)
    assert np.allclose(sin[:, 32:].double().numpy(), np.sin(ang32), atol=2e-6)
    assert torch.equal(cos[:, :32], cos[:, 32:])


def _rows(dtype, N=64, H=4, D=128, seed=0):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(1, N, H, D, generator=g).to(dtype)


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 2e-2), (torch.bfloat16, 1.2e-1)])
def test_rotation_matches_float64(dtype, tol):
    """apply_rotary_ref = the float64 rotation up to 16-bit rounding of the tables,
    the two products and the sum (a few units in the last place of |x| <= ~5)."""
    N, D = 256, 128
    x = _rows(dtype, N=N, D=D)
    pos = torch.randint(0, 131072, (1, N), generator=torch.Generator().manual_seed(1))
    pos[0, :3] = torch.tensor([0, 1, 131071])
    cos, sin = O.rope_tables(D, 131072, 500000.0, LLAMA3)
    out = O.apply_rotary_ref(x, cos[pos], sin[pos]).double().numpy()[0]
    # the closed form uses the tables' own float32 angles, so only the rotation is tested
    ang = torch.outer(torch.arange(131072, dtype=torch.float32), O.rope_inv_freq(D, 500000.0, LLAMA3))
    a = ang[pos[0]].double().numpy()
    xs = x[0].double().numpy()
    c, s = np.cos(a)[:, None, :], np.sin(a)[:, None, :]
    ref = np.concatenate([xs[..., :64] * c - xs[..., 64:] * s, xs[..., 64:] * c + xs[..., :64] * s], -1)
    assert np.abs(out - ref).max() < tol
    # planted mistakes, each of which the same check must reject
    half = D // 2
    x1, x2 = x[..., :half], x[..., half:]
    cc = cos[pos][:, :, None, :].to(dtype)
    ss = sin[pos][:, :, None, :].to(dtype)
    wrong_sign = x * cc + torch.cat((x2, -x1), -1) * ss
    wrong_half = x * cc + torch.cat((-x1, x2), -1) * ss
    wrong_table = x * ss + torch.cat((-x2, x1), -1) * cc
    for w in (wrong_sign, wrong_half, wrong_table):
        assert np.abs(w.double().numpy()[0] - ref).max() > 10 * tol


def test_rotation_special_angles():
    """Position 0 leaves x unchanged; a quarter turn (c rounds to zero, s = 1) gives
    exactly cat(-x2, x1)."""
    x = _rows(torch.float16, N=8)
    D = x.shape[-1]
    one, zero = torch.ones(1, 8, D), torch.zeros(1, 8, D)
    assert torch.equal(O.apply_rotary_ref(x, one, zero), x)
    c = torch.full((1, 8, D), math.cos(np.float32(math.pi / 2)))  # -4.4e-8: rounds to -0 in fp16
    assert torch.equal(O.apply_rotary_ref(x, c, one), torch.cat((-x[..., D // 2:], x[..., :D // 2]), -1))


def test_rope_forward_gathers_positions():
    """rope_forward_ref uses the table row of each position, for q and k alike."""
    cos, sin = O.rope_tables(64, 100, 10000.0)
    q, k = _rows(torch.float16, N=5, H=4, D=64), _rows(torch.float16, N=5, H=2, D=64, seed=3)
    pos = torch.tensor([[7, 0, 99, 3, 3]])
    qr, kr = O.rope_forward_ref(q, k, cos, sin, pos)
    for t, p in enumerate(pos[0].tolist()):
        one = torch.tensor([[p]])
        assert torch.equal(qr[:, t:t + 1], O.apply_rotary_ref(q[:, t:t + 1], cos[one], sin[one]))
        assert torch.equal(kr[:, t:t + 1], O.apply_rotary_ref(k[:, t:t + 1], cos[one], sin[one]))


def test_rotate_f64_invariants():
    """The float64 rotation preserves pair norms and composes: R(a) R(b) = R(a + b)."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal((16, 2, 32))
    f = 10000.0 ** (-np.arange(0, 32, 2) / 32)
    a, b = rng.integers(0, 5000, 16), rng.integers(0, 5000, 16)
    ra = O.rotate_f64(x, a, f)
    n0 = x[..., :16] ** 2 + x[..., 16:] ** 2
    n1 = ra[..., :16] ** 2 + ra[..., 16:] ** 2
    assert np.allclose(n0, n1, rtol=1e-12, atol=1e-12)
    assert np.allclose(O.rotate_f64(ra, b, f), O.rotate_f64(x, a + b, f), atol=1e-9)
    assert np.allclose(O.rotate_f64(x, np.zeros(16), f), x)
