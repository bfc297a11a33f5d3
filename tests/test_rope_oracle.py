"""Pins the varlen RoPE oracle (oracle/rope_oracle.py) without trusting its
own formulas:

  * the rotation as complex multiplication (x1 + i x2) e^{i angle}, in f64;
  * norm preservation of every (x_i, x_{i+D/2}) pair and the
    relative-position property <R(p) q, R(p') k> = f(p - p'), in f64;
  * position 0 leaves a row unchanged in every dtype; rotating back recovers
    the input (f64);
  * a packed batch equals each sequence rotated alone from position 0 (the
    reference's per-sequence loop, FNA2/attention_fna2.py:637-647);
  * the bf16/fp16 rounding helper against torch's own conversions;
  * torch's CPU evaluation of the reference formula in each dtype
    (attention_fna2.py:143-170: arange/outer/cat/cos/sin in the dtype, then
    x * cos + rotate_half(x) * sin) -- library routines, not the reference;
  * a planted mistake in the oracle fails one of these checks.
"""
import numpy as np
import pytest
import torch

from oracle import rope_oracle as RO


def _x(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def test_complex_form_f64():
    T, H, D = 37, 3, 16
    q, k = _x((T, H, D), 1), _x((T, 2, D), 2)
    inv = RO.inv_freq_default(D)
    cu = [0, 10, 37]
    yq, _ = RO.rope_varlen(q, k, cu, inv, "f64")
    pos, _ = RO.positions(cu, T)
    ang = np.outer(pos, inv.astype(np.float64))[:, None, :]
    z = (q[..., :D // 2] + 1j * q[..., D // 2:]) * np.exp(1j * ang)
    np.testing.assert_allclose(yq[..., :D // 2], z.real, atol=1e-12)
    np.testing.assert_allclose(yq[..., D // 2:], z.imag, atol=1e-12)


def test_norm_and_relative_position_f64():
    D = 32
    inv = RO.inv_freq_default(D)
    q, k = _x((1, 1, D), 3), _x((1, 1, D), 4)
    yq, yk = RO.rope_varlen(q, k, [0, 1], inv, "f64")
    h = D // 2
    np.testing.assert_allclose(yq[..., :h] ** 2 + yq[..., h:] ** 2,
                               q[..., :h] ** 2 + q[..., h:] ** 2, rtol=1e-12)

    def rot_at(x, p):
        c, s = RO.cos_sin(np.array([p]), inv, "f64")
        return RO.rotate(x, c, s, "f64")
    for p1, p2, shift in [(5, 2, 7), (100, 40, 13), (3, 3, 50)]:
        a = np.sum(rot_at(q, p1) * rot_at(k, p2))
        b = np.sum(rot_at(q, p1 + shift) * rot_at(k, p2 + shift))
        assert abs(a - b) < 1e-9


@pytest.mark.parametrize("dtype", ["f64", "f32", "f16", "bf16"])
def test_position_zero_is_identity(dtype):
    D = 16
    q = RO.round_to(_x((1, 2, D), 5), dtype)
    k = RO.round_to(_x((1, 1, D), 6), dtype)
    yq, yk = RO.rope_varlen(q, k, [0, 1], RO.inv_freq_default(D), dtype)
    np.testing.assert_array_equal(yq, q)
    np.testing.assert_array_equal(yk, k)


def test_rotate_back_f64():
    T, D = 50, 64
    q, k = _x((T, 4, D), 7), _x((T, 2, D), 8)
    inv = RO.inv_freq_default(D)
    cu = [0, 20, 50]
    yq, yk = RO.rope_varlen(q, k, cu, inv, "f64")
    bq, bk = RO.rope_varlen(yq, yk, cu, inv, "f64", sign=-1)
    np.testing.assert_allclose(bq, q, atol=1e-12)
    np.testing.assert_allclose(bk, k, atol=1e-12)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_packed_equals_per_sequence(dtype):
    lens = [5, 0, 17, 1, 40]
    cu = np.concatenate([[3], 3 + np.cumsum(lens)])  # tokens 0..2 and the tail: outside
    T = int(cu[-1]) + 4
    D = 32
    inv = RO.inv_freq_default(D)
    q = RO.round_to(_x((T, 2, D), 9), dtype)
    k = RO.round_to(_x((T, 1, D), 10), dtype)
    yq, yk = RO.rope_varlen(q, k, cu, inv, dtype)
    np.testing.assert_array_equal(yq[:3], q[:3])
    np.testing.assert_array_equal(yq[cu[-1]:], q[cu[-1]:])
    for b, n in enumerate(lens):
        s = slice(int(cu[b]), int(cu[b]) + n)
        aq, ak = RO.rope_varlen(q[s], k[s], [0, n], inv, dtype)
        np.testing.assert_array_equal(yq[s], aq)
        np.testing.assert_array_equal(yk[s], ak)


def test_rounding_helpers_match_torch():
    x = np.concatenate([_x(4000, 11) * 10.0 ** np.random.default_rng(12).integers(-30, 30, 4000),
                        [0.0, -0.0, np.inf, -np.inf, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9,
                         3.4e38, 1e-40, 65504.0, 65520.0]])
    x32 = x.astype(np.float32)
    for dt, tdt in (("bf16", torch.bfloat16), ("f16", torch.float16)):
        ours = RO.round_to(x32.astype(np.float64), dt)
        ref = torch.from_numpy(x32).to(tdt).to(torch.float64).numpy()
        np.testing.assert_array_equal(ours, ref)
    nan = RO.round_to(np.array([np.nan]), "bf16")
    assert np.isnan(nan).all()


def _torch_reference_formula(q, k, cu, inv, tdt):
    """The reference's per-sequence evaluation with torch ops on the CPU
    (attention_fna2.py:143-170, :637-647), restated."""
    q = torch.from_numpy(q).to(tdt)
    k = torch.from_numpy(k).to(tdt)
    inv_t = torch.from_numpy(inv)
    qo, ko = q.clone(), k.clone()

    def rot_half(x):
        h = x.shape[-1] // 2
        return torch.cat((-x[..., h:], x[..., :h]), dim=-1)
    for b in range(len(cu) - 1):
        s, e = int(cu[b]), int(cu[b + 1])
        if e == s:
            continue
        t = torch.arange(e - s, dtype=tdt)
        freqs = torch.outer(t, inv_t.to(tdt))
        emb = torch.cat((freqs, freqs), dim=-1)
        cos, sin = emb.cos()[:, None, :], emb.sin()[:, None, :]
        qo[s:e] = q[s:e] * cos + rot_half(q[s:e]) * sin
        ko[s:e] = k[s:e] * cos + rot_half(k[s:e]) * sin
    return qo.to(torch.float64).numpy(), ko.to(torch.float64).numpy()


@pytest.mark.parametrize("dtype,tdt", [("f32", torch.float32), ("bf16", torch.bfloat16),
                                       ("f16", torch.float16)])
def test_matches_torch_cpu_formula(dtype, tdt):
    cu = np.array([0, 300, 301, 900])
    T, D = 900, 64
    inv = RO.inv_freq_default(D)
    q = RO.round_to(_x((T, 2, D), 13), dtype)
    k = RO.round_to(_x((T, 1, D), 14), dtype)
    yq, yk = RO.rope_varlen(q, k, cu, inv, dtype)
    tq, tk = _torch_reference_formula(q, k, cu, inv, tdt)
    for a, b in ((yq, tq), (yk, tk)):
        if dtype == "f32":
            # torch's fp32 cos/sin vs the correctly rounded ones: a few ulp
            np.testing.assert_allclose(a, b, rtol=0, atol=2e-6)
        else:
            # equal except where cos/sin straddle a rounding boundary
            diff = np.abs(a - b)
            assert (diff == 0).mean() > 0.999
            ulp = 2.0 ** -7 if dtype == "bf16" else 2.0 ** -10
            assert (diff <= ulp * np.maximum(np.abs(b), 1.0) * 2).all()


def test_planted_mistake_is_caught(monkeypatch):
    """A sign error in the rotation must fail the complex-form check."""
    good = RO.rotate

    def bad(x, c, s, dtype, sign=1):
        return good(x, c, s, dtype, -sign)
    monkeypatch.setattr(RO, "rotate", bad)
    with pytest.raises(AssertionError):
        test_complex_form_f64()


# ── QK-RMSNorm + RoPE (oracle.rope_oracle.norm_rope_varlen / norm_rope_grads) ──

def _norm_case(seed=20):
    rng = np.random.default_rng(seed)
    T, D = 30, 16
    q, k = rng.standard_normal((T, 3, D)), rng.standard_normal((T, 2, D))
    wq, wk = rng.standard_normal(D), rng.standard_normal(D)
    return q, k, wq, wk, [2, 12, 25], RO.inv_freq_default(D)


def _torch_norm_rope(qt, kt, wqt, wkt, cu, inv, eps, table_dtype=torch.float64):
    """The reference chain (attention_fna2.py:95-103 then :163-170) in torch."""
    T, D = qt.shape[0], qt.shape[-1]
    pos, inside = RO.positions(cu, T)
    ang = torch.outer(torch.tensor(pos, dtype=table_dtype), torch.tensor(inv).to(table_dtype))
    c, s = ang.cos().to(qt.dtype)[:, None, :], ang.sin().to(qt.dtype)[:, None, :]
    out = []
    for x, w in ((qt, wqt), (kt, wkt)):
        xn = x * torch.rsqrt((x * x).mean(-1, keepdim=True) + eps) * w
        h = D // 2
        y = torch.cat([xn[..., :h] * c - xn[..., h:] * s, xn[..., h:] * c + xn[..., :h] * s], -1)
        out.append(torch.where(torch.tensor(inside)[:, None, None], y, x))
    return out


def test_norm_rope_grads_match_torch_autograd():
    q, k, wq, wk, cu, inv = _norm_case()
    rng = np.random.default_rng(21)
    gq, gk = rng.standard_normal(q.shape), rng.standard_normal(k.shape)
    dq, dk, dwq, dwk = RO.norm_rope_grads(q, k, cu, inv, wq, wk, 1e-6, gq, gk, table="f64")
    ts = [torch.tensor(a, requires_grad=True) for a in (q, k, wq, wk)]
    yq, yk = _torch_norm_rope(*ts, cu, inv, 1e-6)
    # the forward agrees too (f64 table)
    fq, fk = RO.norm_rope_varlen(q, k, cu, inv, wq, wk, 1e-6, "f64", table="f64")
    np.testing.assert_allclose(fq, yq.detach().numpy(), atol=1e-12)
    g = torch.autograd.grad([yq, yk], ts, [torch.tensor(gq), torch.tensor(gk)])
    for a, b in zip((dq, dk, dwq, dwk), g):
        np.testing.assert_allclose(a, b.numpy(), atol=1e-12)


def test_norm_rope_matches_torch_fp32_chain():
    """fp32 table at positions up to 700 (where an exact-angle table would
    differ by ~1e-5)."""
    rng = np.random.default_rng(22)
    q, k = rng.standard_normal((700, 2, 16)), rng.standard_normal((700, 1, 16))
    wq, wk = rng.standard_normal(16), rng.standard_normal(16)
    cu, inv = [0, 700], RO.inv_freq_default(16)
    ts = [torch.tensor(a, dtype=torch.float32) for a in (q, k, wq, wk)]
    yq, yk = _torch_norm_rope(*ts, cu, inv, 1e-6, table_dtype=torch.float32)
    fq, fk = RO.norm_rope_varlen(q.astype(np.float32), k.astype(np.float32), cu, inv,
                                 wq.astype(np.float32), wk.astype(np.float32), 1e-6, "f32")
    np.testing.assert_allclose(fq, yq.numpy(), atol=5e-6)
    np.testing.assert_allclose(fk, yk.numpy(), atol=5e-6)


def test_norm_rope_scale_invariant():
    q, k, wq, wk, cu, inv = _norm_case(23)
    a = RO.norm_rope_varlen(q, k, cu, inv, wq, wk, 0.0, "f64", table="f64")
    b = RO.norm_rope_varlen(3.7 * q, 0.2 * k, cu, inv, wq, wk, 0.0, "f64", table="f64")
    pos, inside = RO.positions(cu, q.shape[0])
    np.testing.assert_allclose(a[0][inside], b[0][inside], atol=1e-12)
    np.testing.assert_allclose(a[1][inside], b[1][inside], atol=1e-12)


def test_norm_rope_planted_mistake_is_caught(monkeypatch):
    """A dropped 1/D in the norm gradient must fail the autograd check."""
    good = RO.norm_rope_grads

    def bad(q, k, cu, inv, wq, wk, eps, gq, gk, table="f32"):
        dq, dk, dwq, dwk = good(q, k, cu, inv, wq, wk, eps, gq, gk, table)
        return dq * 1.01, dk, dwq, dwk
    monkeypatch.setattr(RO, "norm_rope_grads", bad)
    with pytest.raises(AssertionError):
        test_norm_rope_grads_match_torch_autograd()
