"""CPU restatement of the reference's varlen rotary embedding (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``fna2_amd``) imports this
module; only ``tests/`` and ``bench.py`` use it, and only as the checker.

What it restates (reference = myAiByMe/FNA2, ``FNA2/attention_fna2.py``):

* ``NaylisAttention._apply_rope_varlen`` (:620-647): the packed sequences
  are rotated one by one with positions 0 .. len-1 (the reference walks
  ``cu_seqlens[1:] - cu_seqlens[:-1]`` from offset 0); tokens it does not
  reach keep their values here (it leaves them uninitialised).
* ``RotaryPositionalEmbedding._update_cache`` (:143-155): positions
  ``arange(n)`` and ``inv_freq`` in the tensor's dtype, the angle table
  ``outer(t, inv_freq)`` rounded to that dtype, repeated for both halves
  (``cat((freqs, freqs))``), then ``cos``/``sin`` rounded to that dtype.
* ``forward`` / ``_rotate_half`` (:158-170): ``x * cos + rotate_half(x) * sin``
  with ``rotate_half(x) = cat(-x2, x1)``: each product and the sum are
  separate elementwise ops of the dtype (computed in fp32, rounded).
* ``sign = -1``: the rotation by ``-angle``, i.e. autograd's gradient
  ``g * cos + rotate_half^T(g * sin)`` with the same rounding.

cos and sin are computed in float64 and rounded to fp32 first (an accurate
fp32 routine), then to the dtype, as torch does for bf16/fp16 tensors.
``dtype = "f64"`` skips every rounding (exact rotation, for the invariants).

* ``norm_rope_varlen``: ``RMSNorm`` (attention_fna2.py:95-103,
  ``x * rsqrt(mean(x^2) + eps) * weight``) of every (token, head) row before
  the rotation (``q_norm`` / ``k_norm`` then RoPE, :553-566), with the
  angle table in fp32 (``table="f32"``: the reference's fp32 table; "f64":
  exact angles) and the rest in float64, rounded once to the dtype: the
  fused kernel computes the chain in fp32.  ``norm_rope_grads`` gives
  its gradients (inputs and norm weights) for an upstream gradient.

Pinning (tests/test_rope_oracle.py): the complex-multiplication form of the
rotation, norm preservation and the relative-position property in f64, the
identity at position 0, rotate/rotate-back, per-sequence restarts, the
bf16 rounding helper against torch's conversion, and torch's own CPU
evaluation of the reference formula in each dtype.
"""
from __future__ import annotations

import numpy as np


def round_to(x, dtype: str) -> np.ndarray:
    """Round float64 values to the dtype (round to nearest even), as float64."""
    x = np.asarray(x, dtype=np.float64)
    if dtype == "f64":
        return x
    if dtype == "f32":
        return x.astype(np.float32).astype(np.float64)
    if dtype == "f16":
        with np.errstate(over="ignore"):  # out of range: inf, as the conversion gives
            return x.astype(np.float32).astype(np.float16).astype(np.float64)
    if dtype == "bf16":
        f = x.astype(np.float32)
        u = f.view(np.uint32).astype(np.uint64)
        nan = np.isnan(f)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        out = r.astype(np.uint32).view(np.float32)
        out = np.where(nan, np.float32(np.nan), out)
        return out.astype(np.float64)
    raise ValueError(dtype)


def positions(cu_seqlens, total: int):
    """Position of each token and whether a sequence covers it
    (attention_fna2.py:637-647: sequence b covers [cu[b], cu[b+1]))."""
    cu = np.asarray(cu_seqlens, dtype=np.int64)
    t = np.arange(total)
    b = np.searchsorted(cu, t, side="right") - 1
    inside = (b >= 0) & (b < len(cu) - 1)
    pos = np.where(inside, t - cu[np.clip(b, 0, len(cu) - 1)], 0)
    return pos, inside


def cos_sin(pos, inv_freq, dtype: str):
    """cos/sin table rows [T, D/2] (attention_fna2.py:148-154)."""
    inv = np.asarray(inv_freq, dtype=np.float64)
    if dtype == "f64":
        ang = np.outer(pos.astype(np.float64), inv)
        return np.cos(ang), np.sin(ang)
    inv_r = round_to(round_to(inv, "f32"), dtype)  # the fp32 buffer cast to the dtype
    pos_r = round_to(pos.astype(np.float64), dtype)
    ang = round_to(np.outer(pos_r, inv_r), dtype)  # fp32 product of two dtype values: exact
    c = round_to(round_to(np.cos(ang), "f32"), dtype)
    s = round_to(round_to(np.sin(ang), "f32"), dtype)
    return c, s


def rotate(x, c, s, dtype: str, sign: int = 1):
    """x [T, H, D]; c, s [T, D/2]: x * cos + rotate_half(x) * sin, rounded as
    elementwise ops of the dtype (attention_fna2.py:158-170)."""
    x = np.asarray(x, dtype=np.float64)
    h = x.shape[-1] // 2
    x1, x2 = x[..., :h], x[..., h:]
    c = c[:, None, :]
    s = sign * s[:, None, :]
    r = lambda v: round_to(v, dtype)
    y1 = r(r(x1 * c) + r(-x2 * s))
    y2 = r(r(x2 * c) + r(x1 * s))
    return np.concatenate([y1, y2], axis=-1)


def rope_varlen(q, k, cu_seqlens, inv_freq, dtype: str, sign: int = 1):
    """Rotated q [T, H, D] and k [T, H_KV, D] (float64 arrays holding dtype
    values); tokens outside every sequence unchanged."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    pos, inside = positions(cu_seqlens, q.shape[0])
    c, s = cos_sin(pos, inv_freq, dtype)
    out = []
    for x in (q, k):
        y = rotate(x, c, s, dtype, sign)
        out.append(np.where(inside[:, None, None], y, x))
    return out[0], out[1]


def inv_freq_default(dim: int, base: float = 10000.0) -> np.ndarray:
    """1 / base^(2i/dim) as the fp32 buffer of attention_fna2.py:121-122."""
    i = np.arange(0, dim, 2, dtype=np.float32)
    return (1.0 / (np.float32(base) ** (i / np.float32(dim)))).astype(np.float32)


def _rms_norm(x, w, eps):
    x = np.asarray(x, dtype=np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x * r * np.asarray(w, dtype=np.float64), r


def norm_rope_varlen(q, k, cu_seqlens, inv_freq, wq, wk, eps: float, dtype: str,
                     table: str = "f32"):
    """RMSNorm (weights wq / wk, None: no norm) then the rotation, in float64
    with the angle table in ``table`` precision, rounded once to the dtype.
    Tokens outside every sequence unchanged."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    pos, inside = positions(cu_seqlens, q.shape[0])
    c, s = cos_sin(pos, inv_freq, table)
    out = []
    for x, w in ((q, wq), (k, wk)):
        xn = x if w is None else _rms_norm(x, w, eps)[0]
        y = round_to(rotate(xn, c, s, "f64"), dtype)
        out.append(np.where(inside[:, None, None], y, x))
    return out[0], out[1]


def norm_rope_grads(q, k, cu_seqlens, inv_freq, wq, wk, eps: float, gq, gk,
                    table: str = "f32"):
    """Gradients of sum(gq * y_q) + sum(gk * y_k) for y = rotate(RMSNorm(x)):
    (dq, dk, dwq, dwk) in float64.  dx = r (w . g') - x r^3 <x, w . g'> / D with
    g' = rotate^-1(g); dw = sum over rows of x r g'.  Outside tokens pass the
    gradient through unchanged (and add nothing to dw)."""
    pos, inside = positions(cu_seqlens, np.asarray(q).shape[0])
    c, s = cos_sin(pos, inv_freq, table)
    res = []
    for x, w, g in ((q, wq, gq), (k, wk, gk)):
        x = np.asarray(x, dtype=np.float64)
        g = np.asarray(g, dtype=np.float64)
        gr = rotate(g, c, s, "f64", sign=-1)  # the rotation's transpose
        if w is None:
            dx, dw = gr, None
        else:
            w = np.asarray(w, dtype=np.float64)
            D = x.shape[-1]
            r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
            wg = w * gr
            dx = r * wg - x * r ** 3 * np.sum(x * wg, axis=-1, keepdims=True) / D
            dw = np.sum(np.where(inside[:, None, None], x * r * gr, 0.0), axis=(0, 1))
        dx = np.where(inside[:, None, None], dx, g)
        res.append((dx, dw))
    return res[0][0], res[1][0], res[0][1], res[1][1]

