"""CPU restatement of FlashNaylisAttention-2 forward and backward (numpy).

TEST INFRASTRUCTURE ONLY.  Nothing in the product (``fna2_amd``) imports this
module; only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, and only as the checker.

What it restates (reference = myAiByMe/FNA2, ``FNA2/``):

* Score: ``S = scale * Q K^T + [h < H_G] * gs[h] * Rq Rk^T``
  (flash_naylis_attn.py:157-165, validate_fna2.py:97-99), GQA KV head
  ``h // (H // H_KV)`` (flash_naylis_attn.py:105), vanilla heads
  ``h >= H_G`` carry no bias (flash_naylis_attn.py:121-130).
* Mask: causal ``j <= i`` on local positions (top-left aligned, also in varlen,
  flash_naylis_attn.py:168-170, :322-323); keys beyond the sequence masked
  (:173-174, :325-326).  Non-causal is the same without the causal term (the
  reference's dense kernel supports it, :138-143; its varlen kernel does not,
  which this restatement extends).
* Normalisation: ``O = sum_j exp(S - m) V / (l + 1e-6)``,
  ``LSE = m + log(l + 1e-6)`` (flash_naylis_attn.py:192-195, :340-341).
  A query row with no visible key gives O = 0 and LSE = -inf (the reference
  leaves such rows undefined).
* Backward: ``P = exp(S - LSE)``, ``delta = sum_d dO * O``
  (flash_naylis_attn.py:381), ``dS = P (dO V^T - delta)`` (:522-523),
  ``dV = P^T dO``, ``dK = scale dS^T Q``, ``dRk = gs dS^T Rq``,
  ``d_gs = sum dS * (Rq Rk^T)`` (:526-538), ``dQ = scale dS K``,
  ``dRq = gs dS Rk`` (:678-683); dK/dV summed over each GQA group;
  varlen gradients of graph_scale summed over sequences
  (validate_fna2.py:325).

Layouts follow the reference API: dense q ``[B,H,S,D]``, k/v ``[B,H_KV,S,D]``,
r ``[B,H_G,S,R]``, lse ``[B,H,S]``; varlen q ``[T,H,D]``, lse ``[T,H]`` with
``cu_seqlens`` int32 offsets.

* Decode (``decode``): one query row per sequence against the first len_b
  rows of a KV cache, all visible -- the reference's decode step with the
  graph bias kept when an Rk cache is given (attention_fna2.py:412-429).

Pinning (tests/test_oracle.py): a pure-Python brute force on tiny inputs,
torch's ``scaled_dot_product_attention`` (``is_causal=True`` with gs = 0, an
explicit float mask otherwise), torch autograd of that library forward at
eps = 0, central finite differences of this module's own forward, and the
identities ``O_0 = V_0`` (causal), key-permutation invariance (non-causal),
``sum_j dS_ij = 0`` and ``gs * d_gs = <Rq, dRq> = <Rk, dRk>``.
"""
from __future__ import annotations

import numpy as np

EPS = 1e-6
_BLOCK = 1024  # query rows per chunk (bounds memory at long lengths)


def _as(x, dtype):
    if x is None:
        return None
    if hasattr(x, "detach"):  # torch tensor
        x = x.detach().float().cpu().numpy()
    return np.asarray(x, dtype=dtype)


def _mask(i0, nq, lk, causal):
    """Boolean [nq, lk] visibility for query rows i0..i0+nq-1."""
    qi = np.arange(i0, i0 + nq)[:, None]
    kj = np.arange(lk)[None, :]
    vis = np.ones((nq, lk), dtype=bool)
    if causal:
        vis &= kj <= qi
    return vis


def _scores(Qb, K, Rqb, Rk, g, scale):
    S = scale * (Qb @ K.T)
    if Rqb is not None:
        S = S + g * (Rqb @ Rk.T)
    return S


def head_forward(Q, K, V, Rq, Rk, g, scale, causal, eps=EPS):
    """One (sequence, head): Q [Lq,D], K/V [Lk,D], Rq [Lq,R] / Rk [Lk,R] or None."""
    lq, lk = Q.shape[0], K.shape[0]
    O = np.zeros((lq, V.shape[1]), dtype=Q.dtype)
    lse = np.full((lq,), -np.inf, dtype=Q.dtype)
    if lk == 0:
        return O, lse
    for i0 in range(0, lq, _BLOCK):
        nq = min(_BLOCK, lq - i0)
        kend = min(lk, i0 + nq) if causal else lk
        if kend == 0:
            continue
        Rqb = None if Rq is None else Rq[i0:i0 + nq]
        Rkk = None if Rk is None else Rk[:kend]
        S = _scores(Q[i0:i0 + nq], K[:kend], Rqb, Rkk, g, scale)
        vis = _mask(i0, nq, kend, causal)
        S = np.where(vis, S, -np.inf)
        m = S.max(axis=1)
        live = np.isfinite(m)
        msafe = np.where(live, m, 0.0)
        P = np.exp(S - msafe[:, None])
        l = P.sum(axis=1)
        O[i0:i0 + nq] = (P @ V[:kend]) / (l + eps)[:, None]
        lse[i0:i0 + nq] = np.where(live, m + np.log(l + eps), -np.inf)
    return O, lse


def head_backward(dO, Q, K, V, Rq, Rk, g, scale, causal, O, lse):
    """Gradients of one (sequence, head); returns dQ, dK, dV, dRq, dRk, dg."""
    lq, lk = Q.shape[0], K.shape[0]
    dQ = np.zeros_like(Q)
    dK = np.zeros_like(K)
    dV = np.zeros_like(V)
    dRq = None if Rq is None else np.zeros_like(Rq)
    dRk = None if Rk is None else np.zeros_like(Rk)
    dg = 0.0
    if lk == 0 or lq == 0:
        return dQ, dK, dV, dRq, dRk, dg
    delta = (dO * O).sum(axis=1)
    for i0 in range(0, lq, _BLOCK):
        nq = min(_BLOCK, lq - i0)
        kend = min(lk, i0 + nq) if causal else lk
        if kend == 0:
            continue
        sl = slice(i0, i0 + nq)
        Rqb = None if Rq is None else Rq[sl]
        Rkk = None if Rk is None else Rk[:kend]
        S = _scores(Q[sl], K[:kend], Rqb, Rkk, g, scale)
        vis = _mask(i0, nq, kend, causal)
        lrow = lse[sl][:, None]
        P = np.where(vis & np.isfinite(lrow), np.exp(np.where(vis, S, 0.0) - np.where(np.isfinite(lrow), lrow, 0.0)), 0.0)
        dP = dO[sl] @ V[:kend].T
        dS = P * (dP - delta[sl][:, None])
        dV[:kend] += P.T @ dO[sl]
        dK[:kend] += scale * (dS.T @ Q[sl])
        dQ[sl] = scale * (dS @ K[:kend])
        if Rq is not None:
            dRq[sl] = g * (dS @ Rkk)
            dRk[:kend] += g * (dS.T @ Rqb)
            dg += float(np.sum(dS * (Rqb @ Rkk.T)))
    return dQ, dK, dV, dRq, dRk, dg


def head_rows(dO, Q, K, V, Rq, Rk, g, scale, causal, rows, eps=EPS):
    """The row-local results of one (sequence, head) for the query rows
    ``rows`` only: (out, lse, dQ, dRq) of those rows, each of which needs every
    key but no other query row -- the same formulas as ``head_forward`` and
    ``head_backward`` (delta from these rows' own output), for checking long
    sequences on a row subset.  (dK, dV, dRk and dg sum over every query row
    and are not row-local.)"""
    i = np.asarray(rows, dtype=np.int64)
    lk = K.shape[0]
    Rqi = None if Rq is None else Rq[i]
    S = _scores(Q[i], K, Rqi, Rk, g, scale)
    vis = np.ones((len(i), lk), dtype=bool)
    if causal:
        vis &= np.arange(lk)[None, :] <= i[:, None]
    S = np.where(vis, S, -np.inf)
    m = S.max(axis=1) if lk else np.full(len(i), -np.inf)
    live = np.isfinite(m)
    msafe = np.where(live, m, 0.0)
    P = np.where(vis, np.exp(S - msafe[:, None]), 0.0)
    l = P.sum(axis=1)
    O = (P @ V) / (l + eps)[:, None]
    lse = np.where(live, m + np.log(l + eps), -np.inf)
    Pn = np.where(vis & live[:, None], np.exp(np.where(vis, S, 0.0) - np.where(live, lse, 0.0)[:, None]), 0.0)
    delta = (dO[i] * O).sum(axis=1)
    dS = Pn * (dO[i] @ V.T - delta[:, None])
    dQ = scale * (dS @ K)
    dRq = None if Rq is None else g * (dS @ Rk)
    return O, lse, dQ, dRq


def _segments(varlen, n, cu_q, cu_k, Sq, Sk):
    if varlen:
        cq = np.asarray(cu_q, dtype=np.int64)
        ck = np.asarray(cu_k, dtype=np.int64)
        return [(int(cq[b]), int(cq[b + 1]), int(ck[b]), int(ck[b + 1])) for b in range(len(cq) - 1)]
    return [(0, Sq, 0, Sk)] * n


def forward(q, k, v, rq, rk, gs, scale, causal=True, cu_q=None, cu_k=None,
            dtype=np.float64, eps=EPS):
    """Forward pass.  Returns (out, lse) in the API layouts (numpy, ``dtype``)."""
    varlen = cu_q is not None
    q, k, v = _as(q, dtype), _as(k, dtype), _as(v, dtype)
    rq, rk, gs = _as(rq, dtype), _as(rk, dtype), _as(gs, dtype)
    H = q.shape[1] if varlen else q.shape[1]
    H_KV = k.shape[1]
    H_G = 0 if rq is None else rq.shape[1]
    G = H // H_KV
    if varlen:
        out = np.zeros_like(q)
        lse = np.full(q.shape[:2], -np.inf, dtype=dtype)
        for (qs, qe, ks, ke) in _segments(True, 0, _as(cu_q, np.int64), _as(cu_k, np.int64), 0, 0):
            for h in range(H):
                g = h < H_G
                o, l = head_forward(q[qs:qe, h], k[ks:ke, h // G], v[ks:ke, h // G],
                                    rq[qs:qe, h] if g else None, rk[ks:ke, h] if g else None,
                                    gs[h] if g else 0.0, scale, causal, eps)
                out[qs:qe, h] = o
                lse[qs:qe, h] = l
        return out, lse
    B = q.shape[0]
    out = np.zeros_like(q)
    lse = np.full(q.shape[:3], -np.inf, dtype=dtype)
    for b in range(B):
        for h in range(H):
            g = h < H_G
            o, l = head_forward(q[b, h], k[b, h // G], v[b, h // G],
                                rq[b, h] if g else None, rk[b, h] if g else None,
                                gs[h] if g else 0.0, scale, causal, eps)
            out[b, h] = o
            lse[b, h] = l
    return out, lse


def backward(dout, q, k, v, rq, rk, gs, out, lse, scale, causal=True, cu_q=None,
             cu_k=None, dtype=np.float64):
    """Backward pass.  Returns (dq, dk, dv, drq, drk, dgs) as numpy ``dtype``."""
    varlen = cu_q is not None
    dout, q, k, v = _as(dout, dtype), _as(q, dtype), _as(k, dtype), _as(v, dtype)
    rq, rk, gs = _as(rq, dtype), _as(rk, dtype), _as(gs, dtype)
    out, lse = _as(out, dtype), _as(lse, dtype)
    H, H_KV = q.shape[1], k.shape[1]
    H_G = 0 if rq is None else rq.shape[1]
    G = H // H_KV
    dq, dk, dv = np.zeros_like(q), np.zeros_like(k), np.zeros_like(v)
    drq = None if rq is None else np.zeros_like(rq)
    drk = None if rk is None else np.zeros_like(rk)
    dgs = np.zeros((H_G,), dtype=dtype)

    if varlen:
        # [T, H, *]: a sequence is a row range; pick rows, then the head.
        segs = _segments(True, 0, _as(cu_q, np.int64), _as(cu_k, np.int64), 0, 0)
        units = [((slice(qs, qe), h), (slice(ks, ke), h // G), (slice(ks, ke), h), h)
                 for (qs, qe, ks, ke) in segs for h in range(H)]
    else:
        # [B, H, S, *]: batch, then head.
        units = [((b, h), (b, h // G), (b, h), h) for b in range(q.shape[0]) for h in range(H)]
    for iq, ikv, irk, h in units:
        g = h < H_G
        dQ, dK, dV, dRq, dRk, dg = head_backward(
            dout[iq], q[iq], k[ikv], v[ikv], rq[iq] if g else None, rk[irk] if g else None,
            gs[h] if g else 0.0, scale, causal, out[iq], lse[iq])
        dq[iq] = dQ
        dk[ikv] += dK
        dv[ikv] += dV
        if g:
            drq[iq] = dRq
            drk[irk] += dRk
            dgs[h] += dg
    return dq, dk, dv, drq, drk, dgs


def decode(q, k_cache, v_cache, rq, rk_cache, gs, scale, seqlens=None, dtype=np.float64,
           eps=EPS):
    """One-token decode against a KV cache: for sequence b and head h, the
    query row q[b, h] attends to the first ``seqlens[b]`` cache rows (all of
    them visible), with the graph bias for h < H_G.  q ``[B, H, D]``, caches
    ``[B, H_KV, L, D]``, rq ``[B, H_G, R]``, rk_cache ``[B, H_G, L, R]``.
    Returns (out ``[B, H, D]``, lse ``[B, H]``).

    This is the non-causal ``head_forward`` on one row, i.e. the last row of
    the causal forward over the sequence (the identity the tests pin), and
    for H_G = 0 the reference's decode step, SDPA over
    ``torch.cat(past_kv, new)`` (FNA2/attention_fna2.py:412-429, :445-473).
    """
    q, kc, vc = _as(q, dtype), _as(k_cache, dtype), _as(v_cache, dtype)
    rq, rkc, gs = _as(rq, dtype), _as(rk_cache, dtype), _as(gs, dtype)
    B, H, D = q.shape
    H_KV, L = kc.shape[1], kc.shape[2]
    H_G = 0 if rq is None else rq.shape[1]
    G = H // H_KV
    lens = np.full(B, L, dtype=np.int64) if seqlens is None else \
        np.clip(_as(seqlens, np.int64), 0, L)
    out = np.zeros((B, H, D), dtype=dtype)
    lse = np.full((B, H), -np.inf, dtype=dtype)
    for b in range(B):
        n = int(lens[b])
        for h in range(H):
            g = h < H_G
            o, l = head_forward(q[b, h][None], kc[b, h // G, :n], vc[b, h // G, :n],
                                rq[b, h][None] if g else None, rkc[b, h, :n] if g else None,
                                gs[h] if g else 0.0, scale, False, eps)
            out[b, h] = o[0]
            lse[b, h] = l[0]
    return out, lse


def flops(cu_or_lengths, H, D, R, causal, H_G=None):
    """Algorithmic FLOPs (fwd, bwd) counted per visible (query, key) pair.

    fwd ``4D + 2R`` and bwd ``10D + 6R`` per pair for graph heads (``4D`` /
    ``10D`` for vanilla heads); visible pairs ``L(L+1)/2`` (causal) or ``L^2``
    per sequence.  ``cu_or_lengths`` is a list of (lq, lk) pairs.
    """
    H_G = H if H_G is None else H_G
    pairs = 0
    for lq, lk in cu_or_lengths:
        if causal:
            n = min(lq, lk)
            pairs += n * (n + 1) // 2 + max(lq - lk, 0) * lk
        else:
            pairs += lq * lk
    fwd = pairs * (H_G * (4 * D + 2 * R) + (H - H_G) * 4 * D)
    bwd = pairs * (H_G * (10 * D + 6 * R) + (H - H_G) * 10 * D)
    return fwd, bwd
