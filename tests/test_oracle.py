"""Pins the CPU oracle (oracle/fna2_oracle.py) without trusting its own formulas.

Checks, each chosen so that a plausible mistake in the oracle fails at least
one of them (the mutation tests at the end plant such mistakes):
  * a pure-Python brute force on tiny inputs (independent loops);
  * torch's scaled_dot_product_attention, a library routine: is_causal=True
    when graph_scale = 0, an explicit float mask built with torch otherwise;
  * torch autograd through that SDPA formulation (fp64, eps = 0);
  * central finite differences of the oracle's own forward;
  * identities: O_0 = V_0 (causal), key-permutation invariance (non-causal),
    <Q, dQ> = <K, dK> and gs * d_gs = <Rq, dRq> = <Rk, dRk> per head,
    sum_j dK_j = 0, sum_j dV_j = sum_i dO_i;
  * varlen == per-sequence dense;
  * c1 (fp32) within 1e-4 max abs of fp64;
  * the reference's eager path restated in oracle/eager_reference.py
    (bias rounded to bf16, SDPA) within the reference's own 0.05 tolerance.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import eager_reference as ER
from oracle import fna2_oracle as O


def rnd(shape, seed, std=1.0):
    return np.random.default_rng(seed).standard_normal(shape) * std


def brute_force(q, k, v, rq, rk, gs, scale, causal, eps=O.EPS):
    """Triple loops over (b, h, i); q [B,H,S,D], k/v [B,HKV,Sk,D], r [B,HG,S,R]."""
    B, H, S, D = q.shape
    HKV, Sk = k.shape[1], k.shape[2]
    HG = 0 if rq is None else rq.shape[1]
    out = np.zeros_like(q)
    lse = np.full((B, H, S), -np.inf)
    for b in range(B):
        for h in range(H):
            kv = h // (H // HKV)
            for i in range(S):
                scores = []
                for j in range(Sk):
                    if causal and j > i:
                        continue
                    s = scale * sum(q[b, h, i, d] * k[b, kv, j, d] for d in range(D))
                    if h < HG:
                        s += gs[h] * sum(rq[b, h, i, r] * rk[b, h, j, r] for r in range(rq.shape[3]))
                    scores.append((j, s))
                if not scores:
                    continue
                m = max(s for _, s in scores)
                l = sum(math.exp(s - m) for _, s in scores)
                for j, s in scores:
                    out[b, h, i] += math.exp(s - m) * v[b, kv, j] / (l + eps)
                lse[b, h, i] = m + math.log(l + eps)
    return out, lse


def make(B=1, H=2, S=7, D=4, HKV=1, HG=1, R=3, Sk=None, seed=0, gs_val=None):
    Sk = S if Sk is None else Sk
    q = rnd((B, H, S, D), seed)
    k = rnd((B, HKV, Sk, D), seed + 1)
    v = rnd((B, HKV, Sk, D), seed + 2)
    rq = rnd((B, HG, S, R), seed + 3, 0.5) if HG else None
    rk = rnd((B, HG, Sk, R), seed + 4, 0.5) if HG else None
    gs = rnd((HG,), seed + 5) if gs_val is None else np.full((HG,), gs_val)
    dout = rnd((B, H, S, D), seed + 6)
    return q, k, v, rq, rk, gs, dout


@pytest.mark.parametrize("causal", [True, False])
@pytest.mark.parametrize("shape", [dict(), dict(H=4, HKV=2, HG=3, R=2, S=6, Sk=9),
                                   dict(B=2, H=2, HKV=2, HG=0, R=0, S=5)])
def test_forward_matches_brute_force(causal, shape):
    q, k, v, rq, rk, gs, _ = make(**shape, seed=3)
    scale = 0.7
    o, l = O.forward(q, k, v, rq, rk, gs, scale, causal)
    bo, bl = brute_force(q, k, v, rq, rk, gs, scale, causal)
    np.testing.assert_allclose(o, bo, atol=1e-12)
    np.testing.assert_allclose(l, bl, atol=1e-12)


def _sdpa_torch(q, k, v, rq, rk, gs, scale, causal, eps_free=True):
    """fp64 torch SDPA with an explicit additive mask (autograd-able)."""
    B, H, S, D = q.shape
    HKV, Sk = k.shape[1], k.shape[2]
    G = H // HKV
    ke, ve = k.repeat_interleave(G, 1), v.repeat_interleave(G, 1)
    bias = torch.zeros(B, H, S, Sk, dtype=torch.float64)
    if rq is not None and rq.shape[1]:
        HG = rq.shape[1]
        bias = torch.cat([gs.view(1, HG, 1, 1) * (rq @ rk.transpose(-1, -2)),
                          torch.zeros(B, H - HG, S, Sk, dtype=torch.float64)], 1)
    if causal:
        keep = torch.ones(S, Sk, dtype=torch.bool).tril()
        bias = bias.masked_fill(~keep, float("-inf"))
    return F.scaled_dot_product_attention(q, ke, ve, attn_mask=bias, scale=scale)


def test_forward_matches_torch_sdpa_gs_zero():
    q, k, v, rq, rk, gs, _ = make(B=2, H=4, S=33, D=8, HKV=2, HG=2, R=4, gs_val=0.0, seed=5)
    o, _ = O.forward(q, k, v, rq, rk, gs, 0.3, True, eps=0.0)
    t = lambda x: torch.tensor(x)
    ref = F.scaled_dot_product_attention(t(q), t(k).repeat_interleave(2, 1),
                                         t(v).repeat_interleave(2, 1), is_causal=True, scale=0.3)
    np.testing.assert_allclose(o, ref.numpy(), atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_forward_matches_torch_sdpa_bias(causal):
    q, k, v, rq, rk, gs, _ = make(B=2, H=4, S=17, D=8, HKV=2, HG=3, R=5, seed=6)
    o, _ = O.forward(q, k, v, rq, rk, gs, 0.35, causal, eps=0.0)
    t = lambda x: torch.tensor(x)
    ref = _sdpa_torch(t(q), t(k), t(v), t(rq), t(rk), t(gs), 0.35, causal)
    np.testing.assert_allclose(o, ref.numpy(), atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_backward_matches_torch_autograd(causal):
    q, k, v, rq, rk, gs, dout = make(B=2, H=4, S=11, D=6, HKV=2, HG=3, R=4, Sk=None, seed=7)
    scale = 0.41
    o, l = O.forward(q, k, v, rq, rk, gs, scale, causal, eps=0.0)
    got = O.backward(dout, q, k, v, rq, rk, gs, o, l, scale, causal)
    leaves = [torch.tensor(x, requires_grad=True) for x in (q, k, v, rq, rk, gs)]
    out = _sdpa_torch(*leaves, scale, causal)
    ref = torch.autograd.grad(out, leaves, torch.tensor(dout))
    for g, r in zip(got, ref):
        np.testing.assert_allclose(g, r.numpy(), atol=1e-10)


def test_backward_matches_finite_differences():
    q, k, v, rq, rk, gs, dout = make(B=1, H=2, S=5, D=3, HKV=1, HG=2, R=2, seed=8)
    scale, causal = 0.6, True
    o, l = O.forward(q, k, v, rq, rk, gs, scale, causal, eps=0.0)
    grads = O.backward(dout, q, k, v, rq, rk, gs, o, l, scale, causal)
    args = [q, k, v, rq, rk, gs]

    def loss(a):
        return float(np.sum(dout * O.forward(*a, scale, causal, eps=0.0)[0]))

    rng = np.random.default_rng(0)
    for idx in range(6):
        u = rng.standard_normal(args[idx].shape)
        h = 1e-6
        ap = [a.copy() for a in args]
        am = [a.copy() for a in args]
        ap[idx] = ap[idx] + h * u
        am[idx] = am[idx] - h * u
        fd = (loss(ap) - loss(am)) / (2 * h)
        an = float(np.sum(grads[idx] * u))
        assert abs(fd - an) < 1e-6 * max(1.0, abs(an)), (idx, fd, an)


def test_identities():
    q, k, v, rq, rk, gs, dout = make(B=1, H=3, S=40, D=8, HKV=3, HG=2, R=4, seed=9)
    scale = 0.3
    o, l = O.forward(q, k, v, rq, rk, gs, scale, True)
    np.testing.assert_allclose(o[:, :, 0], v[:, :, 0] / (1 + O.EPS), atol=1e-12)  # O_0 = V_0
    # exact identities hold without the 1e-6 normaliser (they are off by ~delta * 1e-6 with it)
    o, l = O.forward(q, k, v, rq, rk, gs, scale, True, eps=0.0)
    dq, dk, dv, drq, drk, dgs = O.backward(dout, q, k, v, rq, rk, gs, o, l, scale, True)
    for h in range(3):
        a, b = np.sum(q[0, h] * dq[0, h]), np.sum(k[0, h] * dk[0, h])
        assert abs(a - b) < 1e-9 * max(1, abs(a))
        np.testing.assert_allclose(dk[0, h].sum(0), 0, atol=1e-9)
        np.testing.assert_allclose(dv[0, h].sum(0), dout[0, h].sum(0), atol=1e-9)
    for h in range(2):
        x, y, z = gs[h] * dgs[h], np.sum(rq[0, h] * drq[0, h]), np.sum(rk[0, h] * drk[0, h])
        assert abs(x - y) < 1e-9 * max(1, abs(x)) and abs(x - z) < 1e-9 * max(1, abs(x))


@pytest.mark.parametrize("causal", [True, False])
def test_head_rows_equals_the_full_head_on_its_rows(causal):
    """head_rows (row-local out, lse, dQ, dRq of a row subset) against the
    pinned head_forward / head_backward on the same rows; also across
    head_forward's 1024-row chunk boundary, and for a vanilla head."""
    rng = np.random.default_rng(21)
    L, D, R = 1100, 8, 4
    Q, K, V, dO = (rng.standard_normal((L, D)) for _ in range(4))
    Rq, Rk = rng.standard_normal((L, R)) * 0.5, rng.standard_normal((L, R)) * 0.5
    rows = [0, 1, 5, 1023, 1024, 1050, L - 1]
    for g, rq, rk in ((0.7, Rq, Rk), (0.0, None, None)):
        o, l = O.head_forward(Q, K, V, rq, rk, g, 0.3, causal)
        dq, _, _, drq, _, _ = O.head_backward(dO, Q, K, V, rq, rk, g, 0.3, causal, o, l)
        o2, l2, dq2, drq2 = O.head_rows(dO, Q, K, V, rq, rk, g, 0.3, causal, rows)
        np.testing.assert_allclose(o2, o[rows], atol=1e-12)
        np.testing.assert_allclose(l2, l[rows], atol=1e-12)
        np.testing.assert_allclose(dq2, dq[rows], atol=1e-11)
        if rq is not None:
            np.testing.assert_allclose(drq2, drq[rows], atol=1e-11)


def test_noncausal_key_permutation_invariance():
    q, k, v, rq, rk, gs, _ = make(B=1, H=2, S=9, D=5, HKV=2, HG=2, R=3, seed=10)
    o, _ = O.forward(q, k, v, rq, rk, gs, 0.5, False)
    perm = np.random.default_rng(1).permutation(9)
    o2, _ = O.forward(q, k[:, :, perm], v[:, :, perm], rq, rk[:, :, perm], gs, 0.5, False)
    np.testing.assert_allclose(o, o2, atol=1e-12)


def test_varlen_equals_per_sequence_dense():
    lengths = [3, 0, 7, 1, 5]
    H, D, HKV, HG, R = 4, 6, 2, 3, 4
    T = sum(lengths)
    rng = np.random.default_rng(2)
    q, k, v, dout = (rng.standard_normal((T, n, D)) for n in (H, HKV, HKV, H))
    rq, rk = rng.standard_normal((T, HG, R)), rng.standard_normal((T, HG, R))
    gs = rng.standard_normal(HG)
    cu = np.concatenate([[0], np.cumsum(lengths)])
    for causal in (True, False):
        o, l = O.forward(q, k, v, rq, rk, gs, 0.4, causal, cu, cu)
        g = O.backward(dout, q, k, v, rq, rk, gs, o, l, 0.4, causal, cu, cu)
        dgs = np.zeros(HG)
        for b in range(len(lengths)):
            s0, s1 = cu[b], cu[b + 1]
            t4 = lambda x: x[s0:s1].transpose(1, 0, 2)[None]
            od, ld = O.forward(t4(q), t4(k), t4(v), t4(rq), t4(rk), gs, 0.4, causal)
            gd = O.backward(t4(dout), t4(q), t4(k), t4(v), t4(rq), t4(rk), gs, od, ld, 0.4, causal)
            np.testing.assert_allclose(o[s0:s1], od[0].transpose(1, 0, 2), atol=1e-12)
            for gv, gdd in zip(g[:5], gd[:5]):
                np.testing.assert_allclose(gv[s0:s1], gdd[0].transpose(1, 0, 2), atol=1e-12)
            dgs += gd[5]
        np.testing.assert_allclose(g[5], dgs, atol=1e-12)


def test_c1_fp32_within_1e4_of_fp64():
    """Config c1: dense causal forward, fp32, B2 H4 L256 d64 r8 (CPU oracle only)."""
    from fna2_amd import configs
    cfg = configs.get("c1")
    inp = configs.make_inputs(cfg, with_dout=False)
    o32, _ = O.forward(inp.q, inp.k, inp.v, inp.r_q, inp.r_k, inp.graph_scale, inp.scale, True,
                       dtype=np.float32)
    o64, _ = O.forward(inp.q, inp.k, inp.v, inp.r_q, inp.r_k, inp.graph_scale, inp.scale, True)
    assert np.max(np.abs(o32 - o64)) < 1e-4


def test_eager_reference_restatement_exact_in_fp64():
    """The restated eager path (validate_fna2.py:84-112) run on fp64 inputs rounds only
    its bias, which it builds in fp32 as the reference does (:97, rq.float()): it
    must equal the oracle to fp32 bias rounding.  Pins the restatement's
    bias/GQA/vanilla-pad/mask construction."""
    q, k, v, rq, rk, gs, _ = make(B=2, H=8, S=24, D=8, HKV=4, HG=4, R=6, seed=12)
    t = lambda x: torch.tensor(x)
    for causal in (True, False):
        out = ER.sdpa_reference(t(q), t(k), t(v), t(rq), t(rk), t(gs), 0.3, causal)
        ref, _ = O.forward(q, k, v, rq, rk, gs, 0.3, causal, eps=0.0)
        np.testing.assert_allclose(out.numpy(), ref, atol=1e-6)
    lengths = [5, 9, 1]
    cu = torch.tensor([0, 5, 14, 15])
    T = 15
    qv, kv, vv = t(rnd((T, 4, 8), 1)), t(rnd((T, 2, 8), 2)), t(rnd((T, 2, 8), 3))
    rqv, rkv, gv = t(rnd((T, 3, 4), 4)), t(rnd((T, 3, 4), 5)), t(rnd((3,), 6))
    outv = ER.sdpa_reference_varlen(qv, kv, vv, rqv, rkv, gv, cu, cu, 0.3, True)
    refv, _ = O.forward(qv, kv, vv, rqv, rkv, gv, 0.3, True, cu.numpy(), cu.numpy(), eps=0.0)
    np.testing.assert_allclose(outv.numpy(), refv, atol=1e-6)


def test_eager_reference_bf16_within_reference_tolerance():
    """In bf16 the eager path rounds the bias to bf16 (validate_fna2.py:102); at the
    configs' R scale (std 1/sqrt(R)) it stays within the reference's 0.05 (:59)."""
    g = torch.Generator().manual_seed(42)
    mk = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16()
    q, k, v = mk(2, 8, 128, 64), mk(2, 4, 128, 64), mk(2, 4, 128, 64)
    rq, rk = mk(2, 4, 128, 32, std=32 ** -0.5), mk(2, 4, 128, 32, std=32 ** -0.5)
    gs = torch.randn(4, generator=g)
    out = ER.sdpa_reference(q, k, v, rq, rk, gs, 0.125, causal=True)
    ref, _ = O.forward(q, k, v, rq, rk, gs, 0.125, True)
    assert np.max(np.abs(out.double().numpy() - ref)) < 0.05


def _visible_pairs_brute(lengths, causal):
    """Visible (query, key) pairs counted one by one from the oracle's own
    mask (the one its forward and backward apply)."""
    total = 0
    for lq, lk in lengths:
        if lq and lk:
            total += int(O._mask(0, lq, lk, causal).sum())
    return total


def _matmul_flops_per_pair(D, R, graph):
    """FLOPs per visible pair from the products the oracle forms, 2 x inner
    dimension each: forward S = Q K^T (D), bias Rq Rk^T (R), O = P V (D);
    backward recomputed S and bias, dP = dO V^T (D), dV = P^T dO (D),
    dK = dS^T Q (D), dQ = dS K (D), dRq = dS Rk (R), dRk = dS^T Rq (R)."""
    r = R if graph else 0
    fwd = 2 * D + 2 * r + 2 * D
    bwd = (2 * D + 2 * r) + 2 * D + 2 * D + 2 * D + 2 * D + 2 * r + 2 * r
    return fwd, bwd


def test_flops_counts_visible_pairs_by_brute_force():
    """oracle.flops against a pair-by-pair count of the mask on random
    length sets (queries and keys of different lengths, empty sequences,
    causal and not) and the per-pair FLOPs of the oracle's products; with
    graph and vanilla heads mixed."""
    rng = np.random.default_rng(17)
    for causal in (True, False):
        for _ in range(25):
            n = int(rng.integers(1, 6))
            lengths = [(int(rng.integers(0, 70)), int(rng.integers(0, 70))) for _ in range(n)]
            pairs = _visible_pairs_brute(lengths, causal)
            H, H_G, D, R = 5, 3, 16, 8
            fg, bg = _matmul_flops_per_pair(D, R, True)
            fv, bv = _matmul_flops_per_pair(D, R, False)
            fwd, bwd = O.flops(lengths, H, D, R, causal, H_G=H_G)
            assert fwd == pairs * (H_G * fg + (H - H_G) * fv), (lengths, causal)
            assert bwd == pairs * (H_G * bg + (H - H_G) * bv), (lengths, causal)


def test_config_flops_match_brute_force_counts():
    """The bench's FLOP counts (fna2_amd.configs.Config.flops) equal the
    brute-force pair count for c2, c3 and c5 (c3 / c5 from their committed
    packings) and the oracle's count for c4."""
    from fna2_amd import configs
    for name in ("c2", "c3", "c5", "c4"):
        cfg = configs.get(name)
        lens = [(n, n) for n in cfg.seq_lengths()]
        if name == "c4":
            pairs = O.flops(lens, 1, 1, 0, cfg.causal, H_G=0)[0] // 4  # 4D per pair at D = 1
            assert pairs == 16384 * 16385 // 2
        elif name == "c5":
            # the 8192-token sequence is non-causal: all 8192^2 pairs
            pairs = 8192 * 8192 + _visible_pairs_brute(lens[1:], cfg.causal)
        else:
            pairs = _visible_pairs_brute(lens, cfg.causal)
        f, b = _matmul_flops_per_pair(cfg.D, cfg.R, True)
        assert cfg.flops() == (pairs * cfg.H * f, pairs * cfg.H * b), name


# ── planted mistakes: each must make at least one pinning check fail ──────────

def _run_pins():
    """The pinning checks above, on fresh inputs; raises if any fails."""
    test_forward_matches_brute_force(True, dict(H=4, HKV=2, HG=3, R=2, S=6, Sk=9))
    test_forward_matches_torch_sdpa_bias(True)
    test_forward_matches_torch_sdpa_bias(False)
    test_backward_matches_torch_autograd(True)
    test_identities()


@pytest.mark.parametrize("mutation", ["drop_bias", "causal_off_by_one", "transposed_bias",
                                      "drop_gs_in_drk", "wrong_kv_head"])
def test_planted_mistakes_are_caught(monkeypatch, mutation):
    if mutation == "drop_bias":
        monkeypatch.setattr(O, "_scores", lambda Qb, K, Rqb, Rk, g, scale: scale * (Qb @ K.T))
    elif mutation == "causal_off_by_one":
        def bad_mask(i0, nq, lk, causal):
            qi = np.arange(i0, i0 + nq)[:, None]
            kj = np.arange(lk)[None, :]
            return (kj < qi) | (kj == 0) if causal else np.ones((nq, lk), bool)
        monkeypatch.setattr(O, "_mask", bad_mask)
    elif mutation == "transposed_bias":
        def bad_scores(Qb, K, Rqb, Rk, g, scale):
            S = scale * (Qb @ K.T)
            if Rqb is not None:
                n = min(S.shape)
                B = g * (Rqb @ Rk.T)
                B[:n, :n] = B[:n, :n].T
                S = S + B
            return S
        monkeypatch.setattr(O, "_scores", bad_scores)
    elif mutation == "drop_gs_in_drk":
        orig = O.head_backward

        def bad_backward(dO, Q, K, V, Rq, Rk, g, scale, causal, Ov, lse):
            res = list(orig(dO, Q, K, V, Rq, Rk, g, scale, causal, Ov, lse))
            if Rk is not None and g != 0:
                res[4] = res[4] / g
            return tuple(res)
        monkeypatch.setattr(O, "head_backward", bad_backward)
    elif mutation == "wrong_kv_head":
        orig_fwd = O.head_forward
        calls = {"n": 0}

        def bad_fwd(Q, K, V, *a, **kw):
            calls["n"] += 1
            return orig_fwd(Q, K * (1.0 + 0.01 * (calls["n"] % 2)), V, *a, **kw)
        monkeypatch.setattr(O, "head_forward", bad_fwd)
    with pytest.raises(AssertionError):
        _run_pins()


# ── decode (one query row against a KV cache) ─────────────────────────────────

def _decode_case(seed, B=3, H=6, HKV=2, HG=4, D=8, R=4, L=11):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, L, D))
    k = rng.standard_normal((B, HKV, L, D))
    v = rng.standard_normal((B, HKV, L, D))
    rq = rng.standard_normal((B, HG, L, R))
    rk = rng.standard_normal((B, HG, L, R))
    gs = rng.standard_normal(HG)
    lens = np.array([L, 1, 7][:B])
    return q, k, v, rq, rk, gs, lens


def test_decode_is_last_row_of_causal_forward():
    """Row len-1 of the causal forward over the sequence (the causal mask
    path) equals the decode of that row against the first len cache rows (the
    truncation path)."""
    q, k, v, rq, rk, gs, lens = _decode_case(11)
    B, H = q.shape[:2]
    scale = 0.37
    qd = np.stack([q[b, :, lens[b] - 1] for b in range(B)])
    rqd = np.stack([rq[b, :, lens[b] - 1] for b in range(B)])
    out, lse = O.decode(qd, k, v, rqd, rk, gs, scale, seqlens=lens)
    for b in range(B):
        n = lens[b]
        of, lf = O.forward(q[b:b + 1, :, :n], k[b:b + 1, :, :n], v[b:b + 1, :, :n],
                           rq[b:b + 1, :, :n], rk[b:b + 1, :, :n], gs, scale, causal=True)
        np.testing.assert_allclose(out[b], of[0, :, n - 1], rtol=1e-12, atol=1e-12)
        np.testing.assert_allclose(lse[b], lf[0, :, n - 1], rtol=1e-12, atol=1e-12)


def test_decode_without_bias_is_torch_sdpa_over_the_cache():
    """H_G = 0: the reference's decode step, SDPA (no mask) over the cached
    rows with the KV heads repeated per group."""
    q, k, v, _, _, _, lens = _decode_case(12)
    B, H = q.shape[:2]
    G = H // k.shape[1]
    qd = q[:, :, 0]
    out, _ = O.decode(qd, k, v, None, None, None, 0.5, seqlens=lens)
    for b in range(B):
        n = lens[b]
        kt = torch.from_numpy(k[b:b + 1, :, :n]).repeat_interleave(G, dim=1)
        vt = torch.from_numpy(v[b:b + 1, :, :n]).repeat_interleave(G, dim=1)
        ref = F.scaled_dot_product_attention(torch.from_numpy(qd[b:b + 1, :, None]), kt, vt,
                                             scale=0.5)
        np.testing.assert_allclose(out[b], ref[0, :, 0].numpy(), rtol=0, atol=1e-5)


def test_decode_empty_cache_rows():
    q, k, v, rq, rk, gs, _ = _decode_case(13)
    out, lse = O.decode(q[:, :, 0], k, v, rq[:, :, 0], rk, gs, 0.5, seqlens=np.array([0, 0, 0]))
    assert np.all(out == 0) and np.all(np.isneginf(lse))


@pytest.mark.parametrize("mutation", ["len_off_by_one", "bias_on_kv_head_rk"])
def test_decode_planted_mistakes_are_caught(monkeypatch, mutation):
    orig = O.head_forward
    if mutation == "len_off_by_one":
        def bad(Q, K, V, Rq, Rk, g, scale, causal, eps=O.EPS):
            if K.shape[0] > 1 and not causal:
                K, V = K[:-1], V[:-1]
                Rk = None if Rk is None else Rk[:-1]
            return orig(Q, K, V, Rq, Rk, g, scale, causal, eps)
    else:
        def bad(Q, K, V, Rq, Rk, g, scale, causal, eps=O.EPS):
            if Rk is not None and not causal:
                Rk = Rk[::-1]
            return orig(Q, K, V, Rq, Rk, g, scale, causal, eps)
    monkeypatch.setattr(O, "head_forward", bad)
    with pytest.raises(AssertionError):
        test_decode_is_last_row_of_causal_forward()
        test_decode_without_bias_is_torch_sdpa_over_the_cache()
