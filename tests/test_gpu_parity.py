"""GPU parity: the HIP kernels (through the C ABI) against the fp64 CPU oracle.

Small and medium shapes covering the reference's configurations (dense and
varlen, causal and not, GQA, vanilla heads, every supported rank and head
dim), run on the same seeded bf16 inputs.  Tolerances: out 2e-2 max abs,
gradients 5e-2 relative norm, LSE 1e-2 max abs.
"""
import importlib
import math

import numpy as np
import pytest
import torch

from tests import helpers as H

pytestmark = pytest.mark.gpu


def _fna2():
    return importlib.import_module("fna2_amd.flash_naylis_attn")


def _dense_case(gpu, B, Hq, S, D, H_KV, H_G, R, causal, seed, Sk=None, layout="bhsd", gs=None):
    F = _fna2()
    q, k, v, rq, rk, gs_, dout = H.make_dense(B, Hq, S, D, H_KV, H_G, R, seed=seed, Sk=Sk,
                                              layout=layout, gs=gs)
    scale = 1.0 / math.sqrt(D)
    print(f"dense B{B} H{Hq} S{S} Sk{Sk} D{D} HKV{H_KV} HG{H_G} R{R} causal={causal}", flush=True)
    dq_ = [t.to(gpu) if t is not None else None for t in (q, k, v, rq, rk, gs_, dout)]
    out, lse = F._fna2_forward(dq_[0], dq_[1], dq_[2], dq_[3], dq_[4], dq_[5], scale, causal)
    grads = F._fna2_backward(dq_[6], dq_[0], dq_[1], dq_[2], dq_[3], dq_[4], dq_[5], out, lse,
                             scale, causal)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, scale, causal)
    H.check_out(out, lse, ref_out, ref_lse)
    return H.check_grads(grads, ref_g)


@pytest.mark.parametrize("D,R", [(64, 16), (128, 32), (64, 8), (128, 64), (64, 64), (128, 16),
                                 (128, 24), (64, 48)])
def test_dense_causal_ranks(gpu, D, R):
    _dense_case(gpu, 2, 4, 200, D, 4, 4, R, True, seed=D + R)


@pytest.mark.parametrize("causal", [True, False])
def test_dense_gqa_vanilla(gpu, causal):
    # reference validation config "60m": B2 H8 S128 D64 H_KV4 H_G4 R32
    _dense_case(gpu, 2, 8, 128, 64, 4, 4, 32, causal, seed=42)


def test_dense_220m_config(gpu):
    # reference validation config "220m": B2 H12 S256 D64 H_KV4 H_G8 R32
    _dense_case(gpu, 2, 12, 256, 64, 4, 8, 32, True, seed=42)


def test_dense_no_graph_heads(gpu):
    _dense_case(gpu, 1, 4, 300, 128, 2, 0, 0, True, seed=3)


@pytest.mark.parametrize("S,Sk", [(1, 1), (65, 65), (129, 97), (96, 200), (333, 333)])
def test_dense_odd_lengths(gpu, S, Sk):
    _dense_case(gpu, 1, 2, S, 64, 2, 2, 16, True, seed=S, Sk=Sk)
    _dense_case(gpu, 1, 2, S, 128, 1, 1, 32, False, seed=S + 1, Sk=Sk)


def test_dense_strided_layout(gpu):
    # [B, S, H, D] memory passed as [B, H, S, D] views, as the configs state
    _dense_case(gpu, 2, 4, 256, 128, 4, 4, 32, True, seed=5, layout="bshd")


def test_scale_edge_cases(gpu):
    F = _fna2()
    q, k, v, rq, rk, gs, dout = H.make_dense(1, 2, 96, 64, 2, 2, 16, seed=9)
    for scale in (0.0, -0.125, 0.5):
        qg, kg, vg, rqg, rkg, gsg, dog = (t.to(gpu) for t in (q, k, v, rq, rk, gs, dout))
        out, lse = F._fna2_forward(qg, kg, vg, rqg, rkg, gsg, scale, True)
        grads = F._fna2_backward(dog, qg, kg, vg, rqg, rkg, gsg, out, lse, scale, True)
        torch.cuda.synchronize()
        ro, rl, rg = H.oracle_fwd_bwd(q, k, v, rq, rk, gs, dout, scale, True)
        H.check_out(out, lse, ro, rl)
        H.check_grads(grads, rg)


def _varlen_case(gpu, lengths, Hq, D, H_KV, H_G, R, causal, seed, lengths_k=None, gs=None,
                 r_std=None):
    F = _fna2()
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(
        lengths, Hq, D, H_KV, H_G, R, seed=seed, lengths_k=lengths_k, gs=gs, r_std=r_std)
    scale = 1.0 / math.sqrt(D)
    print(f"varlen n={len(lengths)} T={sum(lengths)} H{Hq} D{D} HKV{H_KV} HG{H_G} R{R} "
          f"causal={causal}", flush=True)
    g = [t.to(gpu) if t is not None else None for t in (q, k, v, rq, rk, gs_, dout, cu_q, cu_k)]
    mq = max(lengths) if lengths else 0
    mk = max(lengths_k or lengths) if (lengths_k or lengths) else 0
    out, lse = F._fna2_forward_varlen(g[0], g[1], g[2], g[3], g[4], g[5], g[7], g[8], mq, mk,
                                      scale, causal)
    grads = F._fna2_backward_varlen(g[6], g[0], g[1], g[2], g[3], g[4], g[5], out, lse, g[7],
                                    g[8], mq, mk, scale, causal)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, scale, causal,
                                               cu_q.numpy(), cu_k.numpy())
    H.check_out(out, lse, ref_out, ref_lse)
    return H.check_grads(grads, ref_g)


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_mixed(gpu, causal):
    lengths = [1, 17, 64, 127, 128, 129, 300, 5, 257]
    _varlen_case(gpu, lengths, 4, 128, 2, 3, 32, causal, seed=11)
    _varlen_case(gpu, lengths, 4, 64, 4, 4, 16, causal, seed=12)


@pytest.mark.parametrize("causal", [True, False])
def test_varlen_gqa_d64(gpu, causal):
    """d 64, rank 16 (two key slices per dK/dV wave, ring DMA by the
    consumer waves): GQA groups of 3 with graph and vanilla heads in one
    group, items of one block and of many, sequences of one token."""
    _varlen_case(gpu, [3, 70, 256, 257, 31, 520, 1, 96], 6, 64, 2, 4, 16, causal, seed=31)


@pytest.mark.parametrize("seed", [112, 122, 126, 135])
def test_varlen_random_shapes_d64(gpu, seed):
    """Seeded random packs at d 64, rank <= 32: lengths from 0 to 600 with
    tile multiples (32, 128, 256) and their neighbours over-represented,
    GQA groups of 1 to 4 with any number of graph heads, causal or not."""
    rng = np.random.default_rng(seed)
    edges = [0, 1, 31, 32, 33, 127, 128, 129, 255, 256, 257]
    n = int(rng.integers(3, 10))
    lengths = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(0, 601))
               for _ in range(n)]
    if sum(lengths) == 0:
        lengths[0] = 40
    H_KV = int(rng.integers(1, 3))
    Hq = H_KV * int(rng.integers(1, 5))
    H_G = int(rng.integers(0, Hq + 1))
    R = int(rng.choice([8, 16, 32])) if H_G else 0
    causal = bool(rng.integers(0, 2))
    _varlen_case(gpu, lengths, Hq, 64, H_KV, H_G, R, causal, seed=seed)


@pytest.mark.parametrize("seed", [217, 201, 207, 223, 200, 237, 214, 242, 227, 206])
def test_varlen_random_shapes_d128(gpu, seed):
    """Seeded random packs at d 128 (the forward and dQ read their LDS
    operands k-steps ahead of the MFMAs there, in chains whose length
    depends on the rank tier): every rank from 8 to 64, lengths with the
    32 / 128-key tile edges over-represented, GQA groups of 1 to 3 with any
    number of graph heads, causal or not (the seeds cover ranks 8 to 64,
    each rank tier causal and not)."""
    rng = np.random.default_rng(seed)
    edges = [1, 31, 32, 33, 63, 64, 65, 127, 128, 129, 160, 257]
    n = int(rng.integers(2, 7))
    lengths = [int(rng.choice(edges)) if rng.random() < 0.5 else int(rng.integers(1, 450))
               for _ in range(n)]
    H_KV = int(rng.integers(1, 3))
    Hq = H_KV * int(rng.integers(1, 4))
    H_G = int(rng.integers(0, Hq + 1))
    R = 8 * int(rng.integers(1, 9)) if H_G else 0
    causal = bool(rng.integers(0, 2))
    _varlen_case(gpu, lengths, Hq, 128, H_KV, H_G, R, causal, seed=seed)


def test_varlen_d64_rank_rows_past_20k(gpu):
    """d 64, 8 graph heads of rank 32: a tile's rank rows past 20 KB.  Caught a
    missing wait state between a scalar descriptor write and the inline-asm
    buffer load that reads it."""
    _varlen_case(gpu, [37, 128, 5, 90], 8, 64, 8, 8, 32, True, seed=22)
    _varlen_case(gpu, [300], 8, 64, 8, 8, 32, False, seed=23)


@pytest.mark.parametrize("D,R", [(64, 48), (64, 16), (128, 64)])
def test_vanilla_heads_with_rank_tiles(gpu, D, R):
    """Vanilla heads next to graph heads in every kernel variant whose rank
    MFMAs run for all heads: the vanilla heads' rank tiles come from
    zero-size ranges, so their scores must equal plain attention's."""
    _dense_case(gpu, 2, 4, 160, D, 2, 2, R, True, seed=D + R + 1)
    _varlen_case(gpu, [300, 17, 129, 64], 4, D, 2, 1, R, False, seed=D + R + 2)
    _varlen_case(gpu, [95, 1, 256], 6, D, 3, 4, R, True, seed=D + R + 3)


def test_varlen_cross_lengths(gpu):
    lq = [50, 130, 7, 200]
    lk = [70, 100, 7, 260]
    _varlen_case(gpu, lq, 2, 64, 2, 2, 16, True, seed=13, lengths_k=lk)
    _varlen_case(gpu, lq, 2, 128, 1, 2, 32, False, seed=14, lengths_k=lk)


def test_varlen_empty_sequences(gpu):
    _varlen_case(gpu, [0, 40, 0, 0, 90, 0], 2, 64, 2, 2, 16, True, seed=15)


@pytest.mark.parametrize("use_plan", [False, True])
def test_varlen_uncovered_rows(gpu, use_plan):
    """Tokens outside [cu[0], cu[N]) belong to no sequence: zero gradients there
    (the launch that builds the tile lists zeroes them; with a plan, the dQ
    kernel's spare workgroups do), oracle parity inside."""
    F = _fna2()
    lengths = [3, 40, 90, 5]
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 64, 2, 3, 16, seed=21)
    sub = cu_q[1:-1].clone()  # sequences 1 and 2 only: rows 0-2 and 133-137 uncovered
    lo, hi = int(sub[0]), int(sub[-1])
    scale = 0.125
    print(f"varlen uncovered rows: cu {sub.tolist()} of {q.shape[0]} tokens", flush=True)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout, sub)]
    plan = F._plan_for(g[0], g[1], g[3], g[7], g[7], 90, 90, True, scale) if use_plan else None
    assert (plan is not None) == use_plan
    out, lse = F._fna2_forward_varlen(g[0], g[1], g[2], g[3], g[4], g[5], g[7], g[7], 90, 90,
                                      scale, True, plan=plan)
    # gradients allocated over garbage, so that only the zeroing makes them 0
    torch.cuda.empty_cache()
    junk = torch.full((1 << 20,), float("nan"), device=gpu)
    del junk
    grads = F._fna2_backward_varlen(g[6], g[0], g[1], g[2], g[3], g[4], g[5], out, lse, g[7],
                                    g[7], 90, 90, scale, True, plan=plan)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, scale, True,
                                               sub.numpy(), sub.numpy())
    H.check_out(out[lo:hi], lse[lo:hi], np.asarray(ref_out)[lo:hi], np.asarray(ref_lse)[lo:hi])
    for name, t in zip(("dq", "dk", "dv", "drq", "drk"), grads[:5]):
        outside = torch.cat([t[:lo], t[hi:]]).float()
        assert torch.count_nonzero(outside) == 0, f"{name}: nonzero gradient outside cu"
    H.check_grads(grads, ref_g)


def test_varlen_bias_dominated(gpu):
    # c5-like: rank 16 bias with R std 0.5 and non-causal attention
    _varlen_case(gpu, [300, 16, 128, 40, 77], 4, 64, 4, 4, 16, False, seed=16, gs=1.0,
                 r_std=0.5)


def test_varlen_matches_per_segment_dense(gpu):
    """Reference T3/T3b: packed == per-segment dense (flash_naylis_attn path only)."""
    F = _fna2()
    lengths = [64, 64]
    (q, k, v, rq, rk, gs, dout, cu_q, cu_k) = H.make_varlen(lengths, 8, 64, 4, 4, 32, seed=99,
                                                            device=gpu)
    scale = 0.125
    qs = [t.clone().requires_grad_(True) for t in (q, k, v, rq, rk, gs)]
    out_p = F.flash_naylis_attn(*qs, softmax_scale=scale, is_causal=True, cu_seqlens_q=cu_q,
                                cu_seqlens_k=cu_k, max_seqlen_q=64, max_seqlen_k=64)
    out_p.float().sum().backward()
    outs, grads = [], [[] for _ in range(5)]
    dgs = torch.zeros_like(gs)
    for s0, s1 in ((0, 64), (64, 128)):
        seg = [t[s0:s1].detach().clone().requires_grad_(True) for t in (q, k, v, rq, rk)]
        g_s = gs.detach().clone().requires_grad_(True)
        r4 = [t.transpose(0, 1).unsqueeze(0) for t in seg]
        o = F.flash_naylis_attn(*r4, g_s, softmax_scale=scale, is_causal=True)
        o.float().sum().backward()
        outs.append(o.squeeze(0).transpose(0, 1))
        for i in range(5):
            grads[i].append(seg[i].grad)
        dgs += g_s.grad
    ref = torch.cat(outs, 0)
    assert H.max_abs(out_p, ref) < 1e-2
    for i in range(5):
        assert H.rel_norm(qs[i].grad, torch.cat(grads[i], 0)) < 1e-2
    assert H.rel_norm(qs[5].grad, dgs) < 1e-2


def test_gs_zero_equals_sdpa(gpu):
    """Reference T4: graph_scale = 0 gives plain causal attention (torch SDPA)."""
    F = _fna2()
    q, k, v, rq, rk, gs, _ = H.make_dense(2, 8, 128, 64, 4, 4, 32, seed=7, gs=0.0, device=gpu)
    out = F.flash_naylis_attn(q, k, v, rq, rk, gs, softmax_scale=0.125, is_causal=True)
    ke = k.float().repeat_interleave(2, dim=1)
    ve = v.float().repeat_interleave(2, dim=1)
    ref = torch.nn.functional.scaled_dot_product_attention(q.float(), ke, ve, is_causal=True,
                                                           scale=0.125)
    assert H.max_abs(out, ref) < 2e-2


def test_deterministic(gpu):
    F = _fna2()
    q, k, v, rq, rk, gs, dout = H.make_dense(2, 4, 384, 128, 2, 4, 32, seed=21, device=gpu)
    res = []
    for _ in range(2):
        out, lse = F._fna2_forward(q, k, v, rq, rk, gs, 0.088, True)
        g = F._fna2_backward(dout, q, k, v, rq, rk, gs, out, lse, 0.088, True)
        res.append([out, lse, *g])
    torch.cuda.synchronize()
    for a, b in zip(*res):
        assert torch.equal(a, b)


@pytest.mark.parametrize("use_plan", [False, True])
def test_deterministic_varlen_equal_lengths(gpu, use_plan):
    """Many sequences of one length (c5's pattern: the list builder places
    equal-work tiles in a different order on every run) and graph heads:
    every output, d_graph_scale included, bit for bit the same over runs.
    d_graph_scale sums per-tile partials, which are indexed by the tile's
    (sequence, tile) slot rather than its list position."""
    F = _fna2()
    lengths = [48] * 200 + [700] + [16] * 60
    (q, k, v, rq, rk, gs_, dout, cu_q, _) = H.make_varlen(lengths, 4, 64, 4, 4, 16, seed=41)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout, cu_q)]
    mx, scale = max(lengths), 0.125
    print(f"varlen determinism: {len(lengths)} sequences, plan {use_plan}", flush=True)
    res = []
    for _ in range(3):
        plan = F._plan_for(g[0], g[1], g[3], g[7], g[7], mx, mx, False, scale) if use_plan else None
        out, lse = F._fna2_forward_varlen(*g[:6], g[7], g[7], mx, mx, scale, False, plan=plan)
        grads = F._fna2_backward_varlen(g[6], *g[:6], out, lse, g[7], g[7], mx, mx, scale, False,
                                        plan=plan)
        res.append([out.clone(), lse.clone(), *[t.clone() for t in grads]])
    torch.cuda.synchronize()
    for r in res[1:]:
        for a, b in zip(r, res[0]):
            assert torch.equal(a, b)


def test_row0_equals_v0(gpu):
    """Causal row 0 attends only to key 0: O_0 = V_0 (to bf16 rounding)."""
    F = _fna2()
    q, k, v, rq, rk, gs, _ = H.make_dense(1, 2, 64, 64, 2, 2, 16, seed=4, device=gpu)
    out, _ = F._fna2_forward(q, k, v, rq, rk, gs, 0.125, True)
    assert H.max_abs(out[:, :, 0], v[:, :, 0]) < 1e-2


def test_varlen_no_query_rows_with_plan(gpu):
    """Keys but no query rows: the forward still fills the plan, and the
    backward (no dQ launch) builds its lists itself and writes zero dK, dV,
    dRk."""
    F = _fna2()
    H_, D, R = 4, 64, 16
    g = torch.Generator().manual_seed(31)
    q = torch.randn(0, H_, D, generator=g).bfloat16().to(gpu).requires_grad_(True)
    k = torch.randn(10, H_, D, generator=g).bfloat16().to(gpu).requires_grad_(True)
    v = torch.randn(10, H_, D, generator=g).bfloat16().to(gpu).requires_grad_(True)
    rq = torch.randn(0, H_, R, generator=g).bfloat16().to(gpu).requires_grad_(True)
    rk = torch.randn(10, H_, R, generator=g).bfloat16().to(gpu).requires_grad_(True)
    gs_ = torch.ones(H_, device=gpu, requires_grad=True)
    cu_q = torch.tensor([0, 0, 0], dtype=torch.int32, device=gpu)
    cu_k = torch.tensor([0, 5, 10], dtype=torch.int32, device=gpu)
    print("varlen no query rows, with plan", flush=True)
    out = F.flash_naylis_attn(q, k, v, rq, rk, gs_, softmax_scale=0.125, is_causal=False,
                              cu_seqlens_q=cu_q, cu_seqlens_k=cu_k, max_seqlen_q=0,
                              max_seqlen_k=5)
    assert out.shape == (0, H_, D)
    grads = torch.autograd.grad(out, [k, v, rk], torch.zeros_like(out), allow_unused=True)
    torch.cuda.synchronize()
    for name, t in zip(("dk", "dv", "drk"), grads):
        assert t is not None, f"{name}: the backward did not run"
        assert torch.count_nonzero(t.float()) == 0, name


def test_varlen_no_sequences_zeroes_every_gradient_row(gpu):
    """cu_seqlens = [0] with tokens present: every token lies outside every
    sequence, so every gradient row is zero (the reference zero-fills its
    gradients, FNA2/flash_naylis_attn.py:1247-1252), not left as allocated."""
    F = _fna2()
    H_, D, R, T = 4, 64, 16, 37
    g = torch.Generator().manual_seed(32)
    mk = lambda *s: torch.randn(*s, generator=g).bfloat16().to(gpu)
    q, k, v, dout = mk(T, H_, D), mk(T, H_, D), mk(T, H_, D), mk(T, H_, D)
    rq, rk = mk(T, H_, R), mk(T, H_, R)
    gs_ = torch.ones(H_, device=gpu)
    cu = torch.zeros(1, dtype=torch.int32, device=gpu)
    out, lse = F._fna2_forward_varlen(q, k, v, rq, rk, gs_, cu, cu, 0, 0, 0.125, True)
    torch.cuda.empty_cache()
    junk = torch.full((1 << 20,), float("nan"), device=gpu)  # gradients land on garbage
    del junk
    print("varlen backward, no sequences, 37 tokens", flush=True)
    grads = F._fna2_backward_varlen(dout, q, k, v, rq, rk, gs_, out, lse, cu, cu, 0, 0, 0.125,
                                    True)
    torch.cuda.synchronize()
    for name, t in zip(("dq", "dk", "dv", "drq", "drk", "dgs"), grads):
        assert t is not None, name
        assert torch.count_nonzero(t.float()) == 0, name


def test_backward_ignores_a_plan_no_forward_filled(gpu):
    """A plan buffer that no forward of this problem filled (here: garbage)
    is ignored: the backward builds its own tile lists and matches the
    oracle, instead of reading the garbage as tile records."""
    F = _fna2()
    lengths = [70, 3, 200, 129]
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=33)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout, cu_q, cu_k)]
    scale = 0.09
    out, lse = F._fna2_forward_varlen(g[0], g[1], g[2], g[3], g[4], g[5], g[7], g[8], 200, 200,
                                      scale, True)
    plan = F._plan_for(g[0], g[1], g[3], g[7], g[8], 200, 200, True, scale)
    plan.fill_(0xAB)  # never filled by a forward
    print("varlen backward with an unfilled plan", flush=True)
    grads = F._fna2_backward_varlen(g[6], g[0], g[1], g[2], g[3], g[4], g[5], out, lse, g[7],
                                    g[8], 200, 200, scale, True, plan=plan)
    torch.cuda.synchronize()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, scale, True,
                                               cu_q.numpy(), cu_k.numpy())
    H.check_out(out, lse, ref_out, ref_lse)
    H.check_grads(grads, ref_g)


def test_plan_of_another_key_tile_size_is_ignored(gpu):
    """A plan filled by a d = 128 forward (128-key dK/dV tiles) handed to a
    d = 64, rank-16 backward of the same sequences (256-key tiles): the key
    list's records differ, so the backward must not use it.  Its gradients
    equal those of the same backward without a plan, bit for bit."""
    F = _fna2()
    lengths = [300, 65, 513, 1]
    cu = torch.tensor([0] + list(np.cumsum(lengths)), dtype=torch.int32, device=gpu)
    big = H.make_varlen(lengths, 2, 128, 2, 2, 32, seed=5)
    gb = [t.to(gpu) for t in big]
    plan = F._plan_for(gb[0], gb[1], gb[3], cu, cu, 513, 513, True, 0.1)
    F._fna2_forward_varlen(*gb[:6], cu, cu, 513, 513, 0.1, True, plan=plan)
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 64, 2, 4, 16, seed=6)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout)]
    small = F._plan_for(g[0], g[1], g[3], cu, cu, 513, 513, True, 0.125)
    assert plan.numel() >= small.numel()
    out, lse = F._fna2_forward_varlen(*g[:6], cu, cu, 513, 513, 0.125, True)
    print("d64 r16 backward with a d128 plan", flush=True)
    with_plan = F._fna2_backward_varlen(g[6], *g[:6], out, lse, cu, cu, 513, 513, 0.125, True,
                                        plan=plan)
    no_plan = F._fna2_backward_varlen(g[6], *g[:6], out, lse, cu, cu, 513, 513, 0.125, True)
    torch.cuda.synchronize()
    for name, a, b in zip(("dq", "dk", "dv", "drq", "drk", "dgs"), with_plan, no_plan):
        assert torch.equal(a, b), name
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, 0.125, True,
                                               cu_q.numpy(), cu_k.numpy())
    H.check_grads(with_plan, ref_g)


def test_plan_reused_across_calls_with_the_same_cu_seqlens(gpu):
    """The autograd path reuses a plan for cu_seqlens tensors it saw
    unchanged (the layers of one step): the second call launches no builder
    and its results equal a fresh call's; an in-place write to cu_seqlens
    (new lengths) bumps its version, and the plan is rebuilt."""
    F = _fna2()
    F._PLANS.clear()
    lengths = [200, 1, 77, 300]
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=40)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout)]
    cu = cu_q.to(gpu)

    def run(c, mx):
        leaves = [t.detach().requires_grad_(True) for t in g[:6]]
        out = F.flash_naylis_attn(*leaves, softmax_scale=0.1, is_causal=True, cu_seqlens_q=c,
                                  cu_seqlens_k=c, max_seqlen_q=mx, max_seqlen_k=mx)
        return [out.detach()] + [x.detach() for x in torch.autograd.grad(out, leaves, g[6])]

    print("plan reuse: first call builds, second reuses", flush=True)
    first = run(cu, 300)
    assert len(F._PLANS) == 1
    second = run(cu, 300)
    torch.cuda.synchronize()
    for a, b in zip(first, second):
        assert torch.equal(a, b)
    out, lse = F._fna2_forward_varlen(*g[:6], cu, cu, 300, 300, 0.1, True)
    ref = F._fna2_backward_varlen(g[6], *g[:6], out, lse, cu, cu, 300, 300, 0.1, True)
    torch.cuda.synchronize()
    assert torch.equal(second[0], out)
    for a, b in zip(second[1:], ref):
        assert torch.equal(a, b)
    # new lengths written in place: the cached plan must not be used
    lengths2 = [50, 350, 1, 177]
    cu.copy_(torch.tensor([0] + list(np.cumsum(lengths2)), dtype=torch.int32, device=gpu))
    print("plan reuse: cu_seqlens rewritten in place", flush=True)
    third = run(cu, 350)
    torch.cuda.synchronize()
    cu2 = cu.cpu().numpy()
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, 0.1, True, cu2, cu2)
    H.check_out(third[0], None, ref_out, ref_lse)
    H.check_grads(third[1:], ref_g)


def test_plan_filled_flag_on_a_plan_no_forward_filled_is_ignored(gpu):
    """plan_filled with a plan the library has no record of filling for this
    problem (garbage): the forward builds the lists anyway."""
    F = _fna2()
    lengths = [70, 3, 200, 129]
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=41)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout, cu_q, cu_k)]
    plan = F._plan_for(g[0], g[1], g[3], g[7], g[8], 200, 200, True, 0.09)
    plan.fill_(0xAB)
    print("plan_filled on an unfilled plan", flush=True)
    out, lse = F._fna2_forward_varlen(*g[:6], g[7], g[8], 200, 200, 0.09, True, plan=plan,
                                      plan_filled=True)
    torch.cuda.synchronize()
    ref_out, ref_lse, _ = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, 0.09, True,
                                           cu_q.numpy(), cu_k.numpy(), backward=False)
    H.check_out(out, lse, ref_out, ref_lse)


def test_varlen_lse_layout_matches_reference(gpu):
    """_fna2_forward_varlen returns lse as a contiguous [T, H] tensor, as the
    reference allocates it (flash_naylis_attn.py:780), with the same values
    as the head-major view the autograd path keeps; the backward reads
    either."""
    F = _fna2()
    lengths = [129, 7, 256]
    (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, 4, 128, 2, 4, 32, seed=8)
    g = [t.to(gpu) for t in (q, k, v, rq, rk, gs_, dout, cu_q, cu_k)]
    out, lse = F._fna2_forward_varlen(*g[:6], g[7], g[8], 256, 256, 0.09, True)
    out2, lse_hm = F._fna2_forward_varlen(*g[:6], g[7], g[8], 256, 256, 0.09, True,
                                          lse_head_major=True)
    assert lse.shape == (sum(lengths), 4) and lse.is_contiguous()
    assert lse_hm.shape == lse.shape and lse_hm.stride() == (1, sum(lengths))
    assert torch.equal(lse, lse_hm) and torch.equal(out, out2)
    lse.view(-1)  # flat views work, as on the reference's tensor
    ga = F._fna2_backward_varlen(g[6], *g[:6], out, lse, g[7], g[8], 256, 256, 0.09, True)
    gb = F._fna2_backward_varlen(g[6], *g[:6], out, lse_hm, g[7], g[8], 256, 256, 0.09, True)
    torch.cuda.synchronize()
    for a, b in zip(ga, gb):
        assert torch.equal(a, b)


@pytest.mark.parametrize("mode", ["varlen", "dense"])
def test_rank_features_past_r_are_never_read(gpu, mode):
    """R = 16 with R_q / R_k as views into 32-wide rows whose other 16
    features are NaN: every kernel must read rank features [0, R) only (a
    read past R would put 0 * NaN into the scores).  Features past R of the
    last graph head's last row lie past the end of a dense R_k allocation,
    so the same rule keeps the kernels inside it."""
    F = _fna2()
    Hq, D, R = 4, 64, 16
    if mode == "varlen":
        lengths = [90, 33, 257]
        (q, k, v, rq, rk, gs_, dout, cu_q, cu_k) = H.make_varlen(lengths, Hq, D, 4, 4, R,
                                                                 seed=41)
        pad = lambda t: torch.cat([t, torch.full_like(t, float("nan"))], -1)[..., :R]
    else:
        q, k, v, rq, rk, gs_, dout = H.make_dense(2, Hq, 160, D, 2, 4, R, seed=42, layout="bshd")
        # [B, S, H, 2R] memory seen as [B, H, S, R]
        pad = lambda t: torch.cat([t.transpose(1, 2), torch.full_like(t.transpose(1, 2),
                                                                      float("nan"))],
                                  -1)[..., :R].transpose(1, 2)
    rq_p, rk_p = pad(rq), pad(rk)
    assert rk_p.stride(-2 if mode == "varlen" else 1) == 2 * R and torch.isnan(
        rk_p.as_strided((rk_p.numel() * 2,), (1,))).any()
    scale = 1.0 / math.sqrt(D)
    print(f"rank views into NaN-padded rows, {mode}", flush=True)
    dev = [t.to(gpu) for t in (q, k, v, rq_p, rk_p, gs_, dout)]
    if mode == "varlen":
        cq, ck = cu_q.to(gpu), cu_k.to(gpu)
        out, lse = F._fna2_forward_varlen(*dev[:6], cq, ck, 257, 257, scale, False)
        grads = F._fna2_backward_varlen(dev[6], *dev[:6], out, lse, cq, ck, 257, 257, scale,
                                        False)
        cuq, cuk = cu_q.numpy(), cu_k.numpy()
        causal = False
    else:
        out, lse = F._fna2_forward(*dev[:6], scale, True)
        grads = F._fna2_backward(dev[6], *dev[:6], out, lse, scale, True)
        cuq = cuk = None
        causal = True
    torch.cuda.synchronize()
    for name, t in zip(("out", "dq", "dk", "dv", "drq", "drk", "dgs"), (out,) + tuple(grads)):
        assert torch.isfinite(t.float()).all(), f"{name}: non-finite values"
    ref_out, ref_lse, ref_g = H.oracle_fwd_bwd(q, k, v, rq, rk, gs_, dout, scale, causal, cuq, cuk)
    H.check_out(out, lse, ref_out, ref_lse)
    H.check_grads(grads, ref_g)
