"""One-token decode against a KV cache (fna2_decode) against the oracle.

CPU: the C ABI's validation (fna2_check_decode, host only), the split count
and workspace size; the module's cache format and its eager decode with the
cached R_k against the module's own full forward.
GPU: the decode kernel against oracle.decode (fp64 on the same bf16 inputs)
over head groups of 1 to 32, vanilla heads inside a group, ranks whose chunk
count is odd, ragged and empty cache lengths, several split counts and
softmax scales of both signs and zero; caches read in place from strided
buffers (capacity above the lengths, token-major layout); and, at sizes the
oracle is slow for, two size-independent identities: decode equals the last
row of the causal forward kernel over the sequence, and the result does not
depend on the split count.  The module's decode step (kernel) equals its
full forward's last row (with decode_graph_bias) and the reference's SDPA
decode step (without).

Tolerances (the attention path's): out 2e-2 max abs (bf16), LSE 1e-2.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from fna2_amd import _capi
from oracle import fna2_oracle as O
from tests.helpers import TOL_LSE, TOL_OUT, check_out, max_abs

FAKE = 1 << 20


@pytest.fixture(scope="module")
def lib():
    return _capi.lib()


def _args(**over):
    a = _capi.DecodeArgs()
    a.batch, a.heads, a.heads_kv, a.heads_graph = 4, 16, 4, 12
    a.head_dim, a.rank, a.max_seqlen_k, a.num_splits = 128, 32, 4096, 0
    a.softmax_scale = 0.088
    a.q = _capi.Tensor(FAKE, 16 * 128, 0, 128)
    a.r_q = _capi.Tensor(FAKE, 12 * 32, 0, 32)
    a.k_cache = _capi.Tensor(FAKE, 4 * 4096 * 128, 128, 4096 * 128)
    a.v_cache = _capi.Tensor(FAKE, 4 * 4096 * 128, 128, 4096 * 128)
    a.rk_cache = _capi.Tensor(FAKE, 12 * 4096 * 32, 32, 4096 * 32)
    a.graph_scale = FAKE
    a.out = _capi.Tensor(FAKE, 16 * 128, 0, 128)
    for k, v in over.items():
        setattr(a, k, v)
    return a


def _check(lib, a):
    return _capi.STATUS[lib.fna2_check_decode(ctypes.byref(a))]


def test_check_decode_codes(lib):
    assert _check(lib, _args()) == "FNA2_OK"
    assert _check(lib, _args(q=_capi.empty_tensor())) == "FNA2_E_NULL"
    assert _check(lib, _args(graph_scale=None)) == "FNA2_E_NULL"
    assert _check(lib, _args(heads_graph=0, graph_scale=None, r_q=_capi.empty_tensor(),
                             rk_cache=_capi.empty_tensor())) == "FNA2_OK"
    assert _check(lib, _args(head_dim=96)) == "FNA2_E_HEAD_DIM"
    assert _check(lib, _args(heads_kv=3)) == "FNA2_E_HEADS"
    assert _check(lib, _args(heads=64, heads_kv=1, heads_graph=0)) == "FNA2_E_HEADS"  # group 64
    assert _check(lib, _args(heads_graph=17)) == "FNA2_E_HEADS"
    assert _check(lib, _args(rank=12)) == "FNA2_E_RANK"
    # a group of 8 graph heads at rank 64 is 512 rank columns (> 256)
    assert _check(lib, _args(heads=8, heads_kv=1, heads_graph=8, rank=64)) == "FNA2_E_RANK"
    assert _check(lib, _args(heads=8, heads_kv=1, heads_graph=4, rank=64)) == "FNA2_OK"
    assert _check(lib, _args(num_splits=65)) == "FNA2_E_SHAPE"
    assert _check(lib, _args(max_seqlen_k=-1)) == "FNA2_E_SHAPE"
    assert _check(lib, _args(softmax_scale=float("nan"))) == "FNA2_E_SCALE"
    assert _check(lib, _args(q=_capi.Tensor(FAKE + 8, 16 * 128, 0, 128))) == "FNA2_E_STRIDE"
    assert _check(lib, _args(k_cache=_capi.Tensor(FAKE, 4 * 4096 * 128, 132, 4096 * 128))) \
        == "FNA2_E_STRIDE"
    # a row stride whose 32-row tile passes 2 GiB
    assert _check(lib, _args(k_cache=_capi.Tensor(FAKE, 0, 1 << 25, 128))) == "FNA2_E_SHAPE"
    assert _check(lib, _args(batch=0)) == "FNA2_OK"


def test_split_count_and_workspace(lib):
    a = _args(batch=32, heads=32, heads_kv=8, heads_graph=32, max_seqlen_k=8192)
    n = lib.fna2_decode_num_splits(ctypes.byref(a))
    assert 1 < n <= 64
    keys = -(-8192 // n)
    assert lib.fna2_decode_workspace_bytes(ctypes.byref(a)) >= n * 32 * 32 * (128 + 2) * 4
    a.num_splits = 3
    assert lib.fna2_decode_num_splits(ctypes.byref(a)) == 3
    a.num_splits, a.max_seqlen_k = 8, 40  # at most one split per 32 keys
    assert lib.fna2_decode_num_splits(ctypes.byref(a)) == 2
    a.num_splits = 1
    assert lib.fna2_decode_workspace_bytes(ctypes.byref(a)) == 0
    a.num_splits, a.max_seqlen_k = 0, 0
    assert lib.fna2_decode_num_splits(ctypes.byref(a)) == 1
    assert keys > 0


# ── GPU ───────────────────────────────────────────────────────────────────────

def _case(B, H, HKV, HG, D, R, L, seed, device):
    g = torch.Generator().manual_seed(seed)
    draw = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16().to(device)
    q = draw(B, H, D)
    k = draw(B, HKV, L, D)
    v = draw(B, HKV, L, D)
    rq = draw(B, HG, R, std=R ** -0.5) if HG else None
    rk = draw(B, HG, L, R, std=R ** -0.5) if HG else None
    gs = (torch.randn(HG, generator=g) * 2).float().to(device) if HG else None
    return q, k, v, rq, rk, gs


CASES = [
    # B, H, HKV, HG, D, R, L, lengths
    (3, 8, 2, 6, 128, 32, 300, [300, 1, 77]),     # group 4, vanilla heads in group 2
    (2, 4, 4, 4, 64, 16, 97, [97, 33]),          # group 1
    (2, 16, 2, 0, 128, 0, 130, [130, 64]),       # no graph heads, group 8
    (2, 8, 2, 3, 128, 24, 200, [200, 31]),       # rank 24: 3 chunks a head
    (1, 32, 1, 8, 64, 8, 150, [150]),            # group 32
    (2, 8, 1, 8, 128, 32, 96, [96, 95]),         # 8 graph heads x 32 = widest rank tile
    (2, 4, 2, 4, 128, 64, 64, [0, 64]),          # an empty cache
    # the remaining kernel instances (head dim x rank-tile chunks)
    (2, 8, 8, 8, 128, 32, 90, [90, 45]),         # d128, 4 rank chunks
    (2, 8, 4, 8, 128, 32, 90, [90, 3]),          # d128, 8 rank chunks
    (2, 8, 2, 0, 64, 0, 90, [90, 60]),           # d64, no graph heads
    (2, 8, 2, 8, 64, 32, 90, [90, 61]),          # d64, 16 rank chunks
    (2, 8, 2, 8, 64, 64, 90, [90, 33]),          # d64, 32 rank chunks
]


@pytest.mark.gpu
@pytest.mark.parametrize("case", CASES, ids=lambda c: f"B{c[0]}H{c[1]}kv{c[2]}G{c[3]}d{c[4]}r{c[5]}")
@pytest.mark.parametrize("splits", [0, 1, 5])
def test_decode_matches_oracle(gpu, case, splits):
    from fna2_amd.decode import flash_naylis_decode
    B, H, HKV, HG, D, R, L, lens = case
    q, k, v, rq, rk, gs = _case(B, H, HKV, HG, D, R, L, seed=len(lens) * 100 + D + R, device=gpu)
    seq = torch.tensor(lens, dtype=torch.int32, device=gpu)
    scale = 1.0 / math.sqrt(D)
    print(f"decode case {case} splits {splits}", flush=True)
    out, lse = flash_naylis_decode(q, k, v, rq, rk, gs, softmax_scale=scale, cache_seqlens=seq,
                                   num_splits=splits, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_l = O.decode(q, k, v, rq, rk, gs, scale, seqlens=lens)
    check_out(out, lse, ref_o, ref_l)


@pytest.mark.gpu
@pytest.mark.parametrize("scale", [-0.3, 0.0])
def test_decode_scale_sign_and_zero(gpu, scale):
    from fna2_amd.decode import flash_naylis_decode
    q, k, v, rq, rk, gs = _case(2, 8, 2, 8, 128, 32, 120, seed=5, device=gpu)
    out, lse = flash_naylis_decode(q, k, v, rq, rk, gs, softmax_scale=scale, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_l = O.decode(q, k, v, rq, rk, gs, scale)
    check_out(out, lse, ref_o, ref_l)


@pytest.mark.gpu
def test_decode_all_empty_and_no_batch(gpu):
    from fna2_amd.decode import flash_naylis_decode
    q, k, v, rq, rk, gs = _case(2, 8, 2, 8, 128, 32, 0, seed=6, device=gpu)
    out, lse = flash_naylis_decode(q, k, v, rq, rk, gs, return_lse=True)
    torch.cuda.synchronize()
    assert torch.all(out == 0) and torch.all(torch.isneginf(lse))
    q0 = q[:0]
    out0 = flash_naylis_decode(q0, k[:0], v[:0], rq[:0], rk[:0], gs)
    assert out0.shape == (0, 8, 128)


@pytest.mark.gpu
def test_decode_reads_strided_caches_in_place(gpu):
    """Caches as slices of larger buffers (capacity 512 > 300 rows), and a
    token-major [B, L, H, D] buffer: bit-equal to contiguous caches."""
    from fna2_amd.decode import flash_naylis_decode
    B, H, HKV, HG, D, R, L = 2, 8, 2, 8, 128, 32, 300
    q, k, v, rq, rk, gs = _case(B, H, HKV, HG, D, R, L, seed=7, device=gpu)
    seq = torch.tensor([300, 211], dtype=torch.int32, device=gpu)
    base = flash_naylis_decode(q, k, v, rq, rk, gs, cache_seqlens=seq)
    cap = 512

    def padded(t):
        buf = torch.zeros(t.shape[0], t.shape[1], cap, t.shape[3], dtype=t.dtype, device=gpu)
        buf[:, :, :L] = t
        return buf[:, :, :L]

    def token_major(t):
        buf = torch.zeros(t.shape[0], cap, t.shape[1], t.shape[3], dtype=t.dtype, device=gpu)
        buf[:, :L] = t.transpose(1, 2)
        return buf[:, :L].transpose(1, 2)

    for f in (padded, token_major):
        got = flash_naylis_decode(q, f(k), f(v), rq, f(rk), gs, cache_seqlens=seq)
        torch.cuda.synchronize()
        assert torch.equal(got, base), f.__name__


@pytest.mark.gpu
def test_decode_is_last_row_of_causal_forward(gpu):
    """Size-independent identity at a long cache (2048 rows): the decode of
    row len-1 equals row len-1 of the causal forward kernel."""
    from fna2_amd.decode import flash_naylis_decode
    from fna2_amd.flash_naylis_attn import flash_naylis_attn
    B, H, HKV, HG, D, R, L = 2, 16, 4, 12, 128, 32, 2048
    g = torch.Generator().manual_seed(8)
    draw = lambda *s, std=1.0: (torch.randn(*s, generator=g) * std).bfloat16().to(gpu)
    q, k, v = draw(B, H, L, D), draw(B, HKV, L, D), draw(B, HKV, L, D)
    rq, rk = draw(B, HG, L, R, std=R ** -0.5), draw(B, HG, L, R, std=R ** -0.5)
    gs = (torch.randn(HG, generator=g) * 2).float().to(gpu)
    scale = D ** -0.5
    full = flash_naylis_attn(q, k, v, rq, rk, gs, softmax_scale=scale, is_causal=True)
    lens = [L, 1500]
    seq = torch.tensor(lens, dtype=torch.int32, device=gpu)
    qd = torch.stack([q[b, :, lens[b] - 1] for b in range(B)])
    rqd = torch.stack([rq[b, :, lens[b] - 1] for b in range(B)])
    out = flash_naylis_decode(qd, k, v, rqd, rk, gs, softmax_scale=scale, cache_seqlens=seq)
    torch.cuda.synchronize()
    ref = torch.stack([full[b, :, lens[b] - 1] for b in range(B)])
    err = max_abs(out, ref)
    assert err < TOL_OUT, err


@pytest.mark.gpu
def test_decode_split_count_invariance(gpu):
    """At 16384 cached rows: one split, the library's choice and 64 splits
    agree (only the fp32 summation order differs)."""
    from fna2_amd.decode import flash_naylis_decode
    q, k, v, rq, rk, gs = _case(2, 16, 2, 16, 128, 16, 16384, seed=9, device=gpu)
    outs = [flash_naylis_decode(q, k, v, rq, rk, gs, num_splits=n, return_lse=True)
            for n in (1, 0, 64)]
    torch.cuda.synchronize()
    for o, l in outs[1:]:
        assert max_abs(o, outs[0][0]) < 1e-2
        assert max_abs(l, outs[0][1]) < 1e-4


@pytest.mark.gpu
def test_decode_long_cache_against_oracle(gpu):
    """200,000 cached rows (the 64-split cap; Rk of 8 graph heads spans
    100 MB of one (sequence, KV head)), against the oracle."""
    from fna2_amd.decode import flash_naylis_decode
    B, H, HKV, HG, D, R, L = 1, 8, 1, 8, 128, 32, 200_000
    q, k, v, rq, rk, gs = _case(B, H, HKV, HG, D, R, L, seed=10, device=gpu)
    seq = torch.tensor([L - 7], dtype=torch.int32, device=gpu)
    out, lse = flash_naylis_decode(q, k, v, rq, rk, gs, softmax_scale=D ** -0.5,
                                   cache_seqlens=seq, return_lse=True)
    torch.cuda.synchronize()
    ref_o, ref_l = O.decode(q, k, v, rq, rk, gs, D ** -0.5, seqlens=[L - 7])
    check_out(out, lse, ref_o, ref_l)
