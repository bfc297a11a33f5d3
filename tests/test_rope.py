"""Varlen RoPE on the HIP kernel (fna2_rope_varlen) against the oracle.

CPU: the C ABI's validation (fna2_check_rope, host only).
GPU: the kernel against oracle/rope_oracle.py in bf16 / fp16 / fp32, with
empty sequences and tokens outside every sequence, strided views (q and k
slices of one fused projection), the backward (autograd of the op against
the oracle's inverse rotation), the module's forward_varlen against the
module's dense RoPE run per sequence, and at the headline size
(16384 tokens, 16 + 16 heads, d = 128) a rotate / rotate-back round trip.

Tolerances: the kernel's cos/sin come from the device's fp32 routine, the
oracle's are correctly rounded: fp32 results agree within 1e-5 absolute
(inputs ~ N(0, 1)); bf16 / fp16 results are bit-equal except where cos or
sin straddle a rounding boundary (> 99.9 % equal, the rest within 2 ulp).
"""
import ctypes

import numpy as np
import pytest
import torch

from fna2_amd import _capi
from oracle import rope_oracle as RO

FAKE = 1 << 20
DT = {torch.bfloat16: "bf16", torch.float16: "f16", torch.float32: "f32"}


@pytest.fixture(scope="module")
def lib():
    return _capi.lib()


def _args(**over):
    a = _capi.RopeArgs()
    a.dtype, a.total_tokens, a.heads_q, a.heads_k, a.head_dim = 1, 64, 4, 2, 128
    a.nseq, a.sign, a.cu_seqlens, a.inv_freq = 2, 1, FAKE, FAKE
    a.q = _capi.Tensor(FAKE, 0, 4 * 128, 128)
    a.k = _capi.Tensor(FAKE + (1 << 24), 0, 2 * 128, 128)
    a.q_out = _capi.Tensor(FAKE + (2 << 24), 0, 4 * 128, 128)
    a.k_out = _capi.Tensor(FAKE + (3 << 24), 0, 2 * 128, 128)
    for k, v in over.items():
        setattr(a, k, v)
    return a


def _check(lib, a):
    return _capi.STATUS[lib.fna2_check_rope(ctypes.byref(a))]


def _bwd(lib, **over):
    b = _capi.RopeBwdArgs()
    b.fwd = _args()
    b.fwd.norm_q, b.fwd.norm_eps = FAKE, 1e-6
    b.dq_out = _capi.Tensor(FAKE + (4 << 24), 0, 4 * 128, 128)
    b.dk_out = _capi.Tensor(FAKE + (5 << 24), 0, 2 * 128, 128)
    b.dq = _capi.Tensor(FAKE + (6 << 24), 0, 4 * 128, 128)
    b.dk = _capi.Tensor(FAKE + (7 << 24), 0, 2 * 128, 128)
    b.dnorm_q = FAKE
    b.workspace, b.workspace_bytes = FAKE, 1 << 30
    for k, v in over.items():
        setattr(b, k, v)
    return _capi.STATUS[lib.fna2_check_rope_bwd(ctypes.byref(b))]


def test_check_rope_bwd(lib):
    assert _bwd(lib) == "FNA2_OK"
    assert _bwd(lib, workspace=None) == "FNA2_E_WORKSPACE"
    assert _bwd(lib, workspace_bytes=16) == "FNA2_E_WORKSPACE"
    assert _bwd(lib, dnorm_q=None) == "FNA2_E_NULL"
    assert _bwd(lib, dq=_capi.Tensor(FAKE + (4 << 24) + 256, 0, 4 * 128, 128)) == "FNA2_E_ALIAS"
    a = _args()
    assert lib.fna2_rope_bwd_workspace_bytes(ctypes.byref(a)) == 0  # no norm: none
    a.norm_k, a.norm_eps = FAKE, 1e-6
    assert lib.fna2_rope_bwd_workspace_bytes(ctypes.byref(a)) >= 2 * 4 * 128 * 4
    a.norm_eps = float("nan")
    assert _check(lib, a) == "FNA2_E_SCALE"


def test_check_rope_accepts(lib):
    assert _check(lib, _args()) == "FNA2_OK"
    assert _check(lib, _args(dtype=3, head_dim=64)) == "FNA2_OK"
    # in place
    assert _check(lib, _args(q_out=_capi.Tensor(FAKE, 0, 4 * 128, 128))) == "FNA2_OK"
    # nothing to do: no pointers needed
    assert _check(lib, _args(total_tokens=0, cu_seqlens=None, inv_freq=None)) == "FNA2_OK"


@pytest.mark.parametrize("over,code", [
    (dict(dtype=4), "FNA2_E_DTYPE"),
    (dict(head_dim=96), "FNA2_E_HEAD_DIM"),
    (dict(head_dim=8), "FNA2_E_HEAD_DIM"),
    (dict(head_dim=1024), "FNA2_E_HEAD_DIM"),
    (dict(sign=0), "FNA2_E_SHAPE"),
    (dict(total_tokens=-1), "FNA2_E_SHAPE"),
    (dict(cu_seqlens=None), "FNA2_E_SEQLENS"),
    (dict(inv_freq=None), "FNA2_E_NULL"),
    (dict(q=_capi.Tensor(None, 0, 512, 128)), "FNA2_E_NULL"),
    (dict(q=_capi.Tensor(FAKE + 8, 0, 512, 128)), "FNA2_E_STRIDE"),
    (dict(k=_capi.Tensor(FAKE + (1 << 24), 0, 2 * 128 + 4, 128)), "FNA2_E_STRIDE"),
    # same base, other strides; overlapping ranges
    (dict(q_out=_capi.Tensor(FAKE, 0, 4 * 128, 256)), "FNA2_E_ALIAS"),
    (dict(q_out=_capi.Tensor(FAKE + 4 * 128 * 2, 0, 4 * 128, 128)), "FNA2_E_ALIAS"),
])
def test_check_rope_rejects(lib, over, code):
    assert _check(lib, _args(**over)) == code


def _case(T, H, HKV, D, cu, dtype, seed, device):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(T, H, D, generator=g).to(dtype)
    k = torch.randn(T, HKV, D, generator=g).to(dtype)
    inv = torch.from_numpy(RO.inv_freq_default(D))
    return q.to(device), k.to(device), torch.tensor(cu, dtype=torch.int32, device=device), inv


def _compare(got, want, dtype):
    got = got.to(torch.float64).cpu().numpy()
    if dtype == torch.float32:
        np.testing.assert_allclose(got, want, rtol=0, atol=1e-5)
        return
    diff = np.abs(got - want)
    assert (diff == 0).mean() > 0.999, (diff > 0).mean()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert (diff <= 2 * ulp * np.maximum(np.abs(want), 2.0 ** -14)).all()


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("D", [64, 128])
def test_kernel_matches_oracle(gpu, dtype, D):
    from fna2_amd.rope import rope_varlen_raw
    lens = [700, 0, 33, 1, 1024, 5, 257]
    cu = [7] + list(7 + np.cumsum(lens))
    T = cu[-1] + 9  # tokens before cu[0] and after cu[N]: unchanged
    q, k, cu_t, inv = _case(T, 6, 2, D, cu, dtype, 1, gpu)
    print(f"rope parity dtype={dtype} D={D} T={T}", flush=True)
    yq, yk = rope_varlen_raw(q, k, cu_t, inv.to(gpu))
    torch.cuda.synchronize()
    wq, wk = RO.rope_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(), cu,
                            inv.numpy(), DT[dtype])
    _compare(yq, wq, dtype)
    _compare(yk, wk, dtype)


@pytest.mark.gpu
def test_strided_views_and_single_tensor(gpu):
    """q and k as slices of one fused [T, H + 2 H_KV, D] projection."""
    from fna2_amd.rope import rope_varlen_raw
    T, H, HKV, D = 333, 4, 2, 128
    cu = [0, 100, 333]
    g = torch.Generator().manual_seed(2)
    qkv = torch.randn(T, H + 2 * HKV, D, generator=g).to(torch.bfloat16).to(gpu)
    q, k = qkv[:, :H], qkv[:, H:H + HKV]
    inv = torch.from_numpy(RO.inv_freq_default(D))
    print("rope strided views", flush=True)
    yq, yk = rope_varlen_raw(q, k, torch.tensor(cu, dtype=torch.int32, device=gpu), inv.to(gpu))
    torch.cuda.synchronize()
    wq, wk = RO.rope_varlen(q.float().cpu().numpy(), k.float().cpu().numpy(), cu, inv.numpy(), "bf16")
    _compare(yq, wq, torch.bfloat16)
    _compare(yk, wk, torch.bfloat16)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_is_inverse_rotation(gpu, dtype):
    from fna2_amd.rope import rope_varlen
    T, D = 600, 64
    cu = [0, 250, 250, 600]
    q, k, cu_t, inv = _case(T, 4, 2, D, cu, dtype, 3, gpu)
    q.requires_grad_(True)
    k.requires_grad_(True)
    g = torch.Generator().manual_seed(4)
    gq = torch.randn(q.shape, generator=g).to(dtype).to(gpu)
    gk = torch.randn(k.shape, generator=g).to(dtype).to(gpu)
    print(f"rope backward dtype={dtype}", flush=True)
    yq, yk = rope_varlen(q, k, cu_t, inv.to(gpu))
    torch.autograd.backward([yq, yk], [gq, gk])
    torch.cuda.synchronize()
    wq, wk = RO.rope_varlen(gq.float().cpu().numpy(), gk.float().cpu().numpy(), cu, inv.numpy(),
                            DT[dtype], sign=-1)
    _compare(q.grad, wq, dtype)
    _compare(k.grad, wk, dtype)


@pytest.mark.gpu
def test_module_varlen_equals_dense_per_sequence(gpu):
    from fna2_amd import attention_fna2 as A
    rope = A.RotaryPositionalEmbedding(64, max_seq_len=512).to(gpu)
    lens = [5, 17, 1, 40]
    cu = torch.tensor([0, 5, 22, 23, 63], dtype=torch.int32, device=gpu)
    g = torch.Generator().manual_seed(5)
    q = torch.randn(sum(lens), 4, 64, generator=g).to(gpu)
    k = torch.randn(sum(lens), 2, 64, generator=g).to(gpu)
    print("rope module varlen vs dense", flush=True)
    qo, ko = rope.forward_varlen(q, k, cu)
    off = 0
    for n in lens:
        qs = q[off:off + n].transpose(0, 1)[None]
        ks = k[off:off + n].transpose(0, 1)[None]
        qr, kr = rope(qs, ks)
        torch.testing.assert_close(qo[off:off + n], qr[0].transpose(0, 1), atol=1e-5, rtol=1e-5)
        torch.testing.assert_close(ko[off:off + n], kr[0].transpose(0, 1), atol=1e-5, rtol=1e-5)
        off += n


@pytest.mark.gpu
def test_headline_size_round_trip(gpu):
    """16384 tokens of the c3 pack, 16 + 16 heads, d = 128, fp32: rotating
    back recovers the input (a size-independent property)."""
    import json
    from pathlib import Path

    from fna2_amd.rope import rope_varlen_raw
    cu = json.loads((Path(__file__).parent / "golden" / "cu_seqlens.json").read_text())["c3"]["cu_seqlens"]
    T = cu[-1]
    q, k, cu_t, inv = _case(T, 16, 16, 128, cu, torch.float32, 6, gpu)
    print(f"rope round trip T={T}", flush=True)
    yq, yk = rope_varlen_raw(q, k, cu_t, inv.to(gpu))
    bq, bk = rope_varlen_raw(yq, yk, cu_t, inv.to(gpu), -1)
    torch.cuda.synchronize()
    assert (bq - q).abs().max().item() < 1e-5
    assert (bk - k).abs().max().item() < 1e-5
    # and the rotation moved every token past position 0
    pos0 = torch.zeros(T, dtype=torch.bool, device=gpu)
    pos0[cu_t[:-1].long()] = True
    assert torch.equal(yq[pos0], q[pos0])
    assert (yq[~pos0] - q[~pos0]).abs().max().item() > 0.1


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("which", ["both", "q"])
def test_norm_rope_forward_backward(gpu, dtype, which):
    """QK-RMSNorm + RoPE in one launch, and its backward (inputs and norm
    weights), against the oracle: fp32 chain rounded once (forward); float64
    gradients on the same (rounded) inputs."""
    from fna2_amd.rope import rope_varlen
    lens = [300, 0, 1, 77, 500]
    cu = [3] + list(3 + np.cumsum(lens))
    T, D = cu[-1] + 5, 128
    q, k, cu_t, inv = _case(T, 4, 2, D, cu, dtype, 30, gpu)
    g = torch.Generator().manual_seed(31)
    wq = (1 + 0.3 * torch.randn(D, generator=g)).to(gpu)
    wk = (1 + 0.3 * torch.randn(D, generator=g)).to(gpu) if which == "both" else None
    gq = torch.randn(q.shape, generator=g).to(dtype).to(gpu)
    gk = torch.randn(k.shape, generator=g).to(dtype).to(gpu)
    leaves = [q.clone().requires_grad_(True), k.clone().requires_grad_(True),
              wq.clone().requires_grad_(True)] + ([wk.clone().requires_grad_(True)] if wk is not None else [])
    print(f"norm rope dtype={dtype} which={which}", flush=True)
    yq, yk = rope_varlen(leaves[0], leaves[1], cu_t, inv.to(gpu), leaves[2],
                         leaves[3] if wk is not None else None, 1e-6)
    grads = torch.autograd.grad([yq, yk], leaves, [gq, gk])
    torch.cuda.synchronize()
    npy = lambda t: None if t is None else t.detach().float().cpu().numpy()
    wq_n, wk_n = npy(wq), npy(wk)
    fq, fk = RO.norm_rope_varlen(npy(q), npy(k), cu, inv.numpy(), wq_n, wk_n, 1e-6, DT[dtype])
    _compare_loose = (lambda got, want: np.testing.assert_allclose(
        got.detach().float().cpu().numpy(), want, rtol=0,
        atol=1e-5 if dtype == torch.float32 else 1.5e-2))
    _compare_loose(yq, fq)
    _compare_loose(yk, fk)
    dq, dk, dwq, dwk = RO.norm_rope_grads(npy(q), npy(k), cu, inv.numpy(), wq_n, wk_n, 1e-6,
                                          npy(gq), npy(gk))
    rel = lambda got, want: np.linalg.norm(npy(got) - want) / np.linalg.norm(want)
    tol = 1e-5 if dtype == torch.float32 else 1e-2
    assert rel(grads[0], dq) < tol and rel(grads[1], dk) < tol
    assert rel(grads[2], dwq) < tol
    if wk is not None:
        assert rel(grads[3], dwk) < tol
    # determinism of the weight gradients (fixed-order sums)
    grads2 = torch.autograd.grad(list(rope_varlen(leaves[0], leaves[1], cu_t, inv.to(gpu), leaves[2],
                                                  leaves[3] if wk is not None else None, 1e-6)),
                                 leaves, [gq, gk])
    for a, b in zip(grads, grads2):
        assert torch.equal(a, b)

