"""One-token decode against a KV cache on the gfx950 HIP kernels.

``flash_naylis_decode`` computes, for each sequence b and query head h, the
attention of the one new query row over the first ``cache_seqlens[b]`` rows
of the cache (all visible, the new token's row included):

    S_j = softmax_scale <q_h, K_j> + [h < H_G] graph_scale[h] <rq_h, Rk_hj>

normalised as the training kernels normalise (``O = sum e^{S-m} V / (l +
1e-6)``), so it equals the last row of ``flash_naylis_attn(..., is_causal=
True)`` over the whole sequence.

The reference decodes a step with PyTorch SDPA over
``torch.cat(past_kv, new)`` and drops the graph bias, because its cache holds
no ``R_k`` (FNA2/attention_fna2.py:412-429, :445-473).  Without ``r_q`` this
op is that decode step; with ``r_q`` / ``rk_cache`` the bias is kept.

Caches are ``[B, H_KV, L, D]`` views (``rk_cache``: ``[B, H_G, L, R]``) with
any batch / head / row strides, e.g. slices of a preallocated buffer whose
capacity exceeds the lengths: nothing is copied.  Forward only (no autograd).
There is no fallback: without the HIP library, or off the GPU, it raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple, Union

import torch

from . import _capi


def _rows(t: torch.Tensor, name: str) -> torch.Tensor:
    """[B, H, F] (a [B, H, 1, F] query is squeezed): unit feature stride,
    16-byte aligned rows, else a contiguous copy (queries are small)."""
    if t.dim() == 4:
        assert t.shape[2] == 1, f"{name}: one query row per sequence expected"
        t = t[:, :, 0]
    assert t.dim() == 3, f"{name}: [B, H, F] expected"
    ok = (t.stride(2) == 1 and t.data_ptr() % 16 == 0
          and t.stride(0) % 8 == 0 and t.stride(1) % 8 == 0)
    return t if ok else t.contiguous()


def _cache(t: torch.Tensor, name: str) -> torch.Tensor:
    assert t.dim() == 4, f"{name}: [B, heads, L, F] expected"
    ok = (t.stride(3) == 1 and t.data_ptr() % 16 == 0
          and all(s % 8 == 0 for s in t.stride()[:3]))
    if not ok:
        raise AssertionError(f"{name}: the cache needs a unit feature stride and 16-byte "
                             "aligned rows (it is read in place, never copied)")
    return t


def _t3(t: Optional[torch.Tensor]) -> _capi.Tensor:
    if t is None:
        return _capi.empty_tensor()
    return _capi.Tensor(t.data_ptr(), t.stride(0), 0, t.stride(1))


def _t4(t: Optional[torch.Tensor]) -> _capi.Tensor:
    if t is None:
        return _capi.empty_tensor()
    return _capi.Tensor(t.data_ptr(), t.stride(0), t.stride(2), t.stride(1))


def decode_args(q, k_cache, v_cache, r_q=None, rk_cache=None, graph_scale=None,
                softmax_scale=None, cache_seqlens=None, num_splits: int = 0):
    """(DecodeArgs, tensors kept alive, out, lse): the C-ABI arguments of a call,
    with its output buffers allocated (workspace not yet attached)."""
    q = _rows(q, "q")
    B, H, D = q.shape
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache)):
        assert t.dtype == torch.bfloat16, f"{name} must be bfloat16"
        if not t.is_cuda:
            raise RuntimeError("flash_naylis_decode runs on the gfx950 HIP kernel: "
                               "tensors must be on the GPU")
    k_cache, v_cache = _cache(k_cache, "k_cache"), _cache(v_cache, "v_cache")
    assert k_cache.shape == v_cache.shape, "k_cache and v_cache must have one shape"
    assert k_cache.shape[0] == B and k_cache.shape[3] == D, "cache and q disagree"
    H_KV, L = k_cache.shape[1], k_cache.shape[2]
    H_G = R = 0
    gs = None
    if r_q is not None:
        assert rk_cache is not None and graph_scale is not None, \
            "r_q needs rk_cache and graph_scale"
        r_q = _rows(r_q, "r_q")
        rk_cache = _cache(rk_cache, "rk_cache")
        assert r_q.dtype == torch.bfloat16 and rk_cache.dtype == torch.bfloat16, \
            "r_q and rk_cache must be bfloat16"
        H_G, R = r_q.shape[1], r_q.shape[2]
        assert rk_cache.shape == (B, H_G, L, R), "rk_cache must be [B, H_G, L, R]"
        gs = graph_scale.detach().to(device=q.device, dtype=torch.float32).contiguous()
        assert gs.numel() == H_G, "graph_scale must hold H_G values"
    seq = None
    if cache_seqlens is not None:
        seq = cache_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
        assert seq.numel() == B, "cache_seqlens must hold B lengths"
    scale = float(softmax_scale) if softmax_scale is not None else D ** -0.5
    out = torch.empty((B, H, D), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, H), dtype=torch.float32, device=q.device)
    a = _capi.DecodeArgs()
    a.batch, a.heads, a.heads_kv, a.heads_graph = B, H, H_KV, H_G
    a.head_dim, a.rank, a.max_seqlen_k = D, R, L
    a.num_splits = int(num_splits)
    a.softmax_scale = scale
    a.seqlens_k = None if seq is None else seq.data_ptr()
    a.q, a.r_q = _t3(q), _t3(r_q)
    a.k_cache, a.v_cache, a.rk_cache = _t4(k_cache), _t4(v_cache), _t4(rk_cache)
    a.graph_scale = None if gs is None else gs.data_ptr()
    a.out = _t3(out)
    a.lse = _capi.Tensor(lse.data_ptr(), lse.stride(0), 0, lse.stride(1))
    keep = (q, r_q, k_cache, v_cache, rk_cache, gs, seq)
    return a, keep, out, lse


def decode_supported(heads: int, heads_kv: int, head_dim: int, heads_graph: int = 0,
                     rank: int = 0) -> bool:
    """Whether the decode kernel takes this head geometry: the structural
    limits fna2_check_decode enforces (query heads per KV head <= 32, the
    graph heads of one KV-head group times R within one 256-wide rank tile,
    D in {64, 128}), asked of the library itself with an empty batch (a
    host-only call).  Callers send other shapes to an eager path."""
    a = _capi.DecodeArgs()
    a.batch, a.heads, a.heads_kv, a.heads_graph = 0, int(heads), int(heads_kv), int(heads_graph)
    a.head_dim, a.rank, a.max_seqlen_k, a.num_splits = int(head_dim), int(rank), 0, 0
    a.softmax_scale = 1.0
    try:
        return _capi.lib().fna2_check_decode(ctypes.byref(a)) == 0
    except (OSError, RuntimeError):
        return False


def flash_naylis_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        r_q: Optional[torch.Tensor] = None,
                        rk_cache: Optional[torch.Tensor] = None,
                        graph_scale: Optional[torch.Tensor] = None,
                        softmax_scale: Optional[float] = None,
                        cache_seqlens: Optional[torch.Tensor] = None,
                        num_splits: int = 0, return_lse: bool = False
                        ) -> Union[torch.Tensor, Tuple[torch.Tensor, torch.Tensor]]:
    """Decode one token per sequence.

    q ``[B, H, D]`` (or ``[B, H, 1, D]``), k_cache / v_cache
    ``[B, H_KV, L, D]``, r_q ``[B, H_G, R]``, rk_cache ``[B, H_G, L, R]``,
    graph_scale ``[H_G]``, cache_seqlens ``[B]`` (rows in use, <= L; None:
    all L).  bf16.  Returns out ``[B, H, D]`` bf16 (and the fp32 LSE
    ``[B, H]``).  ``num_splits`` 0 lets the library split the keys."""
    a, keep, out, lse = decode_args(q, k_cache, v_cache, r_q, rk_cache, graph_scale,
                                    softmax_scale, cache_seqlens, num_splits)
    lib = _capi.lib()
    _capi.raise_for(lib.fna2_check_decode(ctypes.byref(a)), "fna2_decode")
    nbytes = lib.fna2_decode_workspace_bytes(ctypes.byref(a))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=out.device)
    a.workspace, a.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(out.device):
        stream = ctypes.c_void_p(torch.cuda.current_stream(out.device).cuda_stream)
        _capi.raise_for(lib.fna2_decode(ctypes.byref(a), stream), "fna2_decode")
    del keep
    return (out, lse) if return_lse else out
