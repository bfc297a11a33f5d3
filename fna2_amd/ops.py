"""``flash_naylis_attn`` as PyTorch custom operators: ``fna2::fwd`` and
``fna2::bwd``.

The reference wraps its Triton launchers in a plain ``torch.autograd.Function``
(FNA2/flash_naylis_attn.py:1307-1373), which ``torch.compile`` cannot trace
through.  Here the launchers of ``flash_naylis_attn.py`` (which call the HIP
kernels through the C ABI) are registered with ``torch.library.custom_op``:

* ``fna2::fwd(q, k, v, r_q, r_k, graph_scale, softmax_scale, is_causal,
  cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k) -> (out, lse,
  plan)``: ``out`` has q's shape, dtype and strides; ``lse`` is fp32
  ``[B, H, S]`` (dense) or ``[T, H]`` (varlen, a view of head-major memory);
  ``plan`` is the uint8 buffer of the varlen tile lists the backward reuses
  (empty in dense mode);
* ``fna2::bwd(dout, q, k, v, r_q, r_k, graph_scale, out, lse, plan, ...) ->
  (dq, dk, dv, dr_q, dr_k, d_graph_scale)``, absent gradients (no graph
  heads) as empty tensors;
* ``register_fake`` gives both their output metadata from the input shapes
  alone (the plan's size is a closed form of the token and sequence counts),
  so ``torch.compile`` / ``make_fx`` trace them without running a kernel;
* ``register_autograd`` differentiates ``fna2::fwd`` with ``fna2::bwd``.

Both ops have CUDA (HIP) kernels only: CPU tensors raise.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from .flash_naylis_attn import (_fna2_backward, _fna2_backward_varlen, _fna2_forward,
                                _fna2_forward_varlen, _plan_for)

# Tile shapes of the varlen lists (the forward / dQ query tiles and the
# dK/dV key tiles, fna2_kernels.h) and the record size.
_QUERY_TILE = 128
_TILE_RECORD = 32
_ALIGN = 256


def key_tile(head_dim: int, heads_graph: int, rank: int) -> int:
    """Keys per dK/dV item (kv_bn in fna2_kernels.h): 256 at d = 64 with a
    rank tile of at most 32, else 128."""
    rpl = (rank + 31) // 32 * 32 if heads_graph > 0 and rank > 0 else 0
    return 256 if head_dim == 64 and rpl <= 32 else 128


def plan_nbytes(total_q, total_k, nseq, head_dim=128, heads_graph=0, rank=0) -> int:
    """Bytes of a varlen plan (fna2_plan_bytes), from the token counts, the
    number of sequences and the shape that sets the key tile; works on
    symbolic sizes."""
    if nseq <= 0:
        return 0
    up = lambda x: (x + _ALIGN - 1) // _ALIGN * _ALIGN
    kt = key_tile(head_dim, heads_graph, rank)
    tiles_q = (total_q + _QUERY_TILE - 1) // _QUERY_TILE + nseq
    tiles_k = (total_k + kt - 1) // kt + nseq
    return up(_TILE_RECORD * tiles_q) + _ALIGN + up(_TILE_RECORD * tiles_k) + _ALIGN


def _like(ref: Tensor, t: Tensor) -> Tensor:
    """t in ref's layout (empty_like(ref) strides), copying only when the
    launcher had to work on a contiguous copy."""
    if t.stride() == ref.stride() or t.numel() == 0:
        return t
    res = torch.empty_like(ref)
    res.copy_(t)
    return res


def _empty(ref: Tensor) -> Tensor:
    return ref.new_empty((0,))


@torch.library.custom_op("fna2::fwd", mutates_args=(), device_types="cuda")
def fna2_fwd(q: Tensor, k: Tensor, v: Tensor, r_q: Optional[Tensor], r_k: Optional[Tensor],
             graph_scale: Optional[Tensor], softmax_scale: float, is_causal: bool,
             cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor],
             max_seqlen_q: int, max_seqlen_k: int) -> tuple[Tensor, Tensor, Tensor]:
    if cu_seqlens_q is None:
        out, lse = _fna2_forward(q, k, v, r_q, r_k, graph_scale, softmax_scale, is_causal)
        plan = q.new_empty((0,), dtype=torch.uint8)
    else:
        cu_k = cu_seqlens_q if cu_seqlens_k is None else cu_seqlens_k
        plan = _plan_for(q, k, r_q, cu_seqlens_q, cu_k, max_seqlen_q, max_seqlen_k, is_causal,
                         softmax_scale)
        out, lse = _fna2_forward_varlen(q, k, v, r_q, r_k, graph_scale, cu_seqlens_q, cu_k,
                                        max_seqlen_q, max_seqlen_k, softmax_scale, is_causal,
                                        plan=plan, lse_head_major=True)
        if plan is None:
            plan = q.new_empty((0,), dtype=torch.uint8)
    return _like(q, out), lse, plan


@fna2_fwd.register_fake
def _fna2_fwd_fake(q, k, v, r_q, r_k, graph_scale, softmax_scale, is_causal, cu_seqlens_q,
                   cu_seqlens_k, max_seqlen_q, max_seqlen_k):
    out = torch.empty_like(q)
    if cu_seqlens_q is None:
        lse = q.new_empty((q.shape[0], q.shape[1], q.shape[2]), dtype=torch.float32)
        plan = q.new_empty((0,), dtype=torch.uint8)
    else:
        lse = q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32).t()  # head-major
        hg = 0 if r_q is None else r_q.shape[1]
        nbytes = plan_nbytes(q.shape[0], k.shape[0], cu_seqlens_q.shape[0] - 1, q.shape[-1], hg,
                             0 if r_q is None else r_q.shape[-1])
        plan = q.new_empty((nbytes,), dtype=torch.uint8)
    return out, lse, plan


@torch.library.custom_op("fna2::bwd", mutates_args=(), device_types="cuda")
def fna2_bwd(dout: Tensor, q: Tensor, k: Tensor, v: Tensor, r_q: Optional[Tensor],
             r_k: Optional[Tensor], graph_scale: Optional[Tensor], out: Tensor, lse: Tensor,
             plan: Tensor, softmax_scale: float, is_causal: bool,
             cu_seqlens_q: Optional[Tensor], cu_seqlens_k: Optional[Tensor], max_seqlen_q: int,
             max_seqlen_k: int) -> tuple[Tensor, Tensor, Tensor, Tensor, Tensor, Tensor]:
    if cu_seqlens_q is None:
        grads = _fna2_backward(dout, q, k, v, r_q, r_k, graph_scale, out, lse, softmax_scale,
                               is_causal)
    else:
        cu_k = cu_seqlens_q if cu_seqlens_k is None else cu_seqlens_k
        grads = _fna2_backward_varlen(dout, q, k, v, r_q, r_k, graph_scale, out, lse,
                                      cu_seqlens_q, cu_k, max_seqlen_q, max_seqlen_k,
                                      softmax_scale, is_causal,
                                      plan=plan if plan.numel() > 0 else None)
    dq, dk, dv, drq, drk, dgs = grads
    return (_like(q, dq), _like(k, dk), _like(v, dv),
            _like(r_q, drq) if drq is not None else _empty(q),
            _like(r_k, drk) if drk is not None else _empty(q),
            dgs if dgs is not None else _empty(q))


@fna2_bwd.register_fake
def _fna2_bwd_fake(dout, q, k, v, r_q, r_k, graph_scale, out, lse, plan, softmax_scale,
                   is_causal, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k):
    graph = r_q is not None and r_q.shape[1] > 0 and graph_scale is not None
    return (torch.empty_like(q), torch.empty_like(k), torch.empty_like(v),
            torch.empty_like(r_q) if graph else _empty(q),
            torch.empty_like(r_k) if graph else _empty(q),
            torch.empty_like(graph_scale) if graph else _empty(q))


def _setup_context(ctx, inputs, output):
    (q, k, v, r_q, r_k, graph_scale, softmax_scale, is_causal, cu_q, cu_k, max_q,
     max_k) = inputs
    out, lse, plan = output
    ctx.save_for_backward(q, k, v, r_q, r_k, graph_scale, out, lse, plan, cu_q, cu_k)
    ctx.softmax_scale = softmax_scale
    ctx.is_causal = is_causal
    ctx.max_seqlen_q = max_q
    ctx.max_seqlen_k = max_k
    ctx.mark_non_differentiable(lse, plan)
    # Gradients of lse and plan are never used: without this, autograd would
    # fill a zero tensor of each (two fill kernels per backward).
    ctx.set_materialize_grads(False)


def _backward(ctx, dout, _dlse, _dplan):
    q, k, v, r_q, r_k, graph_scale, out, lse, plan, cu_q, cu_k = ctx.saved_tensors
    if dout is None:  # out did not reach the loss
        return (None,) * 12
    dq, dk, dv, drq, drk, dgs = torch.ops.fna2.bwd(
        dout, q, k, v, r_q, r_k, graph_scale, out, lse, plan, ctx.softmax_scale, ctx.is_causal,
        cu_q, cu_k, ctx.max_seqlen_q, ctx.max_seqlen_k)
    opt = lambda g, ref: g if ref is not None and g.numel() == ref.numel() else None
    return (dq, dk, dv, opt(drq, r_q), opt(drk, r_k), opt(dgs, graph_scale),
            None, None, None, None, None, None)


fna2_fwd.register_autograd(_backward, setup_context=_setup_context)
