"""Varlen rotary position embedding (and QK-RMSNorm) on the gfx950 HIP kernels.

Replaces the reference's ``NaylisAttention._apply_rope_varlen``
(FNA2/attention_fna2.py:620-647), which walks the packed sequences on the
host (``cu_seqlens.tolist()``: a device synchronisation per call) and
applies ``RotaryPositionalEmbedding.forward`` (:163-170) to each.  Here one
launch (``fna2_rope_varlen`` in ``include/fna2.h``) rotates every token of q
and k, with the position ``t - cu_seqlens[seq(t)]`` found on the device, and
with the reference's rounding in the tensors' dtype (the cos/sin table of
:143-155 is built in that dtype).  Tokens outside
``[cu_seqlens[0], cu_seqlens[-1])`` are left as they are.

Optionally the same launch first RMS-normalises every q / k row with the
``q_norm`` / ``k_norm`` weights (:95-103, applied before the rotation at
:558-566); the chain is then evaluated in fp32 and rounded once.

The backward (``fna2_rope_bwd``) is the rotation by ``-angle`` of the
incoming gradients, plus, with a norm, the RMSNorm backward and the weight
gradients (summed in a fixed order).  There is no fallback: without the
library, or for tensors not on the GPU, the op raises.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Tuple

import torch

from . import _capi

_DTYPES = {torch.bfloat16: _capi.FNA2_BF16, torch.float16: _capi.FNA2_F16,
           torch.float32: _capi.FNA2_F32}


def _view(t: torch.Tensor) -> _capi.Tensor:
    return _capi.Tensor(t.data_ptr(), 0, t.stride(0), t.stride(1))


def _usable(t: torch.Tensor) -> torch.Tensor:
    """A [T, H, D] view the kernel accepts: unit feature stride and 16-byte
    aligned rows (else a contiguous copy)."""
    es = t.element_size()
    ok = (t.stride(2) == 1 and t.data_ptr() % 16 == 0
          and (t.stride(0) * es) % 16 == 0 and (t.stride(1) * es) % 16 == 0)
    return t if ok else t.contiguous()


def _f32(w: Optional[torch.Tensor], device) -> Optional[torch.Tensor]:
    return None if w is None else w.detach().to(device=device, dtype=torch.float32).contiguous()


def _args(q, k, cu, inv, sign, wq, wk, eps) -> _capi.RopeArgs:
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise AssertionError("rope_varlen: q [T, H, D] and k [T, H_KV, D] expected")
    if q.dtype != k.dtype or q.dtype not in _DTYPES:
        raise AssertionError("rope_varlen: q and k must share a bf16/fp16/fp32 dtype")
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("rope_varlen runs on the gfx950 HIP kernel: tensors must be on the GPU")
    T, H, D = q.shape
    if inv.numel() != D // 2:
        raise AssertionError("rope_varlen: inv_freq must hold head_dim / 2 frequencies")
    for w in (wq, wk):
        if w is not None and w.numel() != D:
            raise AssertionError("rope_varlen: norm weights must hold head_dim values")
    a = _capi.RopeArgs()
    a.dtype = _DTYPES[q.dtype]
    a.total_tokens, a.heads_q, a.heads_k, a.head_dim = T, H, k.shape[1], D
    a.nseq = cu.numel() - 1
    a.sign = int(sign)
    a.cu_seqlens, a.inv_freq = cu.data_ptr(), inv.data_ptr()
    a.q, a.k = _view(q), _view(k)
    a.norm_q = None if wq is None else wq.data_ptr()
    a.norm_k = None if wk is None else wk.data_ptr()
    a.norm_eps = float(eps)
    return a


def _stream(dev) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def rope_varlen_raw(q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor,
                    inv_freq: torch.Tensor, sign: int = 1,
                    norm_q: Optional[torch.Tensor] = None, norm_k: Optional[torch.Tensor] = None,
                    eps: float = 1e-6) -> Tuple[torch.Tensor, torch.Tensor]:
    """(Optionally RMS-normalise, then) rotate q ``[T, H, D]`` and k
    ``[T, H_KV, D]`` (no autograd); new tensors."""
    q, k = _usable(q), _usable(k)
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    wq, wk = _f32(norm_q, q.device), _f32(norm_k, q.device)
    a = _args(q, k, cu, inv, sign, wq, wk, eps)
    q_out = torch.empty_like(q, memory_format=torch.contiguous_format)
    k_out = torch.empty_like(k, memory_format=torch.contiguous_format)
    a.q_out, a.k_out = _view(q_out), _view(k_out)
    with torch.cuda.device(q.device):
        _capi.raise_for(_capi.lib().fna2_rope_varlen(ctypes.byref(a), _stream(q.device)),
                        "fna2_rope_varlen")
    return q_out, k_out


def rope_varlen_bwd(dq_out, dk_out, q, k, cu_seqlens, inv_freq, sign=1, norm_q=None,
                    norm_k=None, eps=1e-6, dq=None, dk=None):
    """Gradients (dq, dk, dnorm_q, dnorm_k) of ``rope_varlen_raw`` for the
    gradients of its outputs (q, k: its inputs, needed with a norm).  dq, dk:
    tensors of q's and k's shapes to write into (any row strides, unit last
    stride), else new ones."""
    q, k = _usable(q), _usable(k)
    dq_out, dk_out = _usable(dq_out.to(q.dtype)), _usable(dk_out.to(k.dtype))
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    wq, wk = _f32(norm_q, q.device), _f32(norm_k, q.device)
    b = _capi.RopeBwdArgs()
    b.fwd = _args(q, k, cu, inv, sign, wq, wk, eps)
    if dq is None:
        dq = torch.empty_like(q, memory_format=torch.contiguous_format)
    if dk is None:
        dk = torch.empty_like(k, memory_format=torch.contiguous_format)
    b.dq_out, b.dk_out, b.dq, b.dk = _view(dq_out), _view(dk_out), _view(dq), _view(dk)
    dwq = None if wq is None else torch.empty_like(wq)
    dwk = None if wk is None else torch.empty_like(wk)
    b.dnorm_q = None if dwq is None else dwq.data_ptr()
    b.dnorm_k = None if dwk is None else dwk.data_ptr()
    lib = _capi.lib()
    nbytes = lib.fna2_rope_bwd_workspace_bytes(ctypes.byref(b.fwd))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=q.device)
    b.workspace, b.workspace_bytes = ws.data_ptr(), nbytes
    with torch.cuda.device(q.device):
        _capi.raise_for(lib.fna2_rope_bwd(ctypes.byref(b), _stream(q.device)), "fna2_rope_bwd")
    return dq, dk, dwq, dwk


class RopeVarlenFunc(torch.autograd.Function):
    """y = R(angle) RMSNorm(x) (norm optional) on q and k."""

    @staticmethod
    def forward(ctx, q, k, cu_seqlens, inv_freq, norm_q, norm_k, eps, grad_slab=None):
        ctx.eps = eps
        ctx.grad_slab = grad_slab  # dq, dk into its blocks 0 and 1 (attention_fna2.py)
        ctx.norm = norm_q is not None or norm_k is not None
        ctx.save_for_backward(q if ctx.norm else None, k if ctx.norm else None,
                              cu_seqlens, inv_freq, norm_q, norm_k)
        ctx.shapes = (q.shape, k.shape)
        # the layouts the gradients take in a GradSlab (as q's and k's)
        ctx.layouts = ((q.shape, q.stride()), (k.shape, k.stride()))
        return rope_varlen_raw(q, k, cu_seqlens, inv_freq, 1, norm_q, norm_k, eps)

    @staticmethod
    def backward(ctx, dq, dk):
        # (autograd materialises the gradient of an unused output as zeros)
        q, k, cu, inv, wq, wk = ctx.saved_tensors
        if not ctx.norm:  # the inverse rotation reads no inputs: any same-shaped tensors do
            q, k = dq, dk
        slab = ctx.grad_slab
        oq = None if slab is None else slab.block(0, ctx.layouts[0])
        ok = None if slab is None else slab.block(1, ctx.layouts[1])
        gq, gk, gwq, gwk = rope_varlen_bwd(dq, dk, q, k, cu, inv, 1, wq, wk, ctx.eps, oq, ok)
        if gwq is not None and wq is not None:
            gwq = gwq.to(wq.dtype)
        if gwk is not None and wk is not None:
            gwk = gwk.to(wk.dtype)
        return gq, gk, None, None, gwq, gwk, None, None


def rope_varlen(q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor,
                inv_freq: torch.Tensor, norm_q: Optional[torch.Tensor] = None,
                norm_k: Optional[torch.Tensor] = None, eps: float = 1e-6, grad_slab=None
                ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Varlen RoPE of q ``[T, H, D]`` and k ``[T, H_KV, D]``, optionally
    after the QK RMSNorm with weights ``norm_q`` / ``norm_k`` (differentiable
    in q, k and the weights).  grad_slab: see attention_fna2.GradSlab."""
    return RopeVarlenFunc.apply(q, k, cu_seqlens, inv_freq, norm_q, norm_k, eps, grad_slab)
