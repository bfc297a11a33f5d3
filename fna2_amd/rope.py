"""Varlen rotary position embedding on the gfx950 HIP kernel.

Replaces the reference's ``NaylisAttention._apply_rope_varlen``
(FNA2/attention_fna2.py:620-647), which walks the packed sequences on the
host (``cu_seqlens.tolist()``: a device synchronisation per call) and
applies ``RotaryPositionalEmbedding.forward`` (:163-170) to each.  Here one
launch (``fna2_rope_varlen`` in ``include/fna2.h``) rotates every token of q
and k, with the position ``t - cu_seqlens[seq(t)]`` found on the device, and
with the reference's rounding in the tensors' dtype (the cos/sin table of
:143-155 is built in that dtype).  Tokens outside
``[cu_seqlens[0], cu_seqlens[-1])`` are left as they are.

The backward is the rotation by ``-angle`` of the incoming gradients (the
same kernel, ``sign = -1``).  There is no fallback: without the library, or
for tensors not on the GPU, the op raises.
"""
from __future__ import annotations

import ctypes
from typing import Tuple

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


def rope_varlen_raw(q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor,
                    inv_freq: torch.Tensor, sign: int = 1
                    ) -> Tuple[torch.Tensor, torch.Tensor]:
    """Rotate q ``[T, H, D]`` and k ``[T, H_KV, D]`` (no autograd); new tensors."""
    if q.dim() != 3 or k.dim() != 3 or q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise AssertionError("rope_varlen: q [T, H, D] and k [T, H_KV, D] expected")
    if q.dtype != k.dtype or q.dtype not in _DTYPES:
        raise AssertionError("rope_varlen: q and k must share a bf16/fp16/fp32 dtype")
    if not (q.is_cuda and k.is_cuda):
        raise RuntimeError("rope_varlen runs on the gfx950 HIP kernel: tensors must be on the GPU")
    T, H, D = q.shape
    H_KV = k.shape[1]
    if inv_freq.numel() != D // 2:
        raise AssertionError("rope_varlen: inv_freq must hold head_dim / 2 frequencies")
    q, k = _usable(q), _usable(k)
    cu = cu_seqlens.to(device=q.device, dtype=torch.int32).contiguous()
    inv = inv_freq.to(device=q.device, dtype=torch.float32).contiguous()
    q_out = torch.empty_like(q, memory_format=torch.contiguous_format)
    k_out = torch.empty_like(k, memory_format=torch.contiguous_format)
    a = _capi.RopeArgs()
    a.dtype = _DTYPES[q.dtype]
    a.total_tokens, a.heads_q, a.heads_k, a.head_dim = T, H, H_KV, D
    a.nseq = cu.numel() - 1
    a.sign = int(sign)
    a.cu_seqlens, a.inv_freq = cu.data_ptr(), inv.data_ptr()
    a.q, a.k, a.q_out, a.k_out = _view(q), _view(k), _view(q_out), _view(k_out)
    stream = torch.cuda.current_stream(q.device).cuda_stream
    with torch.cuda.device(q.device):
        _capi.raise_for(_capi.lib().fna2_rope_varlen(ctypes.byref(a), ctypes.c_void_p(stream)),
                        "fna2_rope_varlen")
    return q_out, k_out


class RopeVarlenFunc(torch.autograd.Function):
    """y = R(angle) x on q and k; dx = R(-angle) dy."""

    @staticmethod
    def forward(ctx, q, k, cu_seqlens, inv_freq):
        ctx.save_for_backward(cu_seqlens, inv_freq)
        return rope_varlen_raw(q, k, cu_seqlens, inv_freq, 1)

    @staticmethod
    def backward(ctx, dq, dk):
        # (autograd materialises the gradient of an unused output as zeros)
        cu, inv = ctx.saved_tensors
        gq, gk = rope_varlen_raw(dq, dk, cu, inv, -1)
        return gq, gk, None, None


def rope_varlen(q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor,
                inv_freq: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Varlen RoPE of q ``[T, H, D]`` and k ``[T, H_KV, D]`` (differentiable)."""
    return RopeVarlenFunc.apply(q, k, cu_seqlens, inv_freq)
