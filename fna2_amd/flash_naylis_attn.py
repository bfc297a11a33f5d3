"""FlashNaylisAttention-2 on MI355X: the drop-in for ``FNA2/flash_naylis_attn.py``.

Same public surface as the reference module (myAiByMe/FNA2,
``FNA2/flash_naylis_attn.py``):

* ``BLOCK_M``, ``BLOCK_N``, ``BLOCK_R`` (:49-51) — ``BLOCK_R`` still names the
  default rank that ``NaylisAttention`` checks (attention_fna2.py:225);
* the launchers ``_fna2_forward`` (:700), ``_fna2_forward_varlen`` (:756),
  ``_fna2_backward`` (:807), ``_fna2_backward_varlen`` (:1215);
* ``FlashNaylisAttnFunc`` (:1307, 12 inputs, 12 gradients);
* ``flash_naylis_attn`` (:1380).

The launchers call hand-written gfx950 HIP kernels through the C ABI of
``include/fna2.h`` (``libfna2_hip.so``, bound with ctypes in ``_capi.py``).
There is no Triton and no fallback path: without the library every call
raises.

Differences from the reference, all supersets:

* rank ``R`` may be any multiple of 8 in [8, 64] (the reference requires
  ``R == BLOCK_R == 32``, :719, :778, :1423-1427);
* varlen honours ``is_causal`` (the reference's varlen kernels are always
  causal, :300, :322) — ``_fna2_forward_varlen`` / ``_fna2_backward_varlen``
  take it as an extra trailing keyword that defaults to ``True``;
* ``S_q != S_k`` in dense mode and ``cu_seqlens_q != cu_seqlens_k`` in varlen
  mode (top-left causal alignment, as the reference's masks);
* ``r_q=None`` runs plain attention (no graph heads);
* gradients are exact sums (the reference accumulates dK/dV/dR_k with bf16
  atomics, :546-553) and bitwise reproducible.

Tensors need a unit innermost stride and 16-byte aligned rows; other layouts
are copied with ``.contiguous()`` first.  q, k and v are bfloat16 or float16
(one dtype; out and dq / dk / dv take it), r_q and r_k bfloat16, as in the
reference.
"""
from __future__ import annotations

import collections
import contextlib
import ctypes
import math
from typing import Optional

import torch

from . import _capi

BLOCK_M = 128  # query rows per forward workgroup
BLOCK_N = 64   # keys per forward step
BLOCK_R = 32   # default rel_rank (NaylisAttention's default)

SUPPORTED_HEAD_DIMS = (64, 128)
SUPPORTED_DTYPES = (torch.bfloat16, torch.float16)  # q, k, v (r_q / r_k: bfloat16)
SUPPORTED_RANKS = tuple(range(8, 65, 8))


def rank_supported(r: int) -> bool:
    return r in SUPPORTED_RANKS


# ─────────────────────────────────────────────────────────────────────────────
# tensor views for the C ABI
# ─────────────────────────────────────────────────────────────────────────────

def _aligned(t: torch.Tensor, vec: bool) -> bool:
    if t.stride(-1) != 1 and t.shape[-1] > 1:
        return False
    es = t.element_size()
    unit = 16 // es if vec else 1
    if vec and t.data_ptr() % 16:
        return False
    return all(s % unit == 0 for s in t.stride()[:-1])


def _prep(t: Optional[torch.Tensor], vec: bool = True) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if t.numel() == 0:
        return t
    if not _aligned(t, vec):
        t = t.contiguous()
    return t


def _view4(t: Optional[torch.Tensor]) -> _capi.Tensor:
    """Dense [B, H, S, F] (or fp32 [B, H, S])."""
    if t is None or t.numel() == 0:
        return _capi.empty_tensor()
    return _capi.Tensor(t.data_ptr(), t.stride(0), t.stride(2), t.stride(1))


def _view3(t: Optional[torch.Tensor]) -> _capi.Tensor:
    """Varlen [T, H, F] (or fp32 [T, H])."""
    if t is None or t.numel() == 0:
        return _capi.empty_tensor()
    return _capi.Tensor(t.data_ptr(), 0, t.stride(0), t.stride(1))


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None or t.numel() == 0 else t.data_ptr()


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _check_inputs(q, k, v, r_q, r_k, graph_scale):
    # q, k, v: bf16 or fp16, one dtype (the reference's kernels are generic
    # over it, FNA2/flash_naylis_attn.py:187, :201, :522-529); r_q, r_k: bf16
    # (:1419-1420).
    assert q.dtype in SUPPORTED_DTYPES, f"q must be bfloat16 or float16 (got {q.dtype})"
    for name, t in (("q", q), ("k", k), ("v", v)):
        assert t.dtype == q.dtype, f"{name} must have q's dtype {q.dtype} (got {t.dtype})"
        assert t.is_cuda, f"{name} must be a GPU tensor"
    if r_q is not None:
        assert r_k is not None, "r_q and r_k must both be given"
        assert r_q.dtype == torch.bfloat16 and r_k.dtype == torch.bfloat16, \
            "r_q and r_k must be bfloat16"
        assert graph_scale is not None, "graph_scale is required with r_q / r_k"
    dev = q.device
    for t in (k, v, r_q, r_k, graph_scale):
        if t is not None:
            assert t.device == dev, "all tensors must be on the same device"


def _gs32(graph_scale: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    if graph_scale is None:
        return None
    return graph_scale.detach().to(torch.float32).contiguous()


def _problem(varlen, batch, sq, sk, tq, tk, H, H_KV, H_G, D, R, causal, scale, cu_q=None,
             cu_k=None, dtype=torch.bfloat16) -> _capi.Problem:
    code = _capi.FNA2_F16 if dtype == torch.float16 else _capi.FNA2_BF16
    return _capi.Problem(code, int(varlen), int(batch), int(sq), int(sk), int(tq),
                         int(tk), int(H), int(H_KV), int(H_G), int(D), int(R), int(bool(causal)),
                         float(scale), _ptr(cu_q), _ptr(cu_k))


class KernelTimer:
    """Per-kernel HIP event pairs, recorded by the library around its kernels.

    Used by ``bench.py`` through :func:`kernel_timing`.  Events come from a
    pool created (and materialised by one record) before the timed region, so
    timing adds only the event records themselves to the stream.
    """

    FWD = ("fwd",)
    BWD = ("dq", "dkdv")

    def __init__(self, n_fwd: int, n_bwd: int):
        n = 2 * (n_fwd * len(self.FWD) + n_bwd * len(self.BWD))
        self._pool = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
        for ev in self._pool:
            ev.record()
        torch.cuda.synchronize()
        self._next = 0
        self.records = []  # (kernel name, start event, end event)

    def take(self, names) -> ctypes.Array:
        evs = []
        for name in names:
            if self._next + 2 > len(self._pool):
                raise RuntimeError("KernelTimer pool exhausted")
            s, e = self._pool[self._next], self._pool[self._next + 1]
            self._next += 2
            self.records.append((name, s, e))
            evs += [s, e]
        return (ctypes.c_void_p * len(evs))(*[ev.cuda_event for ev in evs])

    def durations_ms(self) -> dict:
        torch.cuda.synchronize()
        out: dict = {}
        for name, s, e in self.records:
            out.setdefault(name, []).append(s.elapsed_time(e))
        return out


_timer: Optional[KernelTimer] = None


@contextlib.contextmanager
def kernel_timing(timer: KernelTimer):
    """Within the block, every launcher call records its kernels on ``timer``."""
    global _timer
    prev, _timer = _timer, timer
    try:
        yield timer
    finally:
        _timer = prev


def _events(names):
    if _timer is None:
        return None
    return _timer.take(names)


def _workspace(fn, prob: _capi.Problem, dev) -> torch.Tensor:
    nbytes = int(fn(ctypes.byref(prob)))
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device=dev)


def new_plan(prob: _capi.Problem, device) -> Optional[torch.Tensor]:
    """A plan buffer for a varlen problem (None in dense mode): the forward
    builds the backward's tile lists into it, and the backward given it
    launches no list builder."""
    n = int(_capi.lib().fna2_plan_bytes(ctypes.byref(prob)))
    return torch.empty(n, dtype=torch.uint8, device=device) if n > 0 else None


def _run_fwd(prob, q, k, v, r_q, r_k, gs, out, lse, view, plan=None, plan_filled=False):
    L = _capi.lib()
    ws = _workspace(L.fna2_fwd_workspace_bytes, prob, q.device)
    ev = _events(KernelTimer.FWD)
    args = _capi.FwdArgs(prob, view(q), view(k), view(v), view(r_q), view(r_k), _ptr(gs),
                         view(out), view(lse), ws.data_ptr(), ws.numel(),
                         ctypes.cast(ev, ctypes.c_void_p) if ev is not None else None)
    if plan is not None:
        args.plan, args.plan_bytes = plan.data_ptr(), plan.numel()
        args.plan_filled = int(bool(plan_filled))
    with torch.cuda.device(q.device):
        st = L.fna2_fwd(ctypes.byref(args), _stream(q.device))
    _capi.raise_for(st, "fna2_fwd")


def _run_bwd(prob, tensors, view, plan=None):
    (dout, q, k, v, r_q, r_k, gs, out, lse, delta, dq, dk, dv, dr_q, dr_k, d_gs) = tensors
    L = _capi.lib()
    ws = _workspace(L.fna2_bwd_workspace_bytes, prob, q.device)
    ev = _events(KernelTimer.BWD)
    args = _capi.BwdArgs(prob, view(q), view(k), view(v), view(r_q), view(r_k), _ptr(gs),
                         view(out), view(lse), view(dout), view(delta), view(dq), view(dk),
                         view(dv), view(dr_q), view(dr_k), _ptr(d_gs), ws.data_ptr(), ws.numel(),
                         ctypes.cast(ev, ctypes.c_void_p) if ev is not None else None)
    if plan is not None:
        args.plan, args.plan_bytes = plan.data_ptr(), plan.numel()
    with torch.cuda.device(q.device):
        st = L.fna2_bwd(ctypes.byref(args), _stream(q.device))
    _capi.raise_for(st, "fna2_bwd")


# ─────────────────────────────────────────────────────────────────────────────
# launchers (same names and signatures as the reference)
# ─────────────────────────────────────────────────────────────────────────────

def _fna2_forward(
    q: torch.Tensor,            # [B, H, S, D]
    k: torch.Tensor,            # [B, H_KV, S_k, D]
    v: torch.Tensor,            # [B, H_KV, S_k, D]
    r_q: Optional[torch.Tensor],  # [B, H_G, S, R]
    r_k: Optional[torch.Tensor],  # [B, H_G, S_k, R]
    graph_scale: Optional[torch.Tensor],  # [H_G]
    softmax_scale: float,
    is_causal: bool,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Dense forward; returns (out, lse).  Mirrors FNA2/flash_naylis_attn.py:700-753."""
    B, H, S, D = q.shape
    H_KV, S_k = k.shape[1], k.shape[2]
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[3]
    if r_q is not None:
        assert H_G == r_k.shape[1], "r_q and r_k must have the same number of graph heads"
        assert H_G == 0 or rank_supported(R), \
            f"rel_rank must be a multiple of 8 in [8, 64] (got {R})"
    assert D in SUPPORTED_HEAD_DIMS, f"head_dim must be 64 or 128 (got {D})"
    assert H % H_KV == 0, f"num heads {H} must be a multiple of KV heads {H_KV}"
    _check_inputs(q, k, v, r_q, r_k, graph_scale)
    q, k, v, r_q, r_k = (_prep(t) for t in (q, k, v, r_q, r_k))
    gs = _gs32(graph_scale) if H_G else None
    out = torch.empty_like(q)
    lse = torch.empty(B, H, S, device=q.device, dtype=torch.float32)
    prob = _problem(False, B, S, S_k, 0, 0, H, H_KV, H_G, D, R, is_causal, softmax_scale,
                    dtype=q.dtype)
    _run_fwd(prob, q, k, v, r_q if H_G else None, r_k if H_G else None, gs, out, lse, _view4)
    return out, lse


def _fna2_forward_varlen(
    q: torch.Tensor,            # [T, H, D]
    k: torch.Tensor,            # [T_k, H_KV, D]
    v: torch.Tensor,            # [T_k, H_KV, D]
    r_q: Optional[torch.Tensor],  # [T, H_G, R]
    r_k: Optional[torch.Tensor],  # [T_k, H_G, R]
    graph_scale: Optional[torch.Tensor],  # [H_G]
    cu_seqlens_q: torch.Tensor,  # [N + 1] int32
    cu_seqlens_k: torch.Tensor,  # [N + 1] int32
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    is_causal: bool = True,
    plan: Optional[torch.Tensor] = None,
    lse_head_major: bool = False,
    plan_filled: bool = False,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Varlen forward; returns (out [T,H,D], lse [T,H]).  Mirrors :756-804.
    ``plan`` (from ``new_plan``, optional): also build the backward's tile
    lists into it, for an ``_fna2_backward_varlen`` given the same plan.

    ``lse`` is a contiguous ``[T, H]`` tensor, as the reference allocates it
    (:780).  ``lse_head_major=True`` (the autograd and custom-operator paths)
    returns the same values as a ``[T, H]`` view of head-major ``[H, T]``
    memory instead: a forward workgroup's 128 rows of one head are then one
    contiguous run (row-major ``[T, H]`` puts each 4-byte value in its own
    64-byte segment: 75.9 MB written per c3 forward against 68.2).
    ``plan_filled``: an earlier forward of this problem filled ``plan`` for
    these cu_seqlens, unchanged since: its lists are reused (no list-building
    launch)."""
    total_q, H, D = q.shape
    total_k, H_KV = k.shape[0], k.shape[1]
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[2]
    N = cu_seqlens_q.shape[0] - 1
    if r_q is not None:
        assert H_G == r_k.shape[1], "r_q and r_k must have the same number of graph heads"
        assert H_G == 0 or rank_supported(R), \
            f"rel_rank must be a multiple of 8 in [8, 64] (got {R})"
    assert D in SUPPORTED_HEAD_DIMS, f"head_dim must be 64 or 128 (got {D})"
    assert H % H_KV == 0, f"num heads {H} must be a multiple of KV heads {H_KV}"
    assert cu_seqlens_k.shape[0] == N + 1, "cu_seqlens_q and cu_seqlens_k differ in length"
    _check_inputs(q, k, v, r_q, r_k, graph_scale)
    q, k, v, r_q, r_k = (_prep(t) for t in (q, k, v, r_q, r_k))
    cu_q = cu_seqlens_q.to(device=q.device, dtype=torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(device=q.device, dtype=torch.int32).contiguous()
    gs = _gs32(graph_scale) if H_G else None
    out = torch.empty_like(q)
    if lse_head_major:
        lse = torch.empty(H, total_q, device=q.device, dtype=torch.float32).t()
    else:
        lse = torch.empty(total_q, H, device=q.device, dtype=torch.float32)
    prob = _problem(True, N, max_seqlen_q, max_seqlen_k, total_q, total_k, H, H_KV, H_G, D, R,
                    is_causal, softmax_scale, cu_q, cu_k, dtype=q.dtype)
    _run_fwd(prob, q, k, v, r_q if H_G else None, r_k if H_G else None, gs, out, lse, _view3,
             plan, plan_filled)
    return out, lse


def _grads_like(q, k, v, r_q, r_k, H_G):
    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    dr_q = torch.empty_like(r_q) if H_G else None
    dr_k = torch.empty_like(r_k) if H_G else None
    return dq, dk, dv, dr_q, dr_k


def _fna2_backward(
    dout: torch.Tensor,
    q, k, v, r_q, r_k, graph_scale,
    out, lse,
    softmax_scale: float,
    is_causal: bool,
    grads_out: Optional[tuple] = None,
) -> tuple:
    """Dense backward; returns (dq, dk, dv, dr_q, dr_k, d_gs).  Mirrors :807-892.
    ``grads_out``: as for ``_fna2_backward_varlen``."""
    B, H, S, D = q.shape
    H_KV, S_k = k.shape[1], k.shape[2]
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[3]
    dout = _prep(dout if dout.dtype == q.dtype else dout.to(q.dtype))  # as do.to(v.dtype), :522
    q, k, v, r_q, r_k, out = (_prep(t) for t in (q, k, v, r_q, r_k, out))
    gs = _gs32(graph_scale) if H_G else None
    lse = lse.contiguous()
    delta = torch.empty(B, H, S, device=q.device, dtype=torch.float32)
    grads = _grads_like(q, k, v, r_q, r_k, H_G)
    if grads_out is not None:
        grads = tuple(g if o is None else o for g, o in zip(grads, grads_out))
    dq, dk, dv, dr_q, dr_k = grads
    d_gs = torch.empty(max(H_G, 1), device=q.device, dtype=torch.float32)
    prob = _problem(False, B, S, S_k, 0, 0, H, H_KV, H_G, D, R, is_causal, softmax_scale,
                    dtype=q.dtype)
    _run_bwd(prob, (dout, q, k, v, r_q if H_G else None, r_k if H_G else None, gs, out, lse,
                    delta, dq, dk, dv, dr_q, dr_k, d_gs if H_G else None), _view4)
    return dq, dk, dv, dr_q, dr_k, _dgs_out(d_gs, H_G, graph_scale)


def _fna2_backward_varlen(
    dout: torch.Tensor,
    q, k, v, r_q, r_k, graph_scale,
    out, lse,
    cu_seqlens_q: torch.Tensor,
    cu_seqlens_k: torch.Tensor,
    max_seqlen_q: int,
    max_seqlen_k: int,
    softmax_scale: float,
    is_causal: bool = True,
    plan: Optional[torch.Tensor] = None,
    grads_out: Optional[tuple] = None,
) -> tuple:
    """Varlen backward; returns (dq, dk, dv, dr_q, dr_k, d_gs).  Mirrors :1215-1300.
    ``plan``: the one the forward of the same problem filled (optional).
    ``grads_out``: (dq, dk, dv, dr_q, dr_k) tensors to write the gradients
    into, None entries allocated here (any row strides, unit last stride)."""
    total_q, H, D = q.shape
    total_k, H_KV = k.shape[0], k.shape[1]
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[2]
    N = cu_seqlens_q.shape[0] - 1
    dout = _prep(dout if dout.dtype == q.dtype else dout.to(q.dtype))  # as do.to(v.dtype), :522
    q, k, v, r_q, r_k, out = (_prep(t) for t in (q, k, v, r_q, r_k, out))
    cu_q = cu_seqlens_q.to(device=q.device, dtype=torch.int32).contiguous()
    cu_k = cu_seqlens_k.to(device=q.device, dtype=torch.int32).contiguous()
    gs = _gs32(graph_scale) if H_G else None
    # (lse is read through its strides: the forward's head-major view or a
    # row-major [T, H] alike)
    # [T, H] view of head-major memory: the dK/dV kernel reads a head's rows
    delta = torch.empty(H, total_q, device=q.device, dtype=torch.float32).t()
    grads = _grads_like(q, k, v, r_q, r_k, H_G)
    if grads_out is not None:
        grads = tuple(g if o is None else o for g, o in zip(grads, grads_out))
    dq, dk, dv, dr_q, dr_k = grads
    d_gs = torch.empty(max(H_G, 1), device=q.device, dtype=torch.float32)
    prob = _problem(True, N, max_seqlen_q, max_seqlen_k, total_q, total_k, H, H_KV, H_G, D, R,
                    is_causal, softmax_scale, cu_q, cu_k, dtype=q.dtype)
    _run_bwd(prob, (dout, q, k, v, r_q if H_G else None, r_k if H_G else None, gs, out, lse,
                    delta, dq, dk, dv, dr_q, dr_k, d_gs if H_G else None), _view3, plan)
    return dq, dk, dv, dr_q, dr_k, _dgs_out(d_gs, H_G, graph_scale)


def _plan_for(q, k, r_q, cu_q, cu_k, max_q, max_k, is_causal, scale):
    """The plan buffer of a varlen call (its size depends on the shapes only)."""
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[2]
    prob = _problem(True, cu_q.shape[0] - 1, max_q, max_k, q.shape[0], k.shape[0], q.shape[1],
                    k.shape[1], H_G, q.shape[2], R, is_causal, scale, cu_q, cu_k, dtype=q.dtype)
    return new_plan(prob, q.device)


# Plans of recent varlen forwards, by the cu_seqlens tensors they were built
# for.  The tile lists depend only on the sequence extents and the problem's
# shape, so a forward handed the very same cu_seqlens tensors (the layers of
# one model step share them), unchanged since (torch bumps a tensor's version
# counter on every in-place write), reuses the plan and launches no builder.
# The entries hold the cu_seqlens tensors, so their memory cannot be reused by
# other tensors while the entry lives.
_PLANS: "collections.OrderedDict" = collections.OrderedDict()
_PLANS_MAX = 8


def _plan_reused(q, k, r_q, cu_q, cu_k, max_q, max_k, is_causal, scale):
    """(plan, filled): the plan buffer of a varlen forward, and whether an
    earlier forward filled it for these cu_seqlens tensors (same objects and
    version counters, same device, stream and problem shape)."""
    direct = all(t.dtype == torch.int32 and t.is_contiguous() and t.device == q.device
                 for t in (cu_q, cu_k))
    if not direct:  # the launcher converts them: a new tensor every call
        return _plan_for(q, k, r_q, cu_q, cu_k, max_q, max_k, is_causal, scale), False
    H_G = 0 if r_q is None else r_q.shape[1]
    R = 0 if r_q is None else r_q.shape[2]
    key = (q.device, _stream(q.device), id(cu_q), cu_q._version, id(cu_k), cu_k._version,
           cu_q.shape[0], q.shape[0], k.shape[0], q.shape[1], k.shape[1], H_G, q.shape[2], R,
           bool(is_causal))
    hit = _PLANS.get(key)
    if hit is not None and hit[0] is cu_q and hit[1] is cu_k:
        _PLANS.move_to_end(key)
        return hit[2], True
    plan = _plan_for(q, k, r_q, cu_q, cu_k, max_q, max_k, is_causal, scale)
    if plan is not None:
        _PLANS[key] = (cu_q, cu_k, plan)
        while len(_PLANS) > _PLANS_MAX:
            _PLANS.popitem(last=False)
    return plan, False


def _dgs_out(d_gs, H_G, graph_scale):
    if not H_G or graph_scale is None:
        return None
    return d_gs[:H_G].to(graph_scale.dtype)


# ─────────────────────────────────────────────────────────────────────────────
# autograd
# ─────────────────────────────────────────────────────────────────────────────

class FlashNaylisAttnFunc(torch.autograd.Function):
    """autograd wrapper, same contract as FNA2/flash_naylis_attn.py:1307-1373."""

    @staticmethod
    def forward(
        ctx,
        q, k, v, r_q, r_k, graph_scale,
        softmax_scale: float,
        is_causal: bool,
        cu_seqlens_q=None,
        cu_seqlens_k=None,
        max_seqlen_q: int = 0,
        max_seqlen_k: int = 0,
        grad_slab=None,
    ):
        use_varlen = cu_seqlens_q is not None
        if use_varlen:
            if cu_seqlens_k is None:
                cu_seqlens_k = cu_seqlens_q
            # The forward's list-building launch also builds the backward's
            # lists (kept on ctx): the backward then launches no builder; and
            # a forward given the same cu_seqlens tensors again (the next
            # layer) reuses them and launches none either.
            plan, filled = _plan_reused(q, k, r_q, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                        max_seqlen_k, is_causal, softmax_scale)
            out, lse = _fna2_forward_varlen(
                q, k, v, r_q, r_k, graph_scale,
                cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                softmax_scale, is_causal, plan=plan, lse_head_major=True, plan_filled=filled,
            )
            ctx.plan = plan
        else:
            out, lse = _fna2_forward(q, k, v, r_q, r_k, graph_scale, softmax_scale, is_causal)
        ctx.save_for_backward(q, k, v, r_q, r_k, graph_scale, out, lse)
        ctx.softmax_scale = softmax_scale
        ctx.is_causal = is_causal
        ctx.use_varlen = use_varlen
        ctx.cu_seqlens_q = cu_seqlens_q
        ctx.cu_seqlens_k = cu_seqlens_k
        ctx.max_seqlen_q = max_seqlen_q
        ctx.max_seqlen_k = max_seqlen_k
        # where the caller wants dv, dr_q and dr_k written: blocks 2, 3, 4 of
        # a GradSlab (attention_fna2.py); None: new tensors
        ctx.grad_slab = grad_slab
        return out

    @staticmethod
    def backward(ctx, dout):
        q, k, v, r_q, r_k, graph_scale, out, lse = ctx.saved_tensors
        slab = ctx.grad_slab
        outs = None
        if slab is not None:
            outs = (None, None, slab.block(2, v),
                    None if r_q is None else slab.block(3, r_q),
                    None if r_k is None else slab.block(4, r_k))
        if ctx.use_varlen:
            grads = _fna2_backward_varlen(
                dout, q, k, v, r_q, r_k, graph_scale, out, lse,
                ctx.cu_seqlens_q, ctx.cu_seqlens_k, ctx.max_seqlen_q, ctx.max_seqlen_k,
                ctx.softmax_scale, ctx.is_causal, plan=ctx.plan, grads_out=outs,
            )
        else:
            grads = _fna2_backward(
                dout, q, k, v, r_q, r_k, graph_scale, out, lse,
                ctx.softmax_scale, ctx.is_causal, grads_out=outs,
            )
        dq, dk, dv, dr_q, dr_k, d_gs = grads
        return dq, dk, dv, dr_q, dr_k, d_gs, None, None, None, None, None, None, None


# ─────────────────────────────────────────────────────────────────────────────
# public API
# ─────────────────────────────────────────────────────────────────────────────

def _plain_eager(q: torch.Tensor) -> bool:
    """Whether a call runs eagerly on plain tensors: no compiler, tracer or
    tensor mode (make_fx, fake tensors, functionalization) in effect, which
    need the custom operator."""
    from torch.utils._python_dispatch import _get_current_dispatch_mode
    if torch.compiler.is_compiling() or torch.jit.is_tracing():
        return False
    if _get_current_dispatch_mode() is not None:
        return False
    return type(q) in (torch.Tensor, torch.nn.Parameter)


def flash_naylis_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    r_q: Optional[torch.Tensor],
    r_k: Optional[torch.Tensor],
    graph_scale: Optional[torch.Tensor],
    softmax_scale: Optional[float] = None,
    is_causal: bool = True,
    cu_seqlens_q: Optional[torch.Tensor] = None,
    cu_seqlens_k: Optional[torch.Tensor] = None,
    max_seqlen_q: int = 0,
    max_seqlen_k: int = 0,
) -> torch.Tensor:
    """FlashNaylisAttention-2 (FNA2/flash_naylis_attn.py:1380-1434).

    q, k, v       dense [B, H, S, D] / [B, H_KV, S_k, D] (any strides with a
                  unit last stride) or varlen [T, H, D] / [T_k, H_KV, D]
    r_q, r_k      dense [B, H_G, S, R] or varlen [T, H_G, R], bfloat16; heads
                  [0, H_G) get the bias graph_scale[h] * R_q R_k^T
    graph_scale   [H_G]
    softmax_scale 1/sqrt(D) if None
    is_causal     top-left causal mask on local positions
    cu_seqlens_*  varlen offsets (int32); max_seqlen_* are scheduling hints

    Returns the attention output with q's shape, dtype and strides.

    Under ``torch.compile`` (or any tracer or tensor mode) the call is the
    custom operator ``fna2::fwd`` (differentiated by ``fna2::bwd``,
    ``fna2_amd/ops.py``), which they trace.  Run eagerly on plain tensors it
    is ``FlashNaylisAttnFunc.apply``, a plain ``autograd.Function`` as the
    reference uses, on the same launchers: the same results, without the
    custom-operator dispatch (~85 us of host time per forward + backward, a
    quarter of a c3 step's GPU time).
    """
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(q.shape[-1])
    if r_q is not None:
        assert r_q.dtype == torch.bfloat16, "r_q must be bfloat16"
        assert r_k is not None and r_k.dtype == torch.bfloat16, "r_k must be bfloat16"
        R = r_q.shape[-1]
        assert rank_supported(R), f"rel_rank must be a multiple of 8 in [8, 64] (got {R})"
    if not _plain_eager(q):
        out, _, _ = torch.ops.fna2.fwd(
            q, k, v, r_q, r_k, graph_scale,
            float(softmax_scale), bool(is_causal),
            cu_seqlens_q, cu_seqlens_k,
            int(max_seqlen_q), int(max_seqlen_k),
        )
        return out
    return FlashNaylisAttnFunc.apply(q, k, v, r_q, r_k, graph_scale, float(softmax_scale),
                                     bool(is_causal), cu_seqlens_q, cu_seqlens_k,
                                     int(max_seqlen_q), int(max_seqlen_k))
