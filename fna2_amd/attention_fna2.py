"""NaylisAttention on MI355X: the drop-in for ``FNA2/attention_fna2.py``.

The module keeps the reference's constructor and ``forward`` signatures
(attention_fna2.py:197-215, :380-390) and its backend choice
(:220-233, :430-519, :533-617):

* the FNA2 path -- dense (``x`` is ``[B, S, E]``) or varlen (``x`` is
  ``[T, E]`` with ``cu_seqlens_q/k``) -- runs ``flash_naylis_attn``, i.e. the
  gfx950 HIP kernels, with ``R_q``/``R_k`` of shape ``[B, H_G, S, R]`` /
  ``[T, H_G, R]`` and ``graph_scale`` in fp32;
* decoding one token against a KV cache runs the gfx950 decode kernel
  (``flash_naylis_decode``) where the reference runs SDPA over
  ``torch.cat(past_kv, new)`` (:412-429, :445-473): the same result, without
  the graph bias, as there.  ``decode_graph_bias=True`` (an extra keyword)
  keeps ``R_k`` in the cache, ``(k, v, r_k)``, and decodes with the bias, so
  that a decode step equals the last row of the full causal forward.
  ``past_kv`` may also be a ``StaticKVCache`` (preallocated, written in
  place: no per-step copy of the cache);
* the other paths the reference sends elsewhere keep going elsewhere:
  ``soft_cap`` and modules built with ``use_fna2=False`` use PyTorch's SDPA
  with a materialised bias, or the explicit softmax when a ``soft_cap`` or
  custom ``mask`` is given (attention_fna2.py:337-374, :493-516).

``_FNA2_AVAILABLE`` is true when the HIP library loads and the current device
is gfx950.  A module asks for FNA2 with ``use_fna2=None`` (auto) or ``True``;
as in the reference it is used when the rank is supported -- here any
multiple of 8 up to 64 rather than only ``BLOCK_R`` (:225-229).  The FNA2 op
itself never falls back: called without the library it raises.

Varlen RoPE restarts positions at every sequence, as the reference's
``_apply_rope_varlen`` (:620-647), in one launch of the HIP rotary kernel
(``fna2_amd.rope``) with the positions formed on the device (no per-call
host synchronisation).
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _capi
from .flash_naylis_attn import BLOCK_R, flash_naylis_attn, rank_supported
from .flash_naylis_attn import FlashNaylisAttnFunc as _FNA2Func
from .flash_naylis_attn import _plain_eager as _fna2_plain_eager
from .decode import decode_supported, flash_naylis_decode
from .rope import rope_varlen


def _detect_fna2() -> bool:
    if not torch.cuda.is_available():
        return False
    try:
        _capi.lib()
        arch = torch.cuda.get_device_properties(torch.cuda.current_device()).gcnArchName
    except (OSError, RuntimeError, AttributeError):
        return False
    return arch.split(":")[0] == "gfx950"


_FNA2_AVAILABLE = _detect_fna2()
_FNA2_BLOCK_R = BLOCK_R


def _attention(q, k, v, r_q, r_k, graph_scale, grad_slab=None, **kw):
    """flash_naylis_attn, or (varlen, run eagerly, with a GradSlab) its
    autograd function told to write dv, dR_q and dR_k into the slab."""
    if grad_slab is None:
        return flash_naylis_attn(q, k, v, r_q, r_k, graph_scale, **kw)
    return _FNA2Func.apply(q, k, v, r_q, r_k, graph_scale, float(kw["softmax_scale"]),
                           bool(kw["is_causal"]), kw.get("cu_seqlens_q"), kw.get("cu_seqlens_k"),
                           int(kw.get("max_seqlen_q", 0)), int(kw.get("max_seqlen_k", 0)),
                           grad_slab)


_flash_naylis_attn = _attention

# (k, v), or (k, v, r_k) for a module built with decode_graph_bias=True.
KVCache = Tuple[torch.Tensor, ...]


class StaticKVCache:
    """A preallocated KV cache, written in place (an alternative to the
    reference's tuple cache, which ``torch.cat`` grows by a full copy per
    step: attention_fna2.py:415-418).

    ``k``, ``v``: ``[B, H_KV, capacity, D]``; ``r_k``: ``[B, H_G, capacity,
    R]`` for modules built with ``decode_graph_bias=True``.  ``length`` rows
    are in use, the same for every sequence.  Pass it as ``past_kv``: the
    module appends the new rows and attends to the first ``length`` (the
    decode kernel reads them in place), and returns the same object."""

    def __init__(self, k: torch.Tensor, v: torch.Tensor, r_k: Optional[torch.Tensor] = None,
                 length: int = 0):
        assert k.shape == v.shape and k.dim() == 4, "k and v must be [B, H_KV, capacity, D]"
        assert r_k is None or (r_k.dim() == 4 and r_k.shape[:3] == (k.shape[0], r_k.shape[1],
                                                                     k.shape[2]))
        assert 0 <= length <= k.shape[2]
        self.k, self.v, self.r_k, self.length = k, v, r_k, int(length)

    @classmethod
    def empty(cls, batch: int, n_kv_heads: int, capacity: int, head_dim: int,
              graph_heads: int = 0, rank: int = 0, dtype=torch.bfloat16,
              device=None) -> "StaticKVCache":
        mk = lambda h, f: torch.zeros(batch, h, capacity, f, dtype=dtype, device=device)
        return cls(mk(n_kv_heads, head_dim), mk(n_kv_heads, head_dim),
                   mk(graph_heads, rank) if graph_heads > 0 else None)

    @property
    def capacity(self) -> int:
        return self.k.shape[2]

    def append(self, k: torch.Tensor, v: torch.Tensor, r_k: Optional[torch.Tensor] = None):
        """Write rows [length, length + S) from k, v ``[B, H_KV, S, D]`` (and
        r_k ``[B, H_G, S, R]``)."""
        s = k.shape[2]
        if self.length + s > self.capacity:
            raise ValueError(f"StaticKVCache full: {self.length} + {s} rows > capacity "
                             f"{self.capacity}")
        end = self.length + s
        self.k[:, :, self.length:end] = k
        self.v[:, :, self.length:end] = v
        if self.r_k is not None:
            if r_k is None:
                raise ValueError("this cache holds R_k: the module must keep it "
                                 "(decode_graph_bias=True)")
            self.r_k[:, :, self.length:end] = r_k
        self.length = end

    def view(self) -> KVCache:
        """The rows in use: (k, v) or (k, v, r_k), views into the buffers."""
        n = self.length
        out = (self.k[:, :, :n], self.v[:, :, :n])
        return out + ((self.r_k[:, :, :n],) if self.r_k is not None else ())


class RMSNorm(nn.Module):
    """y = x / sqrt(mean(x^2) + eps) * weight over the last dimension."""

    def __init__(self, dim: int, eps: float = 1e-6):
        super().__init__()
        self.eps = eps
        self.weight = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        inv = torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + self.eps)
        return x * inv * self.weight


class RotaryPositionalEmbedding(nn.Module):
    """Rotary embedding on the last dimension (two halves rotated), with the
    optional YaRN frequency stretch of attention_fna2.py:129-142."""

    def __init__(self, dim: int, max_seq_len: int = 2048, base: int = 10000,
                 use_yarn: bool = False, yarn_scale: float = 1.0,
                 yarn_original_max_len: int = 1024):
        super().__init__()
        self.dim = dim
        self.max_seq_len = max_seq_len
        self.base = base
        self.use_yarn = use_yarn
        self.yarn_scale = yarn_scale
        self.yarn_original_max_len = yarn_original_max_len
        half = torch.arange(0, dim, 2, dtype=torch.float32)
        inv_freq = 1.0 / (base ** (half / dim))  # as attention_fna2.py:121-122
        if use_yarn and yarn_scale != 1.0:
            # frequencies past the first max(dim/2, dim/4) even indices are
            # divided by a factor rising linearly from 1 to yarn_scale
            start = max(dim // 2, int(dim * 0.25))
            ramp = 1 + (yarn_scale - 1) * (half - start) / (dim - start)
            inv_freq = inv_freq / torch.where(half < start, torch.ones_like(half), ramp)
        self.register_buffer("inv_freq", inv_freq)
        self._cache_key = None
        self._cos = self._sin = None

    def _table(self, n: int, device, dtype):
        """cos / sin rows of positions 0 .. n-1 (at least): the table is
        built for the largest length asked so far (doubling), so a decode
        loop slices it instead of rebuilding it every step."""
        key = (device, dtype)
        if key != self._cache_key or self._cos.shape[0] < n:
            size = n if key != self._cache_key else max(n, 2 * self._cos.shape[0])
            ang = torch.outer(torch.arange(size, device=device, dtype=dtype),
                              self.inv_freq.to(device=device, dtype=dtype))
            ang = torch.cat((ang, ang), dim=-1)
            self._cos, self._sin, self._cache_key = ang.cos(), ang.sin(), key
        return self._cos, self._sin

    @staticmethod
    def _rotate_half(x: torch.Tensor) -> torch.Tensor:
        h = x.shape[-1] // 2
        return torch.cat((-x[..., h:], x[..., :h]), dim=-1)

    def rotate(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
        return x * cos + self._rotate_half(x) * sin

    def forward(self, q: torch.Tensor, k: torch.Tensor,
                position_offset: int = 0) -> Tuple[torch.Tensor, torch.Tensor]:
        s = q.shape[2]
        cos, sin = self._table(s + position_offset, q.device, q.dtype)
        cos = cos[position_offset:position_offset + s][None, None]
        sin = sin[position_offset:position_offset + s][None, None]
        return self.rotate(q, cos, sin), self.rotate(k, cos, sin)

    def forward_varlen(self, q: torch.Tensor, k: torch.Tensor, cu_seqlens: torch.Tensor,
                       norm_q: Optional[torch.Tensor] = None,
                       norm_k: Optional[torch.Tensor] = None,
                       eps: float = 1e-6, grad_slab=None) -> Tuple[torch.Tensor, torch.Tensor]:
        """q [T, H, D], k [T, H_KV, D]; position of token t = t - cu[seq(t)]
        (the HIP rotary kernel; GPU tensors only).  With norm weights the
        rows are RMS-normalised first, in the same launch.  grad_slab: where
        the backward writes dq, dk (GradSlab blocks 0 and 1)."""
        return rope_varlen(q, k, cu_seqlens, self.inv_freq, norm_q, norm_k, eps, grad_slab)


def _stacked_view(ws) -> Optional[torch.Tensor]:
    """The weights as one [sum rows, E] matrix when they are consecutive row
    blocks of one buffer (no copy), else None."""
    w0 = ws[0]
    E = w0.shape[1]
    if not all(w.dim() == 2 and w.shape[1] == E and w.is_contiguous() and
               w.dtype == w0.dtype and w.device == w0.device for w in ws):
        return None
    st = w0.untyped_storage()
    off = w0.storage_offset()
    for w in ws:
        if w.untyped_storage().data_ptr() != st.data_ptr() or w.storage_offset() != off:
            return None
        off += w.numel()
    rows = sum(w.shape[0] for w in ws)
    return w0.detach().new_empty(0).set_(st, w0.storage_offset(), (rows, E), (E, 1))


class GradSlab:
    """One [rows, sum(sizes)] buffer whose consecutive column blocks receive
    the gradients of the stacked projection's outputs (q, k, v, R_q, R_k),
    written there by the kernels that produce them (the RoPE backward: dq,
    dk; the attention backward: dv, dR_q, dR_k).  The projection's backward
    then finds its cotangents as column blocks of one buffer and runs one dx
    and one dW GEMM, with no concatenation.  Allocated by the first backward
    that asks for a block; a block is a view of it with the gradient's
    shape.  A block asked for again (a second backward through a retained
    graph) starts a new buffer, so that gradients already returned are never
    overwritten."""

    def __init__(self, rows: int, sizes, dtype: torch.dtype, device):
        self.rows, self.sizes, self.dtype, self.device = rows, list(sizes), dtype, device
        self.buf = None
        self.given = set()

    def block(self, i: int, like) -> torch.Tensor:
        """The gradient of output block i in the layout of ``like``: a view
        of column block i of the projection's output (its strides are in
        that output's [rows, sum(sizes)] geometry, which the buffer has too),
        or a (shape, strides) pair of such a view.  Any other layout gets a
        tensor of its own (so the projection's backward takes its per-block
        path)."""
        shape, stride = (like.shape, like.stride()) if torch.is_tensor(like) else like
        if not _block_layout(shape, stride, self.sizes[i], sum(self.sizes), self.rows):
            return torch.empty(shape, dtype=self.dtype, device=self.device)
        if self.buf is None or i in self.given:
            self.buf = torch.empty(self.rows, sum(self.sizes), dtype=self.dtype,
                                   device=self.device)
            self.given = set()
        self.given.add(i)
        c0 = sum(self.sizes[:i])
        return self.buf.as_strided(shape, stride, self.buf.storage_offset() + c0)


def _block_layout(shape, stride, n: int, width: int, rows: int) -> bool:
    """Whether (shape, stride) addresses exactly the first n columns of each
    of ``rows`` rows of a row-major [rows, width] matrix: the dimensions of
    stride below ``width`` tile the n columns densely, the others step whole
    rows."""
    inner = sorted((st, sz) for st, sz in zip(stride, shape) if st < width and sz > 1)
    outer = [(st, sz) for st, sz in zip(stride, shape) if st >= width and sz > 1]
    span = 1
    for st, sz in inner:
        if st != span:
            return False
        span *= sz
    if span != n:
        return False
    last = 0
    for st, sz in outer:
        if st % width:
            return False
        last += (st // width) * (sz - 1)
    return last < rows and math.prod(sz for _, sz in outer) == rows


def _column_blocks(gs, sizes) -> Optional[torch.Tensor]:
    """The gradients as one [rows, sum sizes] matrix when they are consecutive
    column blocks of one buffer with a common row stride (no copy), else None."""
    if any(g is None for g in gs):
        return None
    flat = []
    for g, n in zip(gs, sizes):
        try:
            flat.append(g.view(-1, n))
        except RuntimeError:
            return None
    f0 = flat[0]
    ld = f0.stride(0)
    st = f0.untyped_storage().data_ptr()
    off = f0.storage_offset()
    for f, n in zip(flat, sizes):
        if (f.stride(1) != 1 or f.stride(0) != ld or f.shape[0] != f0.shape[0] or
                f.untyped_storage().data_ptr() != st or f.storage_offset() != off):
            return None
        off += n
    total = sum(sizes)
    if ld < total:
        return None
    return f0.new_empty(0).set_(f0.untyped_storage(), f0.storage_offset(), (f0.shape[0], total),
                                (ld, 1))


class _StackedProjection(torch.autograd.Function):
    """The projections x W_i^T of weights that are consecutive row blocks of
    one buffer, as ONE GEMM over the stacked weights; the outputs are column
    views of its result.  Backward: each dW_i = dY_i^T x is written into its
    row block of one dW buffer (the parameters' gradients are views of it),
    and dx is one GEMM when the dY_i are consecutive column blocks of one
    buffer, else the per-block GEMMs accumulated in place: no concatenation
    of the weights or of the gradients, and no separate additions.

    Under autocast the GEMMs run in the forward's compute dtype (the dtype
    of its output), as ``F.linear`` does: the backward casts x, the weights
    and the incoming gradients to it, and returns dx in x's dtype and each
    dW in the weights' dtype.  As for ``nn.Linear``, a weight that needs no
    gradient gets no dW GEMM, and a block whose output did not reach the
    loss gets ``None``."""

    @staticmethod
    def forward(ctx, x, w_all, sizes, *ws):
        y = F.linear(x, w_all)
        ctx.set_materialize_grads(False)  # an unused output's cotangent stays None
        ctx.save_for_backward(x)
        ctx.w_all = w_all
        ctx.sizes = sizes
        ctx.cdtype = y.dtype
        return tuple(torch.split(y, sizes, dim=-1))

    @staticmethod
    def backward(ctx, *gys):
        (x,) = ctx.saved_tensors
        w_all, sizes, cd = ctx.w_all, ctx.sizes, ctx.cdtype
        E = x.shape[-1]
        x2 = x.reshape(-1, E).to(cd)
        w_c = w_all.to(cd)
        gys = tuple(None if g is None else g.to(cd) for g in gys)
        need_w = ctx.needs_input_grad[3:]
        dw_all = None
        if any(n and g is not None for n, g in zip(need_w, gys)):
            dw_all = torch.empty_like(w_all)
        stacked = _column_blocks(gys, sizes)
        if stacked is not None and all(need_w) and dw_all.dtype == cd:
            # every block's dW in one GEMM: dW_all = dY_all^T x
            torch.mm(stacked.t(), x2, out=dw_all)
            gys_w = ()
            dws = list(torch.split(dw_all, sizes, dim=0))
        else:
            gys_w = gys
            dws = []
        r0 = 0
        for g, n, need in zip(gys_w, sizes, need_w):
            if g is None or not need:
                dws.append(None)
            else:
                blk = dw_all[r0:r0 + n]
                if blk.dtype == cd:
                    torch.mm(g.reshape(-1, n).t(), x2, out=blk)
                else:
                    blk.copy_(torch.mm(g.reshape(-1, n).t(), x2))
                dws.append(blk)
            r0 += n
        dx = None
        if ctx.needs_input_grad[0]:
            if stacked is not None:
                dx = torch.mm(stacked, w_c)
            else:
                r0 = 0
                for g, n in zip(gys, sizes):
                    if g is not None:
                        g2, w = g.reshape(-1, n), w_c[r0:r0 + n]
                        if dx is None:
                            dx = torch.mm(g2, w)
                        else:
                            dx.addmm_(g2, w)
                    r0 += n
                if dx is None:
                    dx = torch.zeros_like(x2)
            dx = dx.view(x.shape).to(x.dtype)
        return (dx, None, None, *dws)


class NaylisAttention(nn.Module):
    """Token-graph attention: softmax(scale Q K^T + gs_h R_q R_k^T) V per head,
    with R_q, R_k low-rank projections of x for the first H_G = num_heads -
    vanilla_heads heads.  Constructor and forward as attention_fna2.py:197-215
    and :380-390."""

    # The packed path's backward writes the gradients of q, k, v, R_q, R_k
    # into one buffer (GradSlab); False: separate tensors (the same values up
    # to the rounding of the projection's GEMMs).
    _grad_slab = True

    def __init__(
        self,
        embed_dim: int,
        num_heads: int,
        dropout: float = 0.0,
        use_rope: bool = True,
        max_seq_len: int = 2048,
        use_yarn: bool = False,
        yarn_scale: float = 1.0,
        yarn_original_max_len: int = 1024,
        n_kv_heads: Optional[int] = None,
        use_qk_norm: bool = True,
        use_flash_attn: bool = True,
        soft_cap: Optional[float] = None,
        rel_rank: int = 32,
        sym_heads: int = 0,
        vanilla_heads: int = 0,
        use_fna2: Optional[bool] = None,
        decode_graph_bias: bool = False,
    ):
        super().__init__()
        assert embed_dim % num_heads == 0
        graph_heads = num_heads - vanilla_heads
        assert 0 <= sym_heads <= graph_heads
        assert 0 <= vanilla_heads < num_heads

        self._fna2_compatible = _FNA2_AVAILABLE and rank_supported(rel_rank)
        want = (soft_cap is None) if use_fna2 is None else bool(use_fna2)
        self._use_fna2 = want and self._fna2_compatible

        self.embed_dim = embed_dim
        self.num_heads = num_heads
        self.head_dim = embed_dim // num_heads
        self.use_rope = use_rope
        self.use_qk_norm = use_qk_norm
        self.soft_cap = soft_cap
        self.rel_rank = rel_rank
        self.sym_heads = sym_heads
        self.vanilla_heads = vanilla_heads
        self.graph_heads = graph_heads
        self.n_kv_heads = num_heads if n_kv_heads is None else n_kv_heads
        assert num_heads % self.n_kv_heads == 0
        self.num_queries_per_kv = num_heads // self.n_kv_heads
        self.kv_dim = self.n_kv_heads * self.head_dim

        self.q_proj = nn.Linear(embed_dim, embed_dim, bias=False)
        self.k_proj = nn.Linear(embed_dim, self.kv_dim, bias=False)
        self.v_proj = nn.Linear(embed_dim, self.kv_dim, bias=False)
        self.out_proj = nn.Linear(embed_dim, embed_dim, bias=False)
        self.dropout = nn.Dropout(dropout)
        if use_qk_norm:
            self.q_norm = RMSNorm(self.head_dim)
            self.k_norm = RMSNorm(self.head_dim)
        else:
            self.q_norm = self.k_norm = None
        self.rope = (RotaryPositionalEmbedding(self.head_dim, max_seq_len, use_yarn=use_yarn,
                                               yarn_scale=yarn_scale,
                                               yarn_original_max_len=yarn_original_max_len)
                     if use_rope else None)
        if graph_heads > 0:
            self.rel_q_proj = nn.Linear(embed_dim, graph_heads * rel_rank, bias=False)
            self.rel_k_proj = nn.Linear(embed_dim, graph_heads * rel_rank, bias=False)
            nn.init.normal_(self.rel_q_proj.weight, std=0.01)
            nn.init.normal_(self.rel_k_proj.weight, std=0.01)
            self.graph_scale = nn.Parameter(torch.zeros(graph_heads))
        else:
            self.rel_q_proj = self.rel_k_proj = None
            self.graph_scale = None
        self._sdpa_ok = hasattr(F, "scaled_dot_product_attention")
        # Keep R_k in the KV cache, (k, v, r_k), and decode with the graph
        # bias (the reference's cache is (k, v) and its decode step drops the
        # bias).
        self.decode_graph_bias = bool(decode_graph_bias) and graph_heads > 0
        # The FNA2 path projects x once, over the stacked weights: keep them
        # as consecutive row blocks of one buffer (the parameters, their
        # names and the state dict are unchanged).
        with torch.no_grad():
            self._pack_projection_weights()

    # ── helpers ────────────────────────────────────────────────────────────
    def _attn_scale(self) -> float:
        if self.rope is not None and self.rope.use_yarn and self.rope.yarn_scale > 1.0:
            return math.sqrt(self.rope.yarn_scale) / math.sqrt(self.head_dim)
        return 1.0 / math.sqrt(self.head_dim)

    def _projection_weights(self):
        ws = [self.q_proj.weight, self.k_proj.weight, self.v_proj.weight]
        if self.graph_heads > 0:
            ws += [self.rel_q_proj.weight, self.rel_k_proj.weight]
        return ws

    def _pack_projection_weights(self) -> torch.Tensor:
        """Make the projection weights consecutive row blocks of one buffer
        (one copy; needed again only after something rebinds a weight, e.g.
        .to(), a load with assign=True) and return the stacked view."""
        ws = self._projection_weights()
        w_all = _stacked_view(ws)
        if w_all is not None:
            return w_all
        w0 = ws[0]
        buf = torch.empty(sum(w.shape[0] for w in ws), w0.shape[1], dtype=w0.dtype,
                          device=w0.device)
        r0 = 0
        for w in ws:
            n = w.shape[0]
            buf[r0:r0 + n].copy_(w.detach())
            w.data = buf[r0:r0 + n]
            r0 += n
        return buf

    def _project(self, x: torch.Tensor):
        """q, k, v and (with graph heads) R_q, R_k from ONE GEMM over the
        stacked weights [W_q; W_k; W_v; W_rq; W_rk], which are kept as
        consecutive row blocks of one buffer (the GEMM reads them in place;
        the backward is one dx and one dW GEMM).  The outputs are views into
        the [.., E + 2 kv_dim + 2 H_G R] result, which the HIP kernels read
        through their strides.  Replaces the five projections of
        attention_fna2.py:401-403, :554-556 and _compute_rq_rk(_varlen)
        (:301-335): x is read once, and R needs no .contiguous() copy; in
        bf16 (the FNA2 path's dtype) R is already bf16, so the reference's
        .to(torch.bfloat16) is not a pass either.  The parameters stay
        separate modules (state dicts unchanged)."""
        with torch.no_grad():
            w_all = self._pack_projection_weights()
        gr = self.graph_heads * self.rel_rank
        sizes = [self.embed_dim, self.kv_dim, self.kv_dim] + ([gr, gr] if gr else [])
        parts = _StackedProjection.apply(x, w_all, sizes, *self._projection_weights())
        lead = x.shape[:-1]
        q = parts[0].view(lead + (self.num_heads, self.head_dim))
        k = parts[1].view(lead + (self.n_kv_heads, self.head_dim))
        v = parts[2].view(lead + (self.n_kv_heads, self.head_dim))
        r_q = r_k = None
        if gr:
            r_q = parts[3].view(lead + (self.graph_heads, self.rel_rank))
            r_k = parts[4].view(lead + (self.graph_heads, self.rel_rank))
            if r_q.dtype != torch.bfloat16:  # fp32 activations (the reference casts too)
                r_q, r_k = r_q.to(torch.bfloat16), r_k.to(torch.bfloat16)
        if x.dim() == 3:  # [B, S, h, *] -> [B, h, S, *]
            q, k, v = (t.transpose(1, 2) for t in (q, k, v))
            if gr:
                r_q, r_k = r_q.transpose(1, 2), r_k.transpose(1, 2)
        return q, k, v, r_q, r_k

    def _dense_bias(self, x: torch.Tensor, dtype: torch.dtype) -> torch.Tensor:
        """gs_h R_q R_k^T for graph heads (zeros for vanilla heads), [B, H, S, S]."""
        assert dtype == torch.bfloat16, "the graph bias is bf16"
        B, S, _ = x.shape
        r_q = self.rel_q_proj(x).view(B, S, self.graph_heads, self.rel_rank).transpose(1, 2)
        r_k = self.rel_k_proj(x).view(B, S, self.graph_heads, self.rel_rank).transpose(1, 2)
        bias = torch.matmul(r_q, r_k.transpose(-2, -1).contiguous())
        if self.sym_heads > 0:
            sym = bias[:, :self.sym_heads]
            bias = torch.cat([(sym + sym.transpose(-2, -1)) * 0.5, bias[:, self.sym_heads:]], 1)
        bias = (self.graph_scale.view(1, -1, 1, 1) * bias).to(dtype)
        if self.vanilla_heads > 0:
            bias = torch.cat([bias, bias.new_zeros(B, self.vanilla_heads, S, S)], dim=1)
        return bias.contiguous()

    def _finish(self, out: torch.Tensor, orig_dtype: torch.dtype) -> torch.Tensor:
        if out.dtype != orig_dtype:
            out = out.to(orig_dtype)
        if out.dtype != self.out_proj.weight.dtype:
            out = out.to(self.out_proj.weight.dtype)
        return self.dropout(self.out_proj(out))

    # ── forward ────────────────────────────────────────────────────────────
    def forward(
        self,
        x: torch.Tensor,
        mask: Optional[torch.Tensor] = None,
        past_kv: Optional[KVCache] = None,
        use_kv_cache: bool = False,
        cu_seqlens_q: Optional[torch.Tensor] = None,
        cu_seqlens_k: Optional[torch.Tensor] = None,
        max_seqlen_q: Optional[int] = None,
        max_seqlen_k: Optional[int] = None,
    ) -> Tuple[torch.Tensor, Optional[KVCache]]:
        if cu_seqlens_q is not None:
            return self._forward_varlen(x, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                        max_seqlen_k)
        if isinstance(past_kv, StaticKVCache):
            return self._forward_static(x, mask, past_kv, use_kv_cache)
        B, S, _ = x.shape
        scale = self._attn_scale()
        keep_rk = self.decode_graph_bias
        if keep_rk and past_kv is not None and len(past_kv) < 3:
            raise ValueError("decode_graph_bias: past_kv must be the (k, v, r_k) cache "
                             "this module returns")
        fused = (self._use_fna2 and self.graph_heads > 0 and self.soft_cap is None
                 and past_kv is None)
        # One new token against a cache: the decode kernel (attention_fna2.py
        # :412-429 decodes with SDPA over torch.cat(past_kv, new)).
        kernel_decode = (self._use_fna2 and past_kv is not None and S == 1
                         and self.soft_cap is None
                         and not (self.training and self.dropout.p > 0)
                         and self._decode_kernel_ok(keep_rk))
        r_q = r_k = None
        if fused or kernel_decode:
            q, k, v, r_q, r_k = self._project(x)
        else:
            q = self.q_proj(x).view(B, S, self.num_heads, self.head_dim).transpose(1, 2)
            k = self.k_proj(x).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
            v = self.v_proj(x).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
            if keep_rk:
                r_q, r_k = self._rel(x)
        slab = None
        offset = past_kv[0].shape[2] if past_kv is not None else 0
        if fused and self.rope is not None:
            # QK-RMSNorm and RoPE in the varlen launch: the batch's rows are B
            # sequences of S tokens (positions 0 .. S - 1), read where the
            # projection wrote them
            assert not self.use_qk_norm or self.q_norm.eps == self.k_norm.eps
            slab = self._slab_for(q, B * S)
            qf = q.transpose(1, 2).reshape(B * S, self.num_heads, self.head_dim)
            kf = k.transpose(1, 2).reshape(B * S, self.n_kv_heads, self.head_dim)
            qr, kr = self.rope.forward_varlen(
                qf, kf, self._batch_cu(B, S, x.device),
                self.q_norm.weight if self.use_qk_norm else None,
                self.k_norm.weight if self.use_qk_norm else None,
                self.q_norm.eps if self.use_qk_norm else 1e-6, grad_slab=slab)
            q = qr.view(B, S, self.num_heads, self.head_dim).transpose(1, 2)
            k = kr.view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
        else:
            if self.use_qk_norm:
                q, k = self.q_norm(q), self.k_norm(k)
            if self.rope is not None:
                q, k = self.rope(q, k, position_offset=offset)
        if past_kv is not None:
            k = torch.cat([past_kv[0], k], dim=2)
            v = torch.cat([past_kv[1], v], dim=2)
            if keep_rk:
                r_k = torch.cat([past_kv[2], r_k], dim=2)
        new_cache: Optional[KVCache] = None
        if use_kv_cache:
            new_cache = (k, v, r_k.contiguous()) if keep_rk else (k, v)

        orig_dtype = q.dtype
        if q.dtype == torch.float32:
            q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
        is_causal = S > 1 and past_kv is None
        use_graph = self.graph_heads > 0 and (S > 1 or past_kv is None)
        cached_bias = keep_rk and past_kv is not None and S == 1

        if fused:
            out = _flash_naylis_attn(q, k, v, r_q, r_k, self.graph_scale.to(torch.float32),
                                     softmax_scale=scale, is_causal=is_causal, grad_slab=slab)
        elif kernel_decode:
            out = flash_naylis_decode(
                q, k, v, r_q if cached_bias else None, r_k if cached_bias else None,
                self.graph_scale if cached_bias else None, softmax_scale=scale).unsqueeze(2)
        else:
            bias = self._cached_bias(r_q, r_k, q.dtype) if cached_bias else None
            out = self._attend_eager(x, q, k, v, mask, past_kv, scale, is_causal, use_graph,
                                     bias)
        out = out.transpose(1, 2).contiguous().view(B, S, self.embed_dim)
        return self._finish(out, orig_dtype), new_cache

    def _forward_static(self, x, mask, cache: StaticKVCache, use_kv_cache: bool):
        """A step against a preallocated cache: an empty cache takes the
        prompt (the ordinary causal forward, whose k / v / r_k rows are then
        written into the cache); a nonempty one takes one token, appended in
        place, and attends to the cache's rows on the decode kernel (or the
        eager backends, as the tuple cache does)."""
        B, S, _ = x.shape
        keep_rk = self.decode_graph_bias
        if keep_rk and cache.r_k is None:
            raise ValueError("decode_graph_bias: the StaticKVCache must hold r_k")
        if cache.length == 0:
            out, new = self.forward(x, mask, None, True)
            cache.append(*new)
            return out, (cache if use_kv_cache else None)
        if S != 1:
            raise ValueError("a StaticKVCache with rows in use takes one token per step")
        scale = self._attn_scale()
        kernel_decode = (self._use_fna2 and self.soft_cap is None
                         and not (self.training and self.dropout.p > 0)
                         and self._decode_kernel_ok(keep_rk))
        r_q = r_k = None
        if kernel_decode:
            q, k, v, r_q, r_k = self._project(x)
        else:
            q = self.q_proj(x).view(B, S, self.num_heads, self.head_dim).transpose(1, 2)
            k = self.k_proj(x).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
            v = self.v_proj(x).view(B, S, self.n_kv_heads, self.head_dim).transpose(1, 2)
            if keep_rk:
                r_q, r_k = self._rel(x)
        if self.use_qk_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        if self.rope is not None:
            q, k = self.rope(q, k, position_offset=cache.length)
        cache.append(k, v, r_k if keep_rk else None)
        rows = cache.view()
        kc, vc = rows[0], rows[1]
        orig_dtype = q.dtype
        if q.dtype == torch.float32:
            q = q.to(torch.bfloat16)
        if kc.dtype != torch.bfloat16:
            kc, vc = kc.to(torch.bfloat16), vc.to(torch.bfloat16)
        if kernel_decode:
            out = flash_naylis_decode(
                q, kc, vc, r_q if keep_rk else None, rows[2] if keep_rk else None,
                self.graph_scale if keep_rk else None, softmax_scale=scale).unsqueeze(2)
        else:
            bias = self._cached_bias(r_q, rows[2], q.dtype) if keep_rk else None
            out = self._attend_eager(x, q, kc, vc, mask, rows, scale, False, False, bias)
        out = out.transpose(1, 2).contiguous().view(B, S, self.embed_dim)
        return self._finish(out, orig_dtype), (cache if use_kv_cache else None)

    def _decode_kernel_ok(self, with_bias: bool) -> bool:
        """The decode kernel serves this head geometry (at most 32 query
        heads per KV head and, with the cached bias, a group's graph heads x
        R within one rank tile); other models decode on the eager path, as
        the reference does."""
        key = bool(with_bias)
        cache = self.__dict__.setdefault("_decode_ok_cache", {})
        if key not in cache:
            cache[key] = decode_supported(self.num_heads, self.n_kv_heads, self.head_dim,
                                          self.graph_heads if with_bias else 0,
                                          self.rel_rank if with_bias else 0)
        return cache[key]

    def _rel(self, x: torch.Tensor):
        """R_q, R_k [B, H_G, S, R] in bf16 (attention_fna2.py:301-318)."""
        B, S, _ = x.shape
        r_q = self.rel_q_proj(x).view(B, S, self.graph_heads, self.rel_rank).transpose(1, 2)
        r_k = self.rel_k_proj(x).view(B, S, self.graph_heads, self.rel_rank).transpose(1, 2)
        return r_q.to(torch.bfloat16), r_k.to(torch.bfloat16)

    def _cached_bias(self, r_q, rk_cache, dtype) -> torch.Tensor:
        """gs_h <Rq_new, Rk_j> against the cached rows, [B, H, 1, L] (zeros
        for vanilla heads), for the eager backends."""
        bias = torch.matmul(r_q.float(), rk_cache.float().transpose(-2, -1).contiguous())
        bias = (self.graph_scale.float().view(1, -1, 1, 1) * bias).to(dtype)
        if self.vanilla_heads > 0:
            B, _, _, L = bias.shape
            bias = torch.cat([bias, bias.new_zeros(B, self.vanilla_heads, 1, L)], dim=1)
        return bias

    def _attend_eager(self, x, q, k, v, mask, past_kv, scale, is_causal, use_graph,
                      bias=None):
        """The reference's non-FNA2 backends: SDPA with a dense bias, or the
        explicit softmax for soft_cap (attention_fna2.py:449-516).  ``bias``:
        a precomputed additive bias (decoding against a cache with R_k)."""
        if self.n_kv_heads != self.num_heads:
            k = k.repeat_interleave(self.num_queries_per_kv, dim=1)
            v = v.repeat_interleave(self.num_queries_per_kv, dim=1)
        p_drop = self.dropout.p if self.training else 0.0
        if bias is None and use_graph:
            bias = self._dense_bias(x, q.dtype)
        if self._sdpa_ok and self.soft_cap is None:
            if bias is not None and is_causal:
                sq, sk = q.shape[2], k.shape[2]
                tri = torch.full((sq, sk), float("-inf"), device=q.device, dtype=q.dtype)
                bias = bias + torch.triu(tri, diagonal=1 + (past_kv[0].shape[2] if past_kv else 0))
            return F.scaled_dot_product_attention(
                q, k, v, attn_mask=None if bias is None else bias.contiguous(),
                is_causal=bias is None and is_causal, dropout_p=p_drop, scale=scale)
        scores = torch.matmul(q, k.transpose(-2, -1)) * scale
        if self.soft_cap is not None:
            scores = self.soft_cap * torch.tanh(scores / self.soft_cap)
        if bias is not None:
            scores = scores + bias
        if is_causal:
            blocked = (mask.unsqueeze(0).unsqueeze(0) if mask is not None else
                       torch.triu(torch.ones(q.shape[2], k.shape[2], device=q.device,
                                             dtype=torch.bool), diagonal=1))
            scores = scores.masked_fill(blocked, float("-inf"))
        w = torch.nan_to_num(F.softmax(scores, dim=-1), nan=0.0)
        if self.training and self.dropout.p > 0:
            w = self.dropout(w)
        return torch.matmul(w, v)

    def _slab_for(self, q: torch.Tensor, rows: int) -> Optional[GradSlab]:
        """A GradSlab for this call's projection gradients, where the RoPE
        launch and the attention op run eagerly on its bf16 outputs."""
        if not (self._grad_slab and torch.is_grad_enabled() and self._use_fna2 and
                q.dtype == torch.bfloat16 and type(q) is torch.Tensor and
                _fna2_plain_eager(q)):
            return None
        gr = self.graph_heads * self.rel_rank
        return GradSlab(rows, [self.embed_dim, self.kv_dim, self.kv_dim] + ([gr, gr] if gr else []),
                        q.dtype, q.device)

    def _batch_cu(self, B: int, S: int, device) -> torch.Tensor:
        """cu_seqlens of B sequences of S tokens (kept for the next call)."""
        key = (B, S, device)
        if getattr(self, "_cu_key", None) != key:
            self._cu = torch.arange(0, B * S + 1, S, dtype=torch.int32, device=device)
            self._cu_key = key
        return self._cu

    def _forward_varlen(self, x, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k):
        """x [T, E] packed (attention_fna2.py:533-617); causal within each sequence."""
        T = x.shape[0]
        scale = self._attn_scale()
        q, k, v, r_q, r_k = self._project(x)
        # The backward's gradients of q, k, v, R_q, R_k as column blocks of
        # one buffer (see GradSlab): where the RoPE launch and the attention
        # kernels run eagerly on bf16 projections.
        slab = self._slab_for(q, T) if self.rope is not None else None
        if self.rope is not None:  # QK-RMSNorm (if any) and RoPE in one launch
            assert not self.use_qk_norm or self.q_norm.eps == self.k_norm.eps
            q, k = self.rope.forward_varlen(
                q, k, cu_seqlens_q,
                self.q_norm.weight if self.use_qk_norm else None,
                self.k_norm.weight if self.use_qk_norm else None,
                self.q_norm.eps if self.use_qk_norm else 1e-6, grad_slab=slab)
        elif self.use_qk_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        orig_dtype = q.dtype
        if q.dtype == torch.float32:
            q, k, v = (t.to(torch.bfloat16) for t in (q, k, v))
        msq = max_seqlen_q if max_seqlen_q is not None else T
        msk = max_seqlen_k if max_seqlen_k is not None else T
        cu_k = cu_seqlens_k if cu_seqlens_k is not None else cu_seqlens_q
        if not self._use_fna2:
            raise RuntimeError("varlen NaylisAttention needs the FNA2 HIP kernels "
                               "(gfx950 and libfna2_hip.so)")
        gs = self.graph_scale.to(torch.float32) if self.graph_heads > 0 else None
        out = _flash_naylis_attn(q, k, v, r_q, r_k, gs, softmax_scale=scale, is_causal=True,
                                 cu_seqlens_q=cu_seqlens_q, cu_seqlens_k=cu_k,
                                 max_seqlen_q=msq, max_seqlen_k=msk, grad_slab=slab)
        return self._finish(out.reshape(T, self.embed_dim), orig_dtype), None
