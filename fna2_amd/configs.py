"""The five benchmark configurations c1–c5 and their seeded synthetic inputs.

Each generator draws on a CPU ``torch.Generator`` (seed 42 unless given) in the
order q, k, v, r_q, r_k, dO; ``N(0, s)`` is read as standard deviation ``s``.
graph_scale = ones(H) (fp32), H_G = H_KV = H, softmax_scale = 1/sqrt(d).
Dense tensors are allocated ``[B, L, H, *]`` contiguous and returned as
``.transpose(1, 2)`` views ``[B, H, L, *]`` (the layout the configs state,
viewed as the API's ``[B, H, S, *]``).

Length rules (the literal "pad or trim the last sequence" cannot reach the
stated totals for most draws):

* c3: draw 63 lengths ``~ U{64..512}``; redraw all 63 from the same generator
  until ``16384 - sum`` lies in [64, 512]; that residual is the 64th length.
* c5: one 8192-token sequence first, then 384 lengths ``~ U{16..128}``
  rescaled by ``24576 / sum``, rounded, clamped to [16, 128]; the residual goes
  to the last sequence, spilling backwards over earlier ones when clamped.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Optional

import torch


@dataclass
class Config:
    name: str
    dtype: torch.dtype
    varlen: bool
    causal: bool
    H: int
    D: int
    R: int
    r_std: float
    B: int = 0
    L: int = 0
    lengths: Optional[list] = None  # varlen
    backward: bool = True
    desc: str = ""

    @property
    def total(self) -> int:
        return sum(self.lengths) if self.varlen else self.B * self.L

    def seq_lengths(self) -> list:
        return list(self.lengths) if self.varlen else [self.L] * self.B

    def cu_seqlens(self) -> torch.Tensor:
        lens = torch.tensor(self.seq_lengths(), dtype=torch.int64)
        cu = torch.zeros(len(lens) + 1, dtype=torch.int64)
        cu[1:] = torch.cumsum(lens, 0)
        return cu.to(torch.int32)

    def flops(self) -> tuple:
        """Algorithmic (fwd, bwd) FLOPs: 4D+2R and 10D+6R per visible pair per head."""
        pairs = 0
        for n in self.seq_lengths():
            pairs += n * (n + 1) // 2 if self.causal else n * n
        return (pairs * self.H * (4 * self.D + 2 * self.R),
                pairs * self.H * (10 * self.D + 6 * self.R))


def c3_lengths(seed: int = 42, n: int = 64, total: int = 16384, lo: int = 64, hi: int = 512) -> list:
    g = torch.Generator().manual_seed(seed)
    while True:
        head = torch.randint(lo, hi + 1, (n - 1,), generator=g).tolist()
        rest = total - sum(head)
        if lo <= rest <= hi:
            return head + [rest]


def c5_lengths(seed: int = 42, long: int = 8192, n_short: int = 384, total: int = 32768,
               lo: int = 16, hi: int = 128) -> list:
    g = torch.Generator().manual_seed(seed)
    short = torch.randint(lo, hi + 1, (n_short,), generator=g).double()
    target = total - long
    short = (short * (target / short.sum())).round().clamp(lo, hi).long().tolist()
    resid = target - sum(short)
    i = n_short - 1
    while resid != 0 and i >= 0:
        new = min(max(short[i] + resid, lo), hi)
        resid -= new - short[i]
        short[i] = new
        i -= 1
    if resid != 0:
        raise ValueError("c5 length rule cannot reach the total")
    return [long] + short


CONFIGS = {
    "c1": Config("c1", torch.float32, False, True, H=4, D=64, R=8, r_std=1 / math.sqrt(8), B=2,
                 L=256, backward=False,
                 desc="dense causal fwd, fp32, B2 H4 L256 d64 r8 (CPU oracle only)"),
    "c2": Config("c2", torch.bfloat16, False, True, H=16, D=64, R=16, r_std=1 / math.sqrt(16),
                 B=4, L=2048, desc="dense causal fwd+bwd, bf16, B4 H16 L2048 d64 r16"),
    "c3": Config("c3", torch.bfloat16, True, True, H=16, D=128, R=32, r_std=1 / math.sqrt(32),
                 lengths=None, desc="varlen causal fwd+bwd, bf16, 16384 tokens / 64 seqs, "
                 "H16 d128 r32"),
    "c4": Config("c4", torch.bfloat16, False, True, H=32, D=128, R=64, r_std=1 / math.sqrt(64),
                 B=1, L=16384, desc="dense causal fwd+bwd, bf16, B1 H32 L16384 d128 r64"),
    "c5": Config("c5", torch.bfloat16, True, False, H=8, D=64, R=16, r_std=2 / math.sqrt(16),
                 lengths=None, desc="skewed varlen non-causal fwd+bwd, bf16, 32768 tokens "
                 "(8192 + 384 short), H8 d64 r16"),
}


def get(name: str, seed: int = 42) -> Config:
    cfg = CONFIGS[name]
    if name == "c3":
        cfg = Config(**{**cfg.__dict__, "lengths": c3_lengths(seed)})
    elif name == "c5":
        cfg = Config(**{**cfg.__dict__, "lengths": c5_lengths(seed)})
    return cfg


@dataclass
class Inputs:
    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    r_q: torch.Tensor
    r_k: torch.Tensor
    graph_scale: torch.Tensor
    dout: Optional[torch.Tensor]
    scale: float
    cu_seqlens: Optional[torch.Tensor] = None
    max_seqlen: int = 0
    extra: dict = field(default_factory=dict)

    def to(self, device) -> "Inputs":
        f = (lambda t: None if t is None else t.to(device))
        return Inputs(f(self.q), f(self.k), f(self.v), f(self.r_q), f(self.r_k),
                      f(self.graph_scale), f(self.dout), self.scale, f(self.cu_seqlens),
                      self.max_seqlen, self.extra)


def make_inputs(cfg: Config, seed: int = 42, with_dout: bool = True) -> Inputs:
    """Seeded inputs of ``cfg`` on the CPU (move them with ``.to(device)``)."""
    g = torch.Generator().manual_seed(seed)
    H, D, R = cfg.H, cfg.D, cfg.R

    def draw(shape, std=1.0):
        return (torch.randn(shape, generator=g) * std).to(cfg.dtype)

    if cfg.varlen:
        T = cfg.total
        q, k, v = draw((T, H, D)), draw((T, H, D)), draw((T, H, D))
        rq, rk = draw((T, H, R), cfg.r_std), draw((T, H, R), cfg.r_std)
        dout = draw((T, H, D)) if with_dout else None
        cu = cfg.cu_seqlens()
        mx = max(cfg.lengths)
    else:
        B, L = cfg.B, cfg.L
        t = lambda x: x.transpose(1, 2)  # [B, L, H, *] -> [B, H, L, *]
        q, k, v = t(draw((B, L, H, D))), t(draw((B, L, H, D))), t(draw((B, L, H, D)))
        rq, rk = t(draw((B, L, H, R), cfg.r_std)), t(draw((B, L, H, R), cfg.r_std))
        dout = t(draw((B, L, H, D))) if with_dout else None
        cu, mx = None, cfg.L
    gs = torch.ones(H, dtype=torch.float32)
    return Inputs(q, k, v, rq, rk, gs, dout, 1.0 / math.sqrt(D), cu, mx)
