"""The reference's eager path restated in torch: SDPA + a materialised bias.

TEST INFRASTRUCTURE ONLY (the CPU baseline of ``bench.py`` and a cross-check
in the tests); the product never imports it.

Restates ``_sdpa_reference`` (myAiByMe/FNA2, FNA2/validate_fna2.py:84-112),
the same construction ``NaylisAttention`` uses without FNA2
(FNA2/attention_fna2.py:337-374, :444-479):

1. GQA: ``repeat_interleave`` K and V to H heads (validate_fna2.py:93-94);
2. bias ``einsum(R_q, R_k) * graph_scale`` in fp32 (:97-98), zero-padded for
   the vanilla heads ``h >= H_G`` (:99-101), then cast to the input dtype
   (:102 — for bf16 inputs this rounds the bias to bf16);
3. causal ``triu(-inf, diagonal=1)`` added to the bias (:104-107);
4. ``scaled_dot_product_attention(q, k, v, attn_mask, scale=scale)`` (:110-112).

Extended (as the kernels are) with ``S_q != S_k`` (top-left causal), a
non-causal mode, and varlen via a loop over ``cu_seqlens`` segments
(FNA2/validate_fna2.py:189-216 checks varlen against per-segment dense).
"""
from __future__ import annotations

import torch
import torch.nn.functional as F


def sdpa_reference(q, k, v, r_q, r_k, graph_scale, scale, causal=True):
    """Dense [B, H, S, D] eager attention with the materialised low-rank bias."""
    B, H, S, D = q.shape
    H_KV, Sk = k.shape[1], k.shape[2]
    G = H // H_KV
    k_exp = k.repeat_interleave(G, dim=1)
    v_exp = v.repeat_interleave(G, dim=1)
    bias = torch.zeros(B, H, S, Sk, dtype=torch.float32, device=q.device)
    if r_q is not None and r_q.shape[1] > 0:
        H_G = r_q.shape[1]
        bias[:, :H_G] = torch.einsum("bhir,bhjr->bhij", r_q.float(), r_k.float()) * \
            graph_scale.float().view(1, H_G, 1, 1)
    bias = bias.to(q.dtype)
    if causal:
        mask = torch.triu(torch.full((S, Sk), float("-inf"), device=q.device, dtype=q.dtype),
                          diagonal=1)
        bias = bias + mask.view(1, 1, S, Sk)
    return F.scaled_dot_product_attention(q, k_exp, v_exp, attn_mask=bias, is_causal=False,
                                          scale=scale)


def sdpa_reference_varlen(q, k, v, r_q, r_k, graph_scale, cu_q, cu_k, scale, causal=True):
    """Varlen [T, H, D]: the dense reference on each cu_seqlens segment."""
    outs = []
    cq = [int(x) for x in cu_q.tolist()]
    ck = [int(x) for x in cu_k.tolist()]
    for b in range(len(cq) - 1):
        qs, qe, ks, ke = cq[b], cq[b + 1], ck[b], ck[b + 1]
        t4 = lambda t, s, e: None if t is None else t[s:e].transpose(0, 1).unsqueeze(0)
        o = sdpa_reference(t4(q, qs, qe), t4(k, ks, ke), t4(v, ks, ke), t4(r_q, qs, qe),
                           t4(r_k, ks, ke), graph_scale, scale, causal)
        outs.append(o.squeeze(0).transpose(0, 1))
    return torch.cat(outs, 0) if outs else q.new_zeros(q.shape)
