"""Host-side extent model of the attention kernels' global memory accesses.

Every global access of the forward, dQ and dK/dV kernels goes either through
a buffer descriptor (base, record count; the kernel adds lane offsets) or
through a plain pointer.  A buffer load at an offset past the record count
reads zeros without touching memory, so what must lie inside a tensor's
allocation is, per descriptor, the bytes actually read below the record
count: from the base to the last row the count admits, up to the widest
feature a lane reads in that row.  This module restates, for each kernel,
every such range (and every store) from the same view structs the launchers
hand to the C ABI (``_view3`` / ``_view4`` of ``fna2_amd/flash_naylis_attn.py``)
and the workspace layout of ``fna2_amd/csrc/fna2_capi.cpp`` (``bwd_ws``,
checked against ``fna2_bwd_workspace_bytes``), and checks that each one lies
inside its tensor's storage.  CPU only: the tensors are CPU tensors of the
launchers' layouts, no kernel runs.

The sweep covers d 64 / 128, ranks 8-64 (the kernels pad the rank to a
32-wide tile and read only features < R), dense and varlen (empty sequences,
tokens outside every sequence, cross lengths), causal and not, GQA with
vanilla heads, and strided views: [B, S, H, D] memory seen as [B, H, S, D],
and the column views of one stacked projection buffer (q, k, v, R_q, R_k of
``NaylisAttention``).  A restatement of the kernels' rank reads before the
fix of the R = 16 over-read (every chunk of the padded rank tile read from
memory) must fail it.

Sources restated (fna2_amd/csrc): fna2_fwd.hip fwd_body (query rows and rank
rows :116-143, key tiles :101-109, the O staging store and LSE store
:242-283); fna2_bwd_dq.hip dq_body (row loads and delta :149-230, tiles,
epilogue stores :316-383, d_gs partials :386-391); fna2_bwd_dkdv.hip
dkdv_body (RingDma::setup/issue, load_k, load_v, issue_kr, write_rows,
write_drk).
"""
import ctypes
import importlib
import math

import numpy as np
import pytest
import torch

from fna2_amd import _capi

F = importlib.import_module("fna2_amd.flash_naylis_attn")

ALIGN = 256


def cdiv(a, b):
    return -(-a // b)


def align_up(x):
    return cdiv(x, ALIGN) * ALIGN


def kv_bn(D, rpl):
    return 256 if D == 64 and rpl <= 32 else 128


def padded_rank(H_G, R):
    return cdiv(R, 32) * 32 if H_G > 0 and R > 0 else 0


class V:
    """A tensor view as the kernels see it: byte address of element 0,
    element strides, element size, and the byte range of its allocation."""

    def __init__(self, name, t_struct, esize, lo, hi):
        self.name, self.ptr = name, int(t_struct.ptr or 0)
        self.sb, self.ss, self.sh = t_struct.stride_b, t_struct.stride_s, t_struct.stride_h
        self.es, self.lo, self.hi = esize, lo, hi


def _storage(t):
    s = t.untyped_storage()
    return s.data_ptr(), s.data_ptr() + s.nbytes()


def view(name, t, varlen):
    lo, hi = _storage(t)
    st = F._view3(t) if varlen else F._view4(t)
    return V(name, st, t.element_size(), lo, hi)


class Model:
    """Collects byte ranges and checks them against their allocations."""

    def __init__(self, P):
        self.P, self.bad, self.n = P, [], 0

    def base(self, v, b, start, h):
        # seq_base (fna2_device.h): varlen rows from the sequence start, dense
        # rows from the batch base; plus the head
        off = start * v.ss if self.P["varlen"] else b * v.sb
        return v.ptr + (off + h * v.sh) * v.es

    def rows(self, v, base, nrows, width, what):
        """Rows 0 .. nrows-1 of `base` (row stride v.ss), `width` bytes each."""
        if nrows <= 0 or width <= 0:
            return
        self.n += 1
        a, z = base, base + (nrows - 1) * v.ss * v.es + width
        if a < v.lo or z > v.hi:
            self.bad.append((what, v.name, a - v.lo, z - v.hi))


def seqs(P):
    """(b, q0, lq, k0, lk) of every sequence, clamped as seq_ext does."""
    if not P["varlen"]:
        return [(b, 0, P["sq"], 0, P["sk"]) for b in range(P["B"])]
    out = []
    cq, ck, tq, tk = P["cu_q"], P["cu_k"], P["total_q"], P["total_k"]
    for b in range(len(cq) - 1):
        qs = min(max(cq[b], 0), tq)
        qe = min(max(cq[b + 1], qs), tq)
        ks = min(max(ck[b], 0), tk)
        ke = min(max(ck[b + 1], ks), tk)
        out.append((b, qs, qe - qs, ks, ke - ks))
    return out


def kv_span(P, q0t, bm, lq, lk):
    hi = lk
    if P["causal"]:
        hi = min(hi, min(lq, q0t + bm))
    return max(hi, 0)


def model_forward(m, P, T):
    """fwd_body, one workgroup per (query tile of 128, head)."""
    D, R, rpl, H, group = P["D"], P["R"], P["rpl"], P["H"], P["group"]
    BM, BN = 128, 32 if D == 128 else 64
    for (b, q0, lq, k0, lk) in seqs(P):
        for qt in range(cdiv(lq, BM)):
            q0t = qt * BM
            qrows = max(min(BM, lq - q0t), 0)
            for h in range(H):
                kvh, graph = h // group, rpl > 0 and h < P["H_G"]
                q, k, v = T["q"], T["k"], T["v"]
                m.rows(q, m.base(q, b, q0, h) + q0t * q.ss * q.es, qrows, 2 * D, "fwd q")
                if graph:
                    rq = T["rq"]
                    m.rows(rq, m.base(rq, b, q0, h) + q0t * rq.ss * rq.es, qrows, 2 * R, "fwd rq")
                for kt in range(cdiv(kv_span(P, q0t, BM, lq, lk), BN)):
                    rows = max(min(BN, lk - kt * BN), 0)
                    m.rows(k, m.base(k, b, k0, kvh) + kt * BN * k.ss * k.es, rows, 2 * D,
                           "fwd k")
                    m.rows(v, m.base(v, b, k0, kvh) + kt * BN * v.ss * v.es, rows, 2 * D,
                           "fwd v")
                    if graph:
                        rk = T["rk"]
                        m.rows(rk, m.base(rk, b, k0, h) + kt * BN * rk.ss * rk.es, rows,
                               2 * R, "fwd rk")
                o, lse = T["out"], T["lse"]
                for w in range(4):
                    wq0 = q0t + 32 * w
                    n = max(min(32, lq - wq0), 0)
                    m.rows(o, m.base(o, b, q0, h) + wq0 * o.ss * o.es, n, 2 * D, "fwd o")
                m.rows(lse, m.base(lse, b, q0, h) + q0t * lse.ss * 4, qrows, 4, "fwd lse")


def model_dq(m, P, T, W):
    """dq_body, one workgroup per (query tile of 128, head)."""
    D, R, rpl, H, group = P["D"], P["R"], P["rpl"], P["H"], P["group"]
    BM, BN = 128, 32 if (D == 128 or rpl <= 32) else 64
    slot = 0
    for (b, q0, lq, k0, lk) in seqs(P):
        for qt in range(cdiv(lq, BM)):
            q0t = qt * BM
            qrows = max(min(BM, lq - q0t), 0)
            for h in range(H):
                kvh, graph = h // group, rpl > 0 and h < P["H_G"]
                for name in ("q", "dout", "out"):
                    t = T[name]
                    m.rows(t, m.base(t, b, q0, h) + q0t * t.ss * t.es, qrows, 2 * D, "dq " + name)
                lse = T["lse"]
                m.rows(lse, m.base(lse, b, q0, h) + q0t * lse.ss * 4, qrows, 4, "dq lse")
                if graph:
                    rq = T["rq"]
                    m.rows(rq, m.base(rq, b, q0, h) + q0t * rq.ss * rq.es, qrows, 2 * R, "dq rq")
                for kt in range(cdiv(kv_span(P, q0t, BM, lq, lk), BN)):
                    rows = max(min(BN, lk - kt * BN), 0)
                    for name, hh in (("k", kvh), ("v", kvh)):
                        t = T[name]
                        m.rows(t, m.base(t, b, k0, hh) + kt * BN * t.ss * t.es, rows, 2 * D,
                               "dq " + name)
                    if graph:
                        rk = T["rk"]
                        m.rows(rk, m.base(rk, b, k0, h) + kt * BN * rk.ss * rk.es, rows, 2 * R,
                               "dq rk")
                for w in range(4):
                    wq0 = q0t + 32 * w
                    n = max(min(32, lq - wq0), 0)
                    dq = T["dq"]
                    m.rows(dq, m.base(dq, b, q0, h) + wq0 * dq.ss * dq.es, n, 2 * D, "dq dq")
                    if graph:
                        drq = T["drq"]
                        m.rows(drq, m.base(drq, b, q0, h) + wq0 * drq.ss * drq.es, n, 2 * R,
                               "dq drq")
                for name in ("delta", "nlse"):
                    t = T[name] if name == "delta" else W["nlse"]
                    m.rows(t, m.base(t, b, q0, h) + q0t * t.ss * 4, qrows, 4, "dq " + name)
                if graph:
                    part = W["partial"]
                    for wv in range(4):
                        off = ((slot * 4 + wv) * P["H_G"] + h) * 4
                        m.rows(part, part.ptr + off, 1, 4, "dq d_gs partial")
            slot += 1


def model_dkdv(m, P, T, W, rank_read="R"):
    """dkdv_body: items (key tile, KV head), every head of the GQA group.
    rank_read: "R" (the kernels: rank chunks past R are read at an
    out-of-range offset) or "padded" (every chunk of the rank tile read:
    the restatement of the R = 16 over-read)."""
    D, R, rpl, group = P["D"], P["R"], P["rpl"], P["group"]
    BN, BM = kv_bn(D, rpl), 32
    rk_width = 2 * R if rank_read == "R" else 2 * rpl
    for (b, q0, lq, k0, lk) in seqs(P):
        for kt in range(cdiv(lk, BN)):
            k0t = kt * BN
            krows = max(min(BN, lk - k0t), 0)
            qb_lo = k0t // BM if P["causal"] else 0
            nqb = max(cdiv(lq, BM) - qb_lo, 0)
            for kvh in range(P["H_KV"]):
                for name in ("k", "v"):  # load_k / load_v, issue_kr
                    t = T[name]
                    m.rows(t, m.base(t, b, k0, kvh) + k0t * t.ss * t.es, krows, 2 * D,
                           "dkdv " + name)
                for name in ("dk", "dv"):  # write_rows
                    t = T[name]
                    m.rows(t, m.base(t, b, k0, kvh) + k0t * t.ss * t.es, krows, 2 * D,
                           "dkdv " + name)
                for hi in range(group):
                    h = kvh * group + hi
                    graph = rpl > 0 and h < P["H_G"]
                    if graph:
                        rk, drk = T["rk"], T["drk"]
                        m.rows(rk, m.base(rk, b, k0, h) + k0t * rk.ss * rk.es, krows, rk_width,
                               "dkdv rk")
                        m.rows(drk, m.base(drk, b, k0, h) + k0t * drk.ss * drk.es, krows, 2 * R,
                               "dkdv drk")
                    if nqb == 0:
                        continue
                    # RingDma: the sequence's query rows from the first block
                    # that sees the tile
                    r0 = qb_lo * BM
                    n = lq - r0
                    for name in ("q", "dout"):
                        t = T[name]
                        m.rows(t, m.base(t, b, q0, h) + r0 * t.ss * t.es, n, 2 * D,
                               "dkdv " + name)
                    if graph:  # rank chunks past R read at an out-of-range offset
                        rq = T["rq"]
                        m.rows(rq, m.base(rq, b, q0, h) + r0 * rq.ss * rq.es, n, 2 * R,
                               "dkdv rq")
                    for t in (T["delta"], W["nlse"]):
                        m.rows(t, m.base(t, b, q0, h) + r0 * t.ss * 4, n, 4, "dkdv " + t.name)


def workspace(P, lib, prob, device="cpu"):
    """The backward workspace as fna2_capi.cpp's bwd_ws lays it out, checked
    against fna2_bwd_workspace_bytes."""
    rpl, H, H_G = P["rpl"], P["H"], P["H_G"]
    rows_q = P["total_q"] if P["varlen"] else P["B"] * P["sq"]
    off = 0
    if P["varlen"] and P["B"] > 0:
        n = P["B"]
        dq_bound = cdiv(P["total_q"], 128) + n
        kv_bound = cdiv(P["total_k"], kv_bn(P["D"], rpl)) + n
        off += align_up(32 * dq_bound) + ALIGN + align_up(32 * kv_bound) + ALIGN
        q_tiles = dq_bound
    else:
        q_tiles = P["B"] * cdiv(P["sq"], 128)
    partial = off
    off += align_up(4 * 4 * max(q_tiles, 1) * max(H_G, 1))
    nlse = off
    off += align_up(rows_q * H * 4)
    assert off == lib.fna2_bwd_workspace_bytes(ctypes.byref(prob)), "bwd_ws restatement"
    ws = torch.empty(max(off, 1), dtype=torch.uint8, device=device)
    lo, hi = _storage(ws)
    base = ws.data_ptr()
    seq_rows = P["total_q"] if P["varlen"] else P["sq"]

    def mk(name, at, ss, sh, sb, es):
        st = _capi.Tensor(base + at, sb, ss, sh)
        return V(name, st, es, lo, hi)

    W = {"partial": mk("partial", partial, 1, 0, 0, 4),
         "nlse": mk("nlse", nlse, 1, seq_rows, 0 if P["varlen"] else H * seq_rows, 4)}
    # the partials region: [q_tiles][4][H_G] floats
    W["partial"].hi = base + partial + 4 * 4 * max(q_tiles, 1) * max(H_G, 1)
    return W, ws


def build_case(layout, varlen, D, R, H, H_KV, H_G, causal, lengths=None, lengths_k=None, B=2,
               S=200, Sk=None, outside=True):
    """Tensors of one case as the launchers allocate and view them (varlen:
    with `outside`, tokens before and after every sequence)."""
    g = torch.Generator().manual_seed(0)
    mk = lambda *s: torch.zeros(*s, dtype=torch.bfloat16)
    if varlen:
        lengths_k = lengths if lengths_k is None else lengths_k
        pq, pk = (2, 1) if outside else (0, 0)  # tokens before the first sequence
        Tq = sum(lengths) + (5 if outside else 0)
        Tk = sum(lengths_k) + (3 if outside else 0)
        cu_q = [pq] + list(pq + np.cumsum(lengths))
        cu_k = [pk] + list(pk + np.cumsum(lengths_k))
        if layout == "stacked":
            # one projection output [T, E_q + 2 E_kv + 2 H_G R]: column views
            Et = H * D + 2 * H_KV * D + 2 * H_G * R
            buf = mk(max(Tq, Tk), Et)
            c = [0, H * D, H * D + H_KV * D, H * D + 2 * H_KV * D, H * D + 2 * H_KV * D + H_G * R]
            q = buf[:Tq, c[0]:c[1]].view(Tq, H, D)
            k = buf[:Tk, c[1]:c[2]].view(Tk, H_KV, D)
            v = buf[:Tk, c[2]:c[3]].view(Tk, H_KV, D)
            rq = buf[:Tq, c[3]:c[4]].view(Tq, H_G, R) if H_G else None
            rk = buf[:Tk, c[4]:c[4] + H_G * R].view(Tk, H_G, R) if H_G else None
        else:
            q, k, v = mk(Tq, H, D), mk(Tk, H_KV, D), mk(Tk, H_KV, D)
            rq = mk(Tq, H_G, R) if H_G else None
            rk = mk(Tk, H_G, R) if H_G else None
        P = dict(varlen=1, B=len(lengths), sq=0, sk=0, total_q=Tq, total_k=Tk,
                 cu_q=[int(x) for x in cu_q], cu_k=[int(x) for x in cu_k])
    else:
        Sk = S if Sk is None else Sk
        if layout == "bshd":  # [B, S, H, D] memory seen as [B, H, S, D]
            q = mk(B, S, H, D).transpose(1, 2)
            k, v = mk(B, Sk, H_KV, D).transpose(1, 2), mk(B, Sk, H_KV, D).transpose(1, 2)
            rq = mk(B, S, H_G, R).transpose(1, 2) if H_G else None
            rk = mk(B, Sk, H_G, R).transpose(1, 2) if H_G else None
        elif layout == "stacked":
            Et = H * D + 2 * H_KV * D + 2 * H_G * R
            buf = mk(B, max(S, Sk), Et)
            c = [0, H * D, H * D + H_KV * D, H * D + 2 * H_KV * D, H * D + 2 * H_KV * D + H_G * R]
            q = buf[:, :S, c[0]:c[1]].view(B, S, H, D).transpose(1, 2)
            k = buf[:, :Sk, c[1]:c[2]].view(B, Sk, H_KV, D).transpose(1, 2)
            v = buf[:, :Sk, c[2]:c[3]].view(B, Sk, H_KV, D).transpose(1, 2)
            rq = buf[:, :S, c[3]:c[4]].view(B, S, H_G, R).transpose(1, 2) if H_G else None
            rk = (buf[:, :Sk, c[4]:c[4] + H_G * R].view(B, Sk, H_G, R).transpose(1, 2)
                  if H_G else None)
        else:
            q, k, v = mk(B, H, S, D), mk(B, H_KV, Sk, D), mk(B, H_KV, Sk, D)
            rq = mk(B, H_G, S, R) if H_G else None
            rk = mk(B, H_G, Sk, R) if H_G else None
        P = dict(varlen=0, B=B, sq=S, sk=Sk, total_q=0, total_k=0)
    P.update(D=D, R=R if H_G else 0, rpl=padded_rank(H_G, R), H=H, H_KV=H_KV, H_G=H_G,
             group=H // H_KV, causal=causal)
    # as the launchers: _prep, then outputs like the inputs
    q, k, v, rq, rk = (F._prep(t) for t in (q, k, v, rq, rk))
    out = torch.empty_like(q)
    dout = torch.zeros_like(q)
    dq, dk, dv, drq, drk = F._grads_like(q, k, v, rq, rk, H_G)
    if varlen:
        lse = torch.empty(P["total_q"], H)  # the launcher's default, contiguous [T, H]
        delta = torch.empty(H, P["total_q"]).t()
    else:
        lse = torch.empty(B, H, S)
        delta = torch.empty(B, H, S)
    tensors = dict(q=q, k=k, v=v, rq=rq, rk=rk, out=out, dout=dout, lse=lse, delta=delta, dq=dq,
                   dk=dk, dv=dv, drq=drq, drk=drk)
    T = {n: view(n, t, varlen) for n, t in tensors.items() if t is not None}
    cu_t = torch.tensor(P["cu_q"], dtype=torch.int32) if varlen else None
    cu_kt = torch.tensor(P["cu_k"], dtype=torch.int32) if varlen else None
    if varlen:
        prob = F._problem(True, P["B"], max(lengths), max(lengths_k), P["total_q"],
                          P["total_k"], H, H_KV, H_G, D, R if H_G else 0, causal, 0.1, cu_t,
                          cu_kt)
    else:
        prob = F._problem(False, B, S, Sk, 0, 0, H, H_KV, H_G, D, R if H_G else 0, causal, 0.1)
    return P, T, prob, tensors


def check_case(*args, rank_read="R", **kw):
    P, T, prob, keep = build_case(*args, **kw)
    lib = _capi.lib()
    W, ws = workspace(P, lib, prob)
    m = Model(P)
    model_forward(m, P, T)
    model_dq(m, P, T, W)
    model_dkdv(m, P, T, W, rank_read=rank_read)
    assert m.n > 0
    return m.bad


CASES = []
for D in (64, 128):
    for R in (8, 16, 24, 32, 48, 64):
        for layout in ("bhsd", "bshd", "stacked"):
            CASES.append(("dense", layout, D, R))
        CASES.append(("varlen", "packed", D, R))
        CASES.append(("varlen", "stacked", D, R))


@pytest.mark.parametrize("mode,layout,D,R", CASES)
@pytest.mark.parametrize("causal", [True, False])
def test_every_access_inside_its_tensor(mode, layout, D, R, causal):
    if mode == "dense":
        bad = check_case(layout, False, D, R, 4, 2, 3, causal, B=2, S=200, Sk=200)
        bad += check_case(layout, False, D, R, 4, 4, 4, causal, B=1, S=70, Sk=300)
    else:
        bad = check_case(layout, True, D, R, 4, 2, 3, causal,
                         lengths=[300, 0, 1, 129, 64, 33], lengths_k=[300, 5, 1, 100, 64, 257])
    assert not bad, bad[:5]


@pytest.mark.parametrize("layout,varlen", [("bhsd", False), ("packed", True)])
def test_model_catches_the_padded_rank_overread(layout, varlen):
    """Reading every chunk of the 32-wide rank tile from memory (the dK/dV
    rank read before rank chunks past R went to an out-of-range offset) runs
    past the end of a contiguous R = 16 R_k allocation at the last graph
    head's last row; the model must flag it."""
    kw = dict(lengths=[100, 37], outside=False) if varlen else dict(B=1, S=96)
    bad = check_case(layout, varlen, 64, 16, 2, 2, 2, True, rank_read="padded", **kw)
    assert any(w[1] == "rk" for w in bad), bad
    assert not check_case(layout, varlen, 64, 16, 2, 2, 2, True, **kw)
