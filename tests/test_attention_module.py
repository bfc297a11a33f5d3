"""NaylisAttention drop-in (fna2_amd/attention_fna2.py).

CPU: the constructor / forward signatures of the reference
(FNA2/attention_fna2.py:197-215, :380-390) and the eager (non-FNA2) path.
(The varlen RoPE kernel has its own tests: tests/test_rope.py.)
GPU: the FNA2 path (HIP kernels) against the module's eager SDPA path with the
same weights, dense (GQA + vanilla heads) and packed varlen against the dense
path run per sequence.
"""
import copy
import inspect

import pytest
import torch

from fna2_amd import attention_fna2 as A

# FNA2/attention_fna2.py:197-215 and :380-390
CTOR = [("embed_dim", inspect.Parameter.empty), ("num_heads", inspect.Parameter.empty),
        ("dropout", 0.0), ("use_rope", True), ("max_seq_len", 2048), ("use_yarn", False),
        ("yarn_scale", 1.0), ("yarn_original_max_len", 1024), ("n_kv_heads", None),
        ("use_qk_norm", True), ("use_flash_attn", True), ("soft_cap", None),
        ("rel_rank", 32), ("sym_heads", 0), ("vanilla_heads", 0), ("use_fna2", None)]
FWD = [("x", inspect.Parameter.empty), ("mask", None), ("past_kv", None),
       ("use_kv_cache", False), ("cu_seqlens_q", None), ("cu_seqlens_k", None),
       ("max_seqlen_q", None), ("max_seqlen_k", None)]


def _params(fn):
    return [(n, p.default) for n, p in inspect.signature(fn).parameters.items() if n != "self"]


def test_signatures_match_reference():
    # the reference's parameters, in order, then one extra keyword
    assert _params(A.NaylisAttention.__init__) == CTOR + [("decode_graph_bias", False)]
    assert _params(A.NaylisAttention.forward) == FWD
    assert A._FNA2_BLOCK_R == 32


def test_yarn_scale_and_frequencies():
    plain = A.RotaryPositionalEmbedding(64)
    yarn = A.RotaryPositionalEmbedding(64, use_yarn=True, yarn_scale=4.0)
    # even indices up to max(dim/2, dim/4) = 32 keep their frequency (the ramp
    # starts at 1 there); above it the divisor rises linearly to yarn_scale
    torch.testing.assert_close(yarn.inv_freq[:17], plain.inv_freq[:17])
    assert torch.all(yarn.inv_freq[17:] < plain.inv_freq[17:])
    torch.testing.assert_close(plain.inv_freq[31] / yarn.inv_freq[31],
                               torch.tensor(1 + 3 * 30 / 32))
    m = A.NaylisAttention(256, 4, use_yarn=True, yarn_scale=4.0)
    assert abs(m._attn_scale() - 2.0 / 8.0) < 1e-12


def test_eager_path_on_cpu_is_causal_attention():
    torch.manual_seed(1)
    m = A.NaylisAttention(128, 4, rel_rank=8, use_fna2=False).eval()
    with torch.no_grad():
        m.graph_scale.fill_(0.7)
    x = torch.randn(2, 9, 128)
    y, cache = m(x, use_kv_cache=True)
    assert y.shape == (2, 9, 128) and cache[0].shape == (2, 4, 9, 32)
    # causality: output at position t ignores later tokens
    x2 = x.clone()
    x2[:, 5:] += 1.0
    y2, _ = m(x2)
    torch.testing.assert_close(y[:, :5], y2[:, :5], atol=1e-5, rtol=1e-5)


def test_decode_graph_bias_cache_and_eager_decode():
    """decode_graph_bias: the cache is (k, v, r_k) and a decode step equals
    the full causal forward's last row (eager backends, CPU)."""
    torch.manual_seed(2)
    m = A.NaylisAttention(128, 4, n_kv_heads=2, rel_rank=8, vanilla_heads=1, use_fna2=False,
                          decode_graph_bias=True).eval()
    with torch.no_grad():
        m.graph_scale.fill_(2.0)
    x = torch.randn(2, 9, 128)
    with torch.no_grad():
        y_full, _ = m(x)
        _, cache = m(x[:, :8], use_kv_cache=True)
        assert len(cache) == 3 and cache[2].shape == (2, 3, 8, 8)
        y_step, cache2 = m(x[:, 8:], past_kv=cache, use_kv_cache=True)
    assert cache2[0].shape[2] == 9 and cache2[2].shape[2] == 9
    assert (y_step[:, 0] - y_full[:, 8]).abs().max().item() < 2e-2
    # without the bias (the reference's decode) the step differs
    plain = copy.deepcopy(m)
    plain.decode_graph_bias = False
    with torch.no_grad():
        y_plain, _ = plain(x[:, 8:], past_kv=cache[:2])
    assert (y_plain[:, 0] - y_full[:, 8]).abs().max().item() > 1e-2
    with pytest.raises(ValueError):
        m(x[:, 8:], past_kv=cache[:2])


def test_static_kv_cache_mechanics():
    c = A.StaticKVCache.empty(2, 3, 8, 16, graph_heads=2, rank=8, dtype=torch.float32)
    assert c.capacity == 8 and c.length == 0 and len(c.view()) == 3
    k = torch.randn(2, 3, 5, 16)
    v = torch.randn(2, 3, 5, 16)
    rk = torch.randn(2, 2, 5, 8)
    c.append(k, v, rk)
    kv, vv, rv = c.view()
    assert c.length == 5 and torch.equal(kv, k) and torch.equal(vv, v) and torch.equal(rv, rk)
    assert kv.data_ptr() == c.k.data_ptr()  # a view: no copy
    c.append(k[:, :, :3], v[:, :, :3], rk[:, :, :3])
    assert torch.equal(c.view()[0][:, :, 5:], k[:, :, :3])
    with pytest.raises(ValueError):
        c.append(k[:, :, :1], v[:, :, :1], rk[:, :, :1])  # full
    with pytest.raises(ValueError):
        A.StaticKVCache.empty(1, 1, 4, 8, 1, 8).append(k[:1, :1, :1, :8], v[:1, :1, :1, :8])


@pytest.mark.parametrize("bias", [False, True])
def test_static_cache_matches_tuple_cache(bias):
    """Prompt + three decode steps: a StaticKVCache (written in place, bf16)
    gives the tuple cache's outputs (eager backends, CPU)."""
    torch.manual_seed(4)
    m = A.NaylisAttention(128, 4, n_kv_heads=2, rel_rank=8, use_fna2=False,
                          decode_graph_bias=bias).eval()
    with torch.no_grad():
        m.graph_scale.fill_(1.5)
    x = torch.randn(2, 11, 128)
    cache = A.StaticKVCache.empty(2, 2, 16, 32, graph_heads=4 if bias else 0, rank=8)
    with torch.no_grad():
        y0, tup = m(x[:, :8], use_kv_cache=True)
        z0, st = m(x[:, :8], past_kv=cache, use_kv_cache=True)
        assert st is cache and cache.length == 8
        torch.testing.assert_close(z0, y0)
        for t in range(8, 11):
            y, tup = m(x[:, t:t + 1], past_kv=tup, use_kv_cache=True)
            z, st = m(x[:, t:t + 1], past_kv=cache, use_kv_cache=True)
            assert (z - y).abs().max().item() < 1e-2
    assert cache.length == 11
    with pytest.raises(ValueError):
        m(x[:, :2], past_kv=cache)  # several tokens against a nonempty cache


# ── GPU: the FNA2 path against the module's own eager path ──────────────────
# The eager reference (bf16 SDPA with a dense bias, and its backward) runs on
# the CPU; only the FNA2 copy runs on the GPU.

def _pair(**kw):
    torch.manual_seed(3)
    ref = A.NaylisAttention(use_fna2=False, **kw)
    with torch.no_grad():
        ref.graph_scale.uniform_(0.5, 1.5)
    fast = copy.deepcopy(ref).cuda()
    fast._use_fna2 = True
    return ref, fast


@pytest.mark.gpu
@pytest.mark.parametrize("kw", [
    dict(embed_dim=512, num_heads=8, rel_rank=32),
    dict(embed_dim=512, num_heads=4, n_kv_heads=2, rel_rank=16, vanilla_heads=1),
    # YaRN-stretched frequencies and scale, and no QK-norm, through the fused launch
    dict(embed_dim=512, num_heads=4, rel_rank=8, use_yarn=True, yarn_scale=4.0,
         max_seq_len=256, yarn_original_max_len=64),
    dict(embed_dim=512, num_heads=4, rel_rank=8, use_qk_norm=False),
])
def test_fna2_path_matches_eager_dense(gpu, kw):
    assert A._FNA2_AVAILABLE
    ref, fast = _pair(**kw)
    x = torch.randn(2, 200, kw["embed_dim"])
    y_ref, _ = ref(x)
    y_fast, _ = fast(x.cuda())
    assert (y_fast.cpu() - y_ref).abs().max().item() < 2e-2
    g = torch.randn_like(y_ref)
    gr = torch.autograd.grad(y_ref, list(ref.parameters()), g)
    gf = torch.autograd.grad(y_fast, list(fast.parameters()), g.cuda())
    for (name, _), a, b in zip(ref.named_parameters(), gr, gf):
        b = b.cpu()
        rel = ((a - b).float().norm() / a.float().norm().clamp_min(1e-6)).item()
        assert rel < 5e-2, (name, rel)


@pytest.mark.gpu
def test_fna2_varlen_matches_dense_per_sequence(gpu):
    _, fast = _pair(embed_dim=512, num_heads=8, rel_rank=32)
    lens = [37, 128, 5, 90]
    x = torch.randn(sum(lens), 512, device="cuda")
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32,
                      device="cuda")
    y, _ = fast(x, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                max_seqlen_k=max(lens))
    off = 0
    for n in lens:
        yd, _ = fast(x[off:off + n][None])
        assert (y[off:off + n] - yd[0]).abs().max().item() < 2e-2
        off += n


@pytest.mark.gpu
def test_fp16_module_fna2_matches_fp32_eager(gpu):
    """An fp16 NaylisAttention (the reference runs its FNA2 kernels on fp16
    q/k/v too): its FNA2 path, dense and varlen, against the same module's
    eager path in fp32 on the CPU, forward and parameter gradients."""
    assert A._FNA2_AVAILABLE
    ref, fast = _pair(embed_dim=512, num_heads=4, n_kv_heads=2, rel_rank=16, vanilla_heads=1)
    fast = fast.half()
    x = torch.randn(2, 150, 512)
    y_ref, _ = ref(x)
    y_fast, _ = fast(x.half().cuda())
    assert y_fast.dtype == torch.float16
    assert (y_fast.float().cpu() - y_ref).abs().max().item() < 2e-2
    g = torch.randn_like(y_ref)
    gr = torch.autograd.grad(y_ref, list(ref.parameters()), g)
    gf = torch.autograd.grad(y_fast, list(fast.parameters()), g.half().cuda())
    for (name, _), a, b in zip(ref.named_parameters(), gr, gf):
        rel = ((a - b.float().cpu()).norm() / a.norm().clamp_min(1e-6)).item()
        assert rel < 5e-2, (name, rel)
    # varlen: each sequence equals the dense eager path on that sequence
    lens = [37, 128, 5, 90]
    xv = torch.randn(sum(lens), 512)
    cu = torch.tensor([0] + torch.tensor(lens).cumsum(0).tolist(), dtype=torch.int32,
                      device="cuda")
    yv, _ = fast(xv.half().cuda(), cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=max(lens),
                 max_seqlen_k=max(lens))
    off = 0
    for n in lens:
        yd, _ = ref(xv[off:off + n][None])
        assert (yv[off:off + n].float().cpu() - yd[0]).abs().max().item() < 2e-2
        off += n


@pytest.mark.parametrize("lead", [(37,), (2, 19)])
def test_fused_projection_equals_separate_projections(lead):
    """One GEMM over the stacked weights gives the five projections
    (attention_fna2.py:401-403, :301-335) as views of one output."""
    torch.manual_seed(1)
    m = A.NaylisAttention(128, 8, n_kv_heads=2, rel_rank=16, vanilla_heads=2, use_fna2=False)
    x = torch.randn(*lead, 128)
    q, k, v, rq, rk = m._project(x)
    H, D, HKV, HG, R = 8, 16, 2, 6, 16
    sep = [m.q_proj(x).view(*lead, H, D), m.k_proj(x).view(*lead, HKV, D),
           m.v_proj(x).view(*lead, HKV, D), m.rel_q_proj(x).view(*lead, HG, R),
           m.rel_k_proj(x).view(*lead, HG, R)]
    if len(lead) == 2:
        sep = [t.transpose(1, 2) for t in sep]
    for got, want in zip((q, k, v), sep[:3]):
        torch.testing.assert_close(got, want, atol=1e-5, rtol=1e-5)
    for got, want in zip((rq, rk), sep[3:]):
        assert got.dtype == torch.bfloat16
        torch.testing.assert_close(got.float(), want.to(torch.bfloat16).float(), atol=1e-2, rtol=0)
    # q, k, v are views of one buffer (no copies)
    assert q.untyped_storage().data_ptr() == k.untyped_storage().data_ptr() == v.untyped_storage().data_ptr()


@pytest.mark.gpu
def test_kernel_decode_step_matches_full_forward_and_reference_decode(gpu):
    """Decoding one token against the cache on the kernel: with
    decode_graph_bias it equals the FNA2 forward's last row; without, the
    reference's decode step (eager SDPA over the cache, no bias; CPU)."""
    ref, fast = _pair(embed_dim=512, num_heads=8, n_kv_heads=2, rel_rank=32, vanilla_heads=2)
    ref.eval()
    fast.eval()
    x = torch.randn(2, 70, 512)
    xc = x.cuda()
    with torch.no_grad():
        _, cache = fast(xc[:, :69], use_kv_cache=True)
        y_step, _ = fast(xc[:, 69:], past_kv=cache)
        _, rcache = ref(x[:, :69], use_kv_cache=True)
        y_ref, _ = ref(x[:, 69:], past_kv=rcache)
    assert (y_step.cpu() - y_ref).abs().max().item() < 2e-2
    biased = copy.deepcopy(fast)
    biased.decode_graph_bias = True
    with torch.no_grad():
        y_full, _ = biased(xc)
        _, bcache = biased(xc[:, :69], use_kv_cache=True)
        assert len(bcache) == 3
        y_bstep, _ = biased(xc[:, 69:], past_kv=bcache)
    assert (y_bstep[:, 0] - y_full[:, 69]).abs().max().item() < 2e-2


def test_decode_kernel_gating_follows_the_library_limits():
    """The module decodes on the kernel only where fna2_check_decode accepts
    the head geometry: at most 32 query heads per KV head and, with the cached
    bias, a group's graph heads x R within one rank tile.  Other models (MQA
    with 64 heads; 8 graph heads per group at rank 64) take the eager path."""
    from fna2_amd import _capi
    from fna2_amd.decode import decode_supported
    if not _capi.available():
        pytest.skip("libfna2_hip.so not built")
    assert decode_supported(16, 4, 128)
    assert decode_supported(32, 1, 128)
    assert not decode_supported(64, 1, 128)                 # group 64
    assert not decode_supported(16, 4, 96)                  # head_dim
    assert decode_supported(16, 4, 128, 16, 32)             # 4 heads x 32 = 128 wide
    assert not decode_supported(64, 8, 128, 64, 64)         # 8 heads x 64 = 512 wide
    assert decode_supported(64, 8, 128, 0, 0)               # same model, no cached bias
    m = A.NaylisAttention(4096, 64, n_kv_heads=8, rel_rank=64, use_fna2=False)
    assert m._decode_kernel_ok(False) and not m._decode_kernel_ok(True)


@pytest.mark.gpu
@pytest.mark.parametrize("kw,bias", [
    (dict(embed_dim=4096, num_heads=64, n_kv_heads=1, rel_rank=16), False),   # MQA, group 64
    (dict(embed_dim=1024, num_heads=16, n_kv_heads=2, rel_rank=64), True),    # 8 x 64 rank
])
def test_decode_outside_kernel_limits_takes_the_eager_path(gpu, kw, bias):
    """Head geometries the decode kernel does not take decode on the eager
    path (as the reference's SDPA step) instead of raising: equal to the
    eager module's step on the CPU (without the bias) or to the FNA2
    forward's last row (with it)."""
    ref, fast = _pair(**kw)
    ref.eval()
    fast.eval()
    assert not fast._decode_kernel_ok(bias)
    x = torch.randn(2, 24, kw["embed_dim"])
    xc = x.cuda()
    with torch.no_grad():
        if not bias:
            _, cache = fast(xc[:, :23], use_kv_cache=True)
            y_step, _ = fast(xc[:, 23:], past_kv=cache)
            _, rcache = ref(x[:, :23], use_kv_cache=True)
            y_ref, _ = ref(x[:, 23:], past_kv=rcache)
            assert (y_step.cpu() - y_ref).abs().max().item() < 2e-2
        else:
            fast.decode_graph_bias = True
            y_full, _ = fast(xc)
            _, bcache = fast(xc[:, :23], use_kv_cache=True)
            y_bstep, _ = fast(xc[:, 23:], past_kv=bcache)
            assert (y_bstep[:, 0] - y_full[:, 23]).abs().max().item() < 2e-2


@pytest.mark.gpu
@pytest.mark.parametrize("bias", [False, True])
def test_kernel_decode_with_static_cache(gpu, bias):
    """A StaticKVCache on the GPU: prompt on the FNA2 forward, then decode
    steps on the decode kernel reading the cache in place; equal to the
    tuple cache's steps (the same kernel over a torch.cat cache)."""
    _, fast = _pair(embed_dim=512, num_heads=8, n_kv_heads=2, rel_rank=32, vanilla_heads=2)
    fast.eval()
    fast.decode_graph_bias = bias
    x = torch.randn(2, 40, 512, device="cuda")
    cache = A.StaticKVCache.empty(2, 2, 64, 64, graph_heads=6 if bias else 0, rank=32,
                                  device="cuda")
    with torch.no_grad():
        _, tup = fast(x[:, :36], use_kv_cache=True)
        fast(x[:, :36], past_kv=cache, use_kv_cache=True)
        for t in range(36, 40):
            y, tup = fast(x[:, t:t + 1], past_kv=tup, use_kv_cache=True)
            z, _ = fast(x[:, t:t + 1], past_kv=cache, use_kv_cache=True)
            torch.cuda.synchronize()
            assert (z - y).abs().max().item() < 2e-2, t


def test_rope_table_is_sliced_not_rebuilt():
    """The cos / sin table grows to the longest length asked and is sliced:
    rotations are the same whichever lengths were asked before (fp32 and
    bf16, whose table positions are rounded as the reference rounds them)."""
    for dtype in (torch.float32, torch.bfloat16):
        torch.manual_seed(5)
        q = torch.randn(1, 2, 7, 64).to(dtype)
        k = torch.randn(1, 2, 7, 64).to(dtype)
        fresh = A.RotaryPositionalEmbedding(64)
        ref = fresh(q, k, position_offset=300)
        grown = A.RotaryPositionalEmbedding(64)
        grown(q[:, :, :1], k[:, :, :1], position_offset=5)     # a short table first
        grown(q, k, position_offset=1000)                       # then a longer one
        got = grown(q, k, position_offset=300)
        assert grown._cos.shape[0] >= 1007
        torch.testing.assert_close(got[0], ref[0], rtol=0, atol=0)
        torch.testing.assert_close(got[1], ref[1], rtol=0, atol=0)


def test_stacked_projection_backward_and_weight_buffer():
    """The projection weights are consecutive row blocks of one buffer (no
    per-call concatenation); the one-GEMM projection's gradients (x and each
    weight) equal those of the five separate projections; after .to() the
    weights are repacked once; the state dict keeps the reference's keys and
    loads back."""
    torch.manual_seed(4)
    m = A.NaylisAttention(64, 4, n_kv_heads=2, rel_rank=8, vanilla_heads=1)
    ws = m._projection_weights()
    assert len({w.untyped_storage().data_ptr() for w in ws}) == 1
    ref = copy.deepcopy(m)
    x = torch.randn(3, 5, 64)
    lead = x.shape[:-1]
    shapes = [(4, 16), (2, 16), (2, 16), (3, 8), (3, 8)]
    cot = [torch.randn(lead + s_) for s_ in shapes]  # fixed cotangents, [B, S, h, f]

    x1 = x.clone().requires_grad_(True)
    outs = m._project(x1)
    loss1 = sum((t.transpose(1, 2).float() * c).sum() for t, c in zip(outs, cot))
    g1 = torch.autograd.grad(loss1, [x1, *m._projection_weights()])

    x2 = x.clone().requires_grad_(True)
    mods = [ref.q_proj, ref.k_proj, ref.v_proj, ref.rel_q_proj, ref.rel_k_proj]
    sep = [mod(x2).view(lead + s_) for mod, s_ in zip(mods, shapes)]
    sep = sep[:3] + [t.to(torch.bfloat16) for t in sep[3:]]
    loss2 = sum((t.float() * c).sum() for t, c in zip(sep, cot))
    g2 = torch.autograd.grad(loss2, [x2, *ref._projection_weights()])
    for a, b in zip(g1, g2):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)

    # .to() rebinds each weight; the next projection repacks them once
    m.to(torch.float64)
    q64 = m._project(x.double())[0]
    ws64 = m._projection_weights()
    assert all(w.dtype == torch.float64 for w in ws64) and q64.dtype == torch.float64
    assert len({w.untyped_storage().data_ptr() for w in ws64}) == 1
    sd = m.state_dict()
    assert {"q_proj.weight", "k_proj.weight", "v_proj.weight", "rel_q_proj.weight",
            "rel_k_proj.weight"} <= set(sd)
    m3 = A.NaylisAttention(64, 4, n_kv_heads=2, rel_rank=8, vanilla_heads=1).double()
    m3.load_state_dict(sd)
    for a, b in zip(m3._projection_weights(), ws64):
        assert torch.equal(a, b)


@pytest.mark.gpu
def test_module_varlen_bf16_attention_against_oracle(gpu, monkeypatch):
    """The bf16 module's packed path end to end on the GPU: the one-GEMM
    projection (R_q / R_k straight from it, no cast), the fused QK-norm +
    RoPE launch and the attention op.  The attention call's inputs are
    recorded and its output and the gradients that reach q, k, v, R_q, R_k
    and graph_scale are checked against the fp64 oracle on those inputs;
    the projection weights receive gradients."""
    import numpy as np

    from oracle import fna2_oracle as O
    from tests import helpers as H
    torch.manual_seed(8)
    m = A.NaylisAttention(512, 4, n_kv_heads=2, rel_rank=32, vanilla_heads=1).to(
        device=gpu, dtype=torch.bfloat16)
    m._use_fna2 = True
    with torch.no_grad():
        m.graph_scale.uniform_(0.5, 1.5)
    rec = {}
    real = A._flash_naylis_attn

    def recording(q, k, v, r_q, r_k, gs, **kw):
        for name, t in (("q", q), ("k", k), ("v", v), ("rq", r_q), ("rk", r_k), ("gs", gs)):
            t.retain_grad()
            rec[name] = t
        out = real(q, k, v, r_q, r_k, gs, **kw)
        out.register_hook(lambda g: rec.__setitem__("dout", g.detach().clone()))
        rec["out"], rec["kw"] = out, kw
        return out

    monkeypatch.setattr(A, "_flash_naylis_attn", recording)
    lens = [37, 200, 1, 90, 128]
    T = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=gpu)
    x = torch.randn(T, 512, device=gpu, dtype=torch.bfloat16, requires_grad=True)
    print(f"module varlen bf16 T={T}", flush=True)
    y, _ = m(x, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=200, max_seqlen_k=200)
    assert rec["rq"].dtype == torch.bfloat16 and rec["rq"].stride(-1) == 1
    # R_q / R_k are views into the projection's output, as v is (read in place)
    assert rec["rq"].untyped_storage().data_ptr() == rec["v"].untyped_storage().data_ptr()
    y.backward(torch.randn_like(y))
    torch.cuda.synchronize()
    cu_np = cu.cpu().numpy()
    scale = rec["kw"]["softmax_scale"]
    args = [rec[n].detach() for n in ("q", "k", "v", "rq", "rk", "gs")]
    ref_out, ref_lse = O.forward(*args, scale, True, cu_np, cu_np)
    H.check_out(rec["out"], None, ref_out, ref_lse)
    ref_g = O.backward(rec["dout"], *args, ref_out, ref_lse, scale, True, cu_np, cu_np)
    got = [rec[n].grad for n in ("q", "k", "v", "rq", "rk", "gs")]
    H.check_grads(got, ref_g)
    for w in m._projection_weights():
        assert w.grad is not None and torch.isfinite(w.grad.float()).all()


@pytest.mark.gpu
@pytest.mark.parametrize("packed", [True, False])
def test_module_gradient_slab(gpu, monkeypatch, packed):
    """The bf16 FNA2 paths (packed, and dense [B, S, E], whose QK-norm and
    RoPE also run in the varlen launch) hand the projection's backward its
    five cotangents as column blocks of one buffer (written there by the
    RoPE and attention backward kernels), so that it runs one dx and one dW
    GEMM; the gradients of x and of every parameter equal those of the path
    with separate gradient tensors (bf16 GEMM rounding apart)."""
    import numpy as np
    torch.manual_seed(12)
    lens = [37, 200, 1, 90, 128]
    T = sum(lens)
    cu = torch.tensor([0] + list(np.cumsum(lens)), dtype=torch.int32, device=gpu)
    shape = (T, 512) if packed else (3, 150, 512)
    x0 = torch.randn(*shape, device=gpu, dtype=torch.bfloat16)
    g = torch.randn(*shape, device=gpu, dtype=torch.bfloat16)
    seen = []
    real = A._column_blocks

    def recording(gs, sizes):
        r = real(gs, sizes)
        seen.append(r is not None)
        return r

    monkeypatch.setattr(A, "_column_blocks", recording)

    def run(slab):
        monkeypatch.setattr(A.NaylisAttention, "_grad_slab", slab)
        torch.manual_seed(3)
        m = A.NaylisAttention(512, 4, n_kv_heads=2, rel_rank=32, vanilla_heads=1).to(
            device=gpu, dtype=torch.bfloat16)
        m._use_fna2 = True
        with torch.no_grad():
            m.graph_scale.uniform_(0.5, 1.5)
        x = x0.clone().requires_grad_(True)
        if packed:
            y, _ = m(x, cu_seqlens_q=cu, cu_seqlens_k=cu, max_seqlen_q=200, max_seqlen_k=200)
        else:
            y, _ = m(x)
        y.backward(g)
        torch.cuda.synchronize()
        return [x.grad] + [p.grad for _, p in m.named_parameters()]

    seen.clear()
    with_slab = run(True)
    assert seen and all(seen), seen  # one buffer: the one-GEMM backward ran
    seen.clear()
    without = run(False)
    assert seen and not any(seen), seen
    for a, b in zip(with_slab, without):
        assert (a is None) == (b is None)
        if a is not None:
            rel = ((a.float() - b.float()).norm() / b.float().norm().clamp_min(1e-6)).item()
            assert rel < 2e-2, rel


def test_grad_slab_blocks_and_second_pass():
    """GradSlab blocks are column views of one buffer; asking for a block
    again (a second backward) starts a new buffer, leaving the views already
    handed out untouched."""
    s = A.GradSlab(5, [8, 4, 4], torch.float32, "cpu")
    y = torch.zeros(5, 16)  # the projection's output geometry
    q, v = y[:, :8].view(5, 2, 4), y[:, 12:]
    a0, a1 = s.block(0, q), s.block(2, v)
    assert a0.shape == q.shape and a0.stride() == q.stride() and a1.stride() == v.stride()
    assert a0.untyped_storage().data_ptr() == a1.untyped_storage().data_ptr()
    assert a1.storage_offset() - a0.storage_offset() == 12
    a0.fill_(1.0)
    b0 = s.block(0, (q.shape, q.stride()))  # a second pass
    assert b0.untyped_storage().data_ptr() != a0.untyped_storage().data_ptr()
    b0.fill_(2.0)
    assert torch.all(a0 == 1.0)
    blocks = [s.block(1, y[:, 8:12]), s.block(2, v)]
    assert A._column_blocks([b0.view(5, 8)] + blocks, [8, 4, 4]) is not None
    # a transposed [B, H, S, D] view (the dense path) keeps its strides
    yd = torch.zeros(2, 3, 16)  # B = 2, S = 3
    kd = yd[..., 8:12].view(2, 3, 2, 2).transpose(1, 2)
    sd = A.GradSlab(6, [8, 4, 4], torch.float32, "cpu")
    gk = sd.block(1, kd)
    assert gk.shape == kd.shape and gk.stride() == kd.stride()
    # a layout that is not a column block (here a contiguous tensor, which
    # would spill into the next blocks) gets a tensor of its own
    c = torch.zeros(6, 2, 2)
    gc = sd.block(1, c)
    assert gc.untyped_storage().data_ptr() != gk.untyped_storage().data_ptr()
    assert A._block_layout(kd.shape, kd.stride(), 4, 16, 6)
    assert not A._block_layout(c.shape, c.stride(), 4, 16, 6)


def test_stacked_projection_gradient_paths_agree():
    """Backward of the one-GEMM projection: incoming gradients that are
    consecutive column blocks of one buffer take one dx GEMM; separate ones
    take per-block GEMMs accumulated in place.  Both give the same dx and
    dW (each dW a row view of one buffer)."""
    torch.manual_seed(9)
    m = A.NaylisAttention(64, 4, n_kv_heads=2, rel_rank=8)
    ws = m._projection_weights()
    sizes = [64, 32, 32, 32, 32]
    x = torch.randn(7, 64, requires_grad=True)
    w_all = m._pack_projection_weights()
    outs = A._StackedProjection.apply(x, w_all, sizes, *ws)
    g_all = torch.randn(7, sum(sizes))
    blocks = list(torch.split(g_all, sizes, dim=-1))
    assert A._column_blocks(blocks, sizes) is not None
    g1 = torch.autograd.grad(outs, [x, *ws], blocks, retain_graph=True)
    sep = [b.clone() for b in blocks]
    assert A._column_blocks(sep, sizes) is None
    g2 = torch.autograd.grad(outs, [x, *ws], sep)
    for a, b in zip(g1, g2):
        torch.testing.assert_close(a, b, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(g1[0], g_all @ w_all, rtol=1e-5, atol=1e-5)
    torch.testing.assert_close(torch.cat(g1[1:]), g_all.t() @ x.detach(), rtol=1e-5, atol=1e-5)


def test_stacked_projection_under_autocast_with_fp32_params():
    """Mixed precision: fp32 parameters under autocast(bf16).  The one-GEMM
    projection runs in bf16 as F.linear does; its backward returns dx in x's
    dtype and dW in the weights' dtype, equal to five autocast nn.Linear
    projections' gradients."""
    torch.manual_seed(12)
    m = A.NaylisAttention(64, 4, n_kv_heads=2, rel_rank=8)
    ref = copy.deepcopy(m)
    x = torch.randn(2, 6, 64)
    sizes = [64, 32, 32, 32, 32]
    cot = [torch.randn(12, n) for n in sizes]
    x1 = x.clone().requires_grad_(True)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        outs = A._StackedProjection.apply(x1, m._pack_projection_weights(), sizes,
                                          *m._projection_weights())
    assert all(o.dtype == torch.bfloat16 for o in outs)
    loss1 = sum((o.reshape(12, -1).float() * c).sum() for o, c in zip(outs, cot))
    g1 = torch.autograd.grad(loss1, [x1, *m._projection_weights()])
    assert g1[0].dtype == torch.float32 and all(g.dtype == torch.float32 for g in g1[1:])

    x2 = x.clone().requires_grad_(True)
    mods = [ref.q_proj, ref.k_proj, ref.v_proj, ref.rel_q_proj, ref.rel_k_proj]
    with torch.autocast("cpu", dtype=torch.bfloat16):
        sep = [mod(x2) for mod in mods]
    loss2 = sum((o.reshape(12, -1).float() * c).sum() for o, c in zip(sep, cot))
    g2 = torch.autograd.grad(loss2, [x2, *ref._projection_weights()])
    for a, b in zip(g1, g2):
        torch.testing.assert_close(a, b, rtol=2e-2, atol=2e-2)

    # the module's forward + backward under autocast with fp32 params
    m2 = copy.deepcopy(ref)
    with torch.autocast("cpu", dtype=torch.bfloat16):
        y = m2(x.clone().requires_grad_(True))[0]
    y.float().sum().backward()
    assert all(p.grad is not None and p.grad.dtype == torch.float32
               for p in m2._projection_weights())


def test_stacked_projection_frozen_and_unused_weights():
    """As for nn.Linear: a frozen weight gets no gradient (no dW GEMM), and a
    block whose output does not reach the loss gets None, not zeros."""
    torch.manual_seed(13)
    m = A.NaylisAttention(64, 4, n_kv_heads=2, rel_rank=8)
    ws = m._projection_weights()
    ws[1].requires_grad_(False)  # k_proj frozen
    sizes = [64, 32, 32, 32, 32]
    x = torch.randn(5, 64, requires_grad=True)
    outs = A._StackedProjection.apply(x, m._pack_projection_weights(), sizes, *ws)
    loss = outs[0].sum() + outs[1].sum() + outs[2].sum() + outs[3].sum()  # rel_k unused
    loss.backward()
    assert ws[1].grad is None
    assert ws[4].grad is None
    for i in (0, 2, 3):
        torch.testing.assert_close(ws[i].grad, torch.ones(5, sizes[i]).t() @ x.detach(),
                                   rtol=1e-5, atol=1e-5)
    w_all = m._pack_projection_weights()
    torch.testing.assert_close(x.grad, torch.ones(5, 160) @ w_all[:160], rtol=1e-5, atol=1e-5)
