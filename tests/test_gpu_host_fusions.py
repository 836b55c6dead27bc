"""GPU checks of the decoder hosts' fused elementwise passes.

Kernels:
* ``ops.add_rms_norm``: a block's residual add with the RMSNorm that reads its result
  (``gdn2_add_rms_norm_fwd``);
* ``ops.silu_mul``: SwiGLU's ``silu(a) * b`` on the fused w1 / w2 projection
  (``gdn2_silu_mul_fwd``);
* ``ops.linear``: the linear layers of a decode step, at most 8 rows
  (``gdn2_skinny_linear``).

Checks:
* **Two ops = one pass.** ``add_rms_norm`` against torch's add followed by the unfused
  norm entry point (``ops.rms_norm``), bit for bit, for both outputs, in bf16, fp16 and
  fp32, with an fp32 weight, and on row counts that leave a workgroup part-filled.
* **Reference rounding.** Both kernels against the reference's torch formulas evaluated
  in the io dtype (``models/normalization.py:48-50``, ``gdn2_gpt/model.py:74-77``).
* **Oracle.** ``add_rms_norm`` against the float64 oracle of the RMSNorm on the rounded sum.
* **Model.** The config-3 host's forward with the fused passes against the same model
  with them switched off, bit for bit, uncached and on a cached decode step.
* **Few-row linear.** Against the fp32 product rounded once and against torch's GEMM in
  the io dtype: equal up to one unit in the last place (a different fp32 summation
  order); strided rows, leading batch axes, fallbacks to torch's GEMM (more than 8 rows,
  unsupported K, fp32, autograd) and graph replays.
* **Attention decode** (``ops.attention_decode``, ``gdn2_attn_decode``): against float64
  attention over the same rounded inputs (GQA, D = 64 and 128, first and last cache
  position), the cache rows it stores, an out-of-range position, and the host's
  attention layer against its torch path.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rel_l2

pytestmark = pytest.mark.gpu


def _bits_equal(a: torch.Tensor, b: torch.Tensor) -> None:
    assert a.dtype == b.dtype and a.shape == b.shape
    diff = (a != b) & ~(torch.isnan(a) & torch.isnan(b))
    assert not bool(diff.any()), f"{int(diff.sum())} of {a.numel()} elements differ"


@pytest.mark.parametrize("dtype,N,rows", [(torch.bfloat16, 1024, 37 * 5), (torch.bfloat16, 2048, 3),
                                          (torch.bfloat16, 64, 1001), (torch.float16, 512, 65),
                                          (torch.float32, 1024, 130), (torch.float32, 16, 7)])
def test_add_rms_norm_equals_add_then_norm(gpu_device, dtype, N, rows):
    from qwendopamine_amd.ops import add_rms_norm, rms_norm

    print(f"[case] add_rms_norm dtype={dtype} N={N} rows={rows}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(N + rows)
    x = (torch.randn(rows, N, generator=g) * 2).to(gpu_device, dtype)
    h = (torch.randn(rows, N, generator=g) * 0.5).to(gpu_device, dtype)
    w = torch.randn(N, generator=g).to(gpu_device, dtype)
    s, out = add_rms_norm(x, h, w, 1e-5)
    s_ref = x + h
    out_ref = rms_norm(s_ref, w, 1e-5)
    torch.cuda.synchronize()
    _bits_equal(s, s_ref)
    _bits_equal(out, out_ref)
    ref = orc.rmsnorm(s_ref.double().cpu().numpy(), w.double().cpu().numpy(), 1e-5)
    assert rel_l2(out, ref) <= REL_TOL[dtype]
    if dtype != torch.float32:
        s32, out32 = add_rms_norm(x, h, w.float(), 1e-5)
        ref32 = rms_norm(s_ref, w.float(), 1e-5)
        torch.cuda.synchronize()
        assert out32.dtype == torch.float32
        _bits_equal(s32, s_ref)
        _bits_equal(out32, ref32)


def test_add_rms_norm_rounds_like_the_reference(gpu_device):
    """``x = x + h; norm_2(x)`` of reference Block.forward in bf16 by torch against the pass."""
    from qwendopamine_amd.ops import add_rms_norm

    print("[case] add_rms_norm reference rounding", flush=True)
    torch.manual_seed(5)
    x = torch.randn(4, 300, 1024, device=gpu_device, dtype=torch.bfloat16) * 3
    h = torch.randn(4, 300, 1024, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(1024, device=gpu_device, dtype=torch.bfloat16)
    s, out = add_rms_norm(x, h, w, 1e-5)
    xs = x + h
    ref = w * (xs * torch.rsqrt(xs.pow(2).mean(-1, keepdim=True) + 1e-5))
    torch.cuda.synchronize()
    _bits_equal(s, xs)
    a, b = out.float(), ref.float()
    same = (a == b).float().mean().item()
    worst = ((a - b).abs() / (b.abs() + 1e-2)).max().item()
    print(f"  bit-identical {same:.5f}, worst relative diff {worst:.2e}", flush=True)
    assert same >= 0.99 and worst <= 2.0 ** -7


def test_add_rms_norm_rejects(gpu_device):
    from qwendopamine_amd.ops import add_rms_norm, add_rms_norm_supported

    print("[case] add_rms_norm rejects", flush=True)
    x = torch.zeros(4, 1000, device=gpu_device, dtype=torch.bfloat16)
    assert not add_rms_norm_supported(x)
    with pytest.raises(NotImplementedError):
        add_rms_norm(x, x, torch.ones(1000, device=gpu_device, dtype=torch.bfloat16))
    y = torch.zeros(4, 1024, device=gpu_device, dtype=torch.bfloat16)
    assert add_rms_norm_supported(y)
    with pytest.raises(ValueError):
        add_rms_norm(y, y[:, :512], torch.ones(1024, device=gpu_device, dtype=torch.bfloat16))


@pytest.mark.parametrize("dtype,H,rows", [(torch.bfloat16, 3072, 17), (torch.bfloat16, 512, 1000),
                                          (torch.float16, 64, 3), (torch.float32, 3072, 5)])
def test_silu_mul_matches_torch(gpu_device, dtype, H, rows):
    """Against ``F.silu(a) * b`` in the io dtype: the same two roundings.  torch's silu
    and the kernel's both evaluate x / (1 + exp(-x)) in float, so the rounded results
    agree except where the two float exps differ in the last bit across a rounding
    boundary: at most one unit in the last place of the io dtype, on a tiny share."""
    from qwendopamine_amd.ops import silu_mul

    print(f"[case] silu_mul dtype={dtype} H={H} rows={rows}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(H + rows)
    ab = (torch.randn(rows, 2 * H, generator=g) * 3).to(gpu_device, dtype)
    out = silu_mul(ab)
    a, b = ab.chunk(2, dim=-1)
    ref = F.silu(a) * b
    torch.cuda.synchronize()
    assert out.dtype == dtype and out.shape == (rows, H)
    o, r = out.float(), ref.float()
    same = (o == r).float().mean().item()
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10, torch.float32: 2.0 ** -22}[dtype]
    worst = ((o - r).abs() / (r.abs() + 1e-6)).max().item()
    print(f"  bit-identical {same:.6f}, worst relative diff {worst:.2e}", flush=True)
    assert same >= 0.999
    assert worst <= ulp
    # Strided rows: a column range of a wider row, as a fused projection with a bias-free
    # third block would hand over.
    wide = torch.randn(rows, 2 * H + 64, generator=g).to(gpu_device, dtype)
    view = wide[:, : 2 * H]
    torch.cuda.synchronize()
    _bits_equal(silu_mul(view), silu_mul(view.contiguous()))


def _small(dtype, dev):
    from qwendopamine_amd.hybrid import HybridConfig, HybridDecoder

    torch.manual_seed(0)
    cfg = HybridConfig(n_layer=4, n_embd=256, n_head=4, head_size=64, n_query_groups=2,
                       intermediate_size=512, vocab_size=1000, gdn2_layers=[0, 1, 2], block_size=512)
    return HybridDecoder(cfg).to(dev, dtype).eval()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_hybrid_forward_fused_equals_unfused(gpu_device, dtype, monkeypatch):
    """The host's residual adds fused with the following norms change no bit of the
    logits: uncached, a cached prefill and a cached decode step."""
    from qwendopamine_amd import ops

    print(f"[case] hybrid fused vs unfused host {dtype}", flush=True)
    m = _small(dtype, gpu_device)
    idx = torch.randint(0, 1000, (2, 80), device=gpu_device)

    def run():
        with torch.no_grad():
            full = m(idx)
            m.setup_caches(2, 81)
            pre = m(idx, input_pos=torch.arange(80, device=gpu_device))
            step = m(idx[:, -1:], input_pos=torch.tensor([80], device=gpu_device))
        torch.cuda.synchronize()
        return full, pre, step

    calls = {"n": 0}
    real = ops.add_rms_norm

    def counted(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    monkeypatch.setattr(ops, "add_rms_norm", counted)
    fused = run()
    assert calls["n"] == 3 * 2 * 4  # two per block, three forwards
    monkeypatch.setattr(ops, "add_rms_norm_supported", lambda x: False)
    plain = run()
    for f, p in zip(fused, plain):
        _bits_equal(f, p)


def _ulp_close(y: torch.Tensor, ref: torch.Tensor, dtype) -> None:
    """Two roundings of the same fp32 sums (different summation orders): equal except
    where the orders straddle a rounding boundary, i.e. at most one unit in the last
    place of the io dtype, plus an absolute floor near zero."""
    ulp = {torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}[dtype]
    a, b = y.float(), ref.float()
    scale = b.abs().amax().item()
    worst = ((a - b).abs() / (b.abs() + 1e-3 * scale)).max().item()
    same = (a == b).float().mean().item()
    print(f"  bit-identical {same:.4f}, worst relative diff {worst:.2e}", flush=True)
    assert worst <= ulp
    assert same >= 0.9


@pytest.mark.parametrize("dtype,M,K,N,bias", [(torch.bfloat16, 4, 1024, 6144, False),
                                              (torch.bfloat16, 4, 3072, 1024, False),
                                              (torch.bfloat16, 1, 512, 7, True),
                                              (torch.bfloat16, 4, 4096, 1000, True),
                                              (torch.bfloat16, 8, 2048, 500, True),
                                              (torch.bfloat16, 3, 2048, 129, False),
                                              (torch.float16, 5, 1024, 300, True)])
def test_linear_few_rows_matches_fp32(gpu_device, dtype, M, K, N, bias):
    """``ops.linear`` on the few-row kernel against the fp32 product rounded once, and
    against torch's own GEMM (``F.linear``) in the io dtype."""
    from qwendopamine_amd.ops import linear

    print(f"[case] linear dtype={dtype} M={M} K={K} N={N} bias={bias}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * 7 + K + N)
    x = torch.randn(M, K, generator=g).to(gpu_device, dtype)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(gpu_device, dtype)
    b = torch.randn(N, generator=g).to(gpu_device, dtype) if bias else None
    with torch.no_grad():
        y = linear(x, w, b)
        ref = x.float() @ w.float().t() + (b.float() if bias else 0.0)
        yt = F.linear(x, w, b)
    torch.cuda.synchronize()
    assert y.dtype == dtype and y.shape == (M, N)
    _ulp_close(y, ref.to(dtype), dtype)
    _ulp_close(y, yt, dtype)


def test_linear_strided_rows_and_fallbacks(gpu_device):
    """Rows of x taken from a wider tensor give the contiguous result bit for bit; a
    leading batch shape is kept; more than 8 rows, an unsupported K, fp32, or a gradient
    are torch's GEMM exactly."""
    from qwendopamine_amd.ops import linear

    print("[case] linear strides and fallbacks", flush=True)
    torch.manual_seed(9)
    wide = torch.randn(4, 1024 + 64, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(333, 1024, device=gpu_device, dtype=torch.bfloat16) * 0.03
    with torch.no_grad():
        _bits_equal(linear(wide[:, :1024], w), linear(wide[:, :1024].contiguous(), w))
        x3 = torch.randn(2, 1, 1024, device=gpu_device, dtype=torch.bfloat16)
        y3 = linear(x3, w)
        assert y3.shape == (2, 1, 333)
        _bits_equal(y3.reshape(2, 333), linear(x3.reshape(2, 1024), w))
        for x in (torch.randn(9, 1024, device=gpu_device, dtype=torch.bfloat16),
                  torch.randn(4, 1000, device=gpu_device, dtype=torch.bfloat16)):
            ww = torch.randn(50, x.shape[1], device=gpu_device, dtype=torch.bfloat16)
            _bits_equal(linear(x, ww), F.linear(x, ww))
        x32, w32 = torch.randn(4, 1024, device=gpu_device), torch.randn(50, 1024, device=gpu_device)
        _bits_equal(linear(x32, w32), F.linear(x32, w32))
    xg = torch.randn(4, 1024, device=gpu_device, dtype=torch.bfloat16, requires_grad=True)
    yg = linear(xg, w)
    assert yg.grad_fn is not None
    torch.cuda.synchronize()


def test_linear_graph_replays(gpu_device):
    """Captured in a HIP graph, the few-row product replays to the eager result, with
    new inputs copied in between replays."""
    from qwendopamine_amd.ops import linear

    print("[case] linear graph replays", flush=True)
    torch.manual_seed(11)
    x = torch.randn(4, 1024, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(2048, 1024, device=gpu_device, dtype=torch.bfloat16) * 0.03
    with torch.no_grad():
        linear(x, w)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y = linear(x, w)
        for rep in range(3):
            x.copy_(torch.randn(4, 1024, device=gpu_device, dtype=torch.bfloat16))
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            _bits_equal(y, linear(x, w))


def test_skinny_linear_wide_output_through_the_c_abi(gpu_device):
    """A wide output (more row groups than workgroups: each workgroup loops over groups
    with the next group's rows requested ahead) through the C entry point directly, as
    ``ops.linear`` leaves such widths to torch's GEMM."""
    from qwendopamine_amd import _native as nat

    print("[case] skinny linear wide output (C ABI)", flush=True)
    torch.manual_seed(13)
    M, K, N = 3, 1024, 40000
    x = torch.randn(M, K, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(N, K, device=gpu_device, dtype=torch.bfloat16) * 0.03
    b = torch.randn(N, device=gpu_device, dtype=torch.bfloat16)
    y = torch.empty(M, N, device=gpu_device, dtype=torch.bfloat16)
    lib = nat.load()
    st = lib.gdn2_skinny_linear(nat.ptr(x), K, nat.ptr(w), K, nat.ptr(b), nat.ptr(y), N, nat.DTYPE_BF16, M, N, K,
                                nat.stream_handle(x.device))
    nat.check(st, "gdn2_skinny_linear")
    ref = (x.float() @ w.float().t() + b.float()).to(torch.bfloat16)
    torch.cuda.synchronize()
    _ulp_close(y, ref, torch.bfloat16)
    assert lib.gdn2_skinny_linear(nat.ptr(x), K, nat.ptr(w), K, None, nat.ptr(y), N, nat.DTYPE_F32, M, N, K,
                                  nat.stream_handle(x.device)) == nat.ERR_UNSUPPORTED
    assert lib.gdn2_skinny_linear(nat.ptr(x), K, nat.ptr(w), K, None, nat.ptr(y), N, nat.DTYPE_BF16, 9, N, K,
                                  nat.stream_handle(x.device)) == nat.ERR_UNSUPPORTED


def _attn_reference(qkv, cos, sin, pos, kc, vc, n_head, dtype):
    """float64 attention of one token over cache positions 0..pos, with q and k rotated
    in fp32 and rounded to the io dtype (as the host's torch path and the kernel do);
    returns (out [B, n_head, D], rotated k [B, G, D], v [B, G, D])."""
    B, G, L, D = kc.shape
    qpk = n_head // G
    x = qkv.reshape(B, G, qpk + 2, D).float()
    pairs = cos.shape[-1]
    c, s = cos.reshape(-1).float(), sin.reshape(-1).float()

    def rot(t):
        t = t.clone()
        a, b = t[..., 0:2 * pairs:2].clone(), t[..., 1:2 * pairs:2].clone()
        t[..., 0:2 * pairs:2] = a * c - b * s
        t[..., 1:2 * pairs:2] = a * s + b * c
        return t.to(dtype).double()

    q = rot(x[:, :, :qpk])                       # [B, G, qpk, D]
    k = rot(x[:, :, qpk])                        # [B, G, D]
    v = x[:, :, qpk + 1].to(dtype).double()
    K = kc[:, :, :pos + 1].double().clone()
    V = vc[:, :, :pos + 1].double().clone()
    K[:, :, pos], V[:, :, pos] = k, v
    sc = torch.einsum("bgqd,bgld->bgql", q, K) / math.sqrt(D)
    o = torch.einsum("bgql,bgld->bgqd", torch.softmax(sc, dim=-1), V)
    return o.reshape(B, n_head, D), k, v


@pytest.mark.parametrize("dtype,G,qpk,D,L,pos", [(torch.bfloat16, 16, 1, 64, 2304, 2047),
                                                 (torch.bfloat16, 4, 4, 128, 300, 0),
                                                 (torch.float16, 2, 2, 128, 513, 512),
                                                 (torch.float16, 2, 2, 128, 1025, 1024),
                                                 (torch.bfloat16, 3, 1, 64, 100, 37),
                                                 (torch.bfloat16, 4, 2, 64, 2304, 10)])
def test_attention_decode_matches_float64(gpu_device, dtype, G, qpk, D, L, pos):
    """``ops.attention_decode`` against float64 attention over the same rounded inputs:
    the output to within its io-dtype rounding, the cache rows at ``pos`` equal to the
    rotated k and v, every other cache row untouched.  Caches over 1024 positions split
    the positions over several workgroups (a token early in a long cache leaves most
    splits empty)."""
    from qwendopamine_amd.ops import attention_decode

    print(f"[case] attention_decode dtype={dtype} G={G} qpk={qpk} D={D} L={L} pos={pos}", flush=True)
    gen = torch.Generator(device="cpu").manual_seed(G * 100 + D + pos)
    B, n_head = 3, G * qpk
    qkv = torch.randn(B, 1, G * (qpk + 2) * D, generator=gen).to(gpu_device, dtype)
    kc = torch.randn(B, G, L, D, generator=gen).to(gpu_device, dtype)
    vc = torch.randn(B, G, L, D, generator=gen).to(gpu_device, dtype)
    ang = torch.rand(1, D // 2, generator=gen) * 6.0
    cos, sin = torch.cos(ang).to(gpu_device), torch.sin(ang).to(gpu_device)
    kc0, vc0 = kc.clone(), vc.clone()
    ref, k_ref, v_ref = _attn_reference(qkv.cpu(), cos.cpu(), sin.cpu(), pos, kc0.cpu(), vc0.cpu(), n_head, dtype)
    # The same rotation as row pos of whole tables, which the kernel indexes itself.
    tab_c = torch.randn(L, D // 2, generator=gen).to(gpu_device)
    tab_s = torch.randn(L, D // 2, generator=gen).to(gpu_device)
    tab_c[pos], tab_s[pos] = cos[0], sin[0]
    kc_t, vc_t = kc.clone(), vc.clone()
    with torch.no_grad():
        out = attention_decode(qkv, cos, sin, torch.tensor([pos], device=gpu_device), kc, vc, n_head)
        out_t = attention_decode(qkv, tab_c, tab_s, torch.tensor([pos], device=gpu_device), kc_t, vc_t, n_head)
    torch.cuda.synchronize()
    assert torch.equal(out_t, out) and torch.equal(kc_t, kc) and torch.equal(vc_t, vc)
    assert out.shape == (B, n_head, D) and out.dtype == dtype
    err = rel_l2(out, ref.numpy())
    print(f"  rel_l2 {err:.2e}", flush=True)
    assert err <= 4e-3
    # The rotation in fp32 may contract into fused multiply-adds: a rounding flip to
    # the io dtype is possible, at most one unit in the last place.
    kk = kc[:, :, pos].cpu().double()
    ulp = 2.0 ** -7 if dtype == torch.bfloat16 else 2.0 ** -10
    assert (kk == k_ref).double().mean().item() >= 0.99
    assert ((kk - k_ref).abs() <= ulp * k_ref.abs() + 1e-6).all()
    assert torch.equal(vc[:, :, pos].cpu().double(), v_ref)
    keep = torch.ones(L, dtype=torch.bool)
    keep[pos] = False
    assert torch.equal(kc[:, :, keep], kc0[:, :, keep]) and torch.equal(vc[:, :, keep], vc0[:, :, keep])


def test_attention_decode_out_of_range_position(gpu_device):
    """A position outside the caches writes zeros and leaves the caches alone."""
    from qwendopamine_amd.ops import attention_decode

    print("[case] attention_decode out-of-range position", flush=True)
    torch.manual_seed(17)
    B, G, L, D = 2, 4, 64, 64
    qkv = torch.randn(B, 1, G * 3 * D, device=gpu_device, dtype=torch.bfloat16)
    kc = torch.randn(B, G, L, D, device=gpu_device, dtype=torch.bfloat16)
    vc = torch.randn_like(kc)
    kc0, vc0 = kc.clone(), vc.clone()
    cos, sin = torch.ones(1, D // 2, device=gpu_device), torch.zeros(1, D // 2, device=gpu_device)
    with torch.no_grad():
        out = attention_decode(qkv, cos, sin, torch.tensor([L], device=gpu_device), kc, vc, G)
    torch.cuda.synchronize()
    assert not bool(out.any())
    assert torch.equal(kc, kc0) and torch.equal(vc, vc0)


def test_hybrid_attention_layer_fused_vs_torch_path(gpu_device, monkeypatch):
    """The host's attention layer on one cached token: the fused launch against the
    layer's torch path (RoPE, cache update, masked softmax) on the same state: caches
    equal, outputs equal to the torch path's rounding of scores and probabilities."""
    from qwendopamine_amd import ops
    from qwendopamine_amd.hybrid import CausalSelfAttention, HybridConfig

    print("[case] hybrid attention layer fused vs torch path", flush=True)
    torch.manual_seed(19)
    cfg = HybridConfig(n_layer=1, n_embd=1024, n_head=16, head_size=64, n_query_groups=8, gdn2_layers=[])
    att = CausalSelfAttention(cfg, 0).to(gpu_device, torch.bfloat16).eval()
    B, L, pos = 4, 400, 311
    x = torch.randn(B, 1, 1024, device=gpu_device, dtype=torch.bfloat16)
    from qwendopamine_amd.hybrid import build_rope_cache
    cos_t, sin_t = build_rope_cache(L, 64, gpu_device)
    ip = torch.tensor([pos], device=gpu_device)
    cos, sin = cos_t.index_select(0, ip), sin_t.index_select(0, ip)
    mask = torch.tril(torch.ones(L, L, dtype=torch.bool, device=gpu_device))[None, None].index_select(2, ip)
    base = (torch.randn(B, 8, L, 64, device=gpu_device, dtype=torch.bfloat16),
            torch.randn(B, 8, L, 64, device=gpu_device, dtype=torch.bfloat16))
    outs, caches = [], []
    for fused in (True, False):
        if not fused:
            monkeypatch.setattr(ops, "attention_decode_supported", lambda *a: False)
        att.kv_cache = (base[0].clone(), base[1].clone())
        with torch.no_grad():
            outs.append(att(x, cos, sin, ip, mask))
        caches.append(att.kv_cache)
    torch.cuda.synchronize()
    a, b = outs[0].float(), outs[1].float()
    err = ((a - b).norm() / b.norm()).item()
    print(f"  fused vs torch path rel_l2 {err:.2e}", flush=True)
    assert err <= 1e-2
    for (k0, v0), (k1, v1) in zip([caches[0]], [caches[1]]):
        same = (k0 == k1).float().mean().item()
        assert same >= 0.999 and torch.equal(v0, v1)


@pytest.mark.parametrize("dtype,M,K,N0,N1", [(torch.bfloat16, 4, 64, 1024, 1024), (torch.bfloat16, 8, 128, 300, 77),
                                             (torch.float16, 4, 32, 64, 1000), (torch.bfloat16, 1, 256, 5, 4096)])
def test_linear_pair_matches_fp32(gpu_device, dtype, M, K, N0, N1):
    """``ops.linear_pair`` (the module's two second-stage gate projections in one launch)
    against the fp32 products rounded once, with x taken as column ranges of a wider
    row (as the fused input projection hands them over) and a bias on the second."""
    from qwendopamine_amd.ops import linear_pair

    print(f"[case] linear_pair dtype={dtype} M={M} K={K} N=({N0}, {N1})", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M + K + N0 + N1)
    wide = torch.randn(M, 3 * K + 16, generator=g).to(gpu_device, dtype)
    x0, x1 = wide[:, 16:16 + K], wide[:, 16 + K:16 + 2 * K]
    w0 = (torch.randn(N0, K, generator=g) * K ** -0.5).to(gpu_device, dtype)
    w1 = (torch.randn(N1, K, generator=g) * K ** -0.5).to(gpu_device, dtype)
    b1 = torch.randn(N1, generator=g).to(gpu_device, dtype)
    with torch.no_grad():
        y0, y1 = linear_pair(x0, w0, None, x1, w1, b1)
    r0 = (x0.float() @ w0.float().t()).to(dtype)
    r1 = (x1.float() @ w1.float().t() + b1.float()).to(dtype)
    torch.cuda.synchronize()
    assert y0.shape == (M, N0) and y1.shape == (M, N1)
    _ulp_close(y0, r0, dtype)
    _ulp_close(y1, r1, dtype)


def test_linear_pair_fallback(gpu_device):
    """An inner dimension the kernel does not take is torch's GEMMs exactly."""
    from qwendopamine_amd.ops import linear_pair

    print("[case] linear_pair fallback", flush=True)
    torch.manual_seed(23)
    x = torch.randn(4, 48, device=gpu_device, dtype=torch.bfloat16)
    w = torch.randn(100, 48, device=gpu_device, dtype=torch.bfloat16)
    with torch.no_grad():
        y0, y1 = linear_pair(x, w, None, x, w, None)
    _bits_equal(y0, F.linear(x, w))
    _bits_equal(y1, F.linear(x, w))


@pytest.mark.parametrize("dtype,rows,n", [(torch.bfloat16, 4, 151936), (torch.float32, 3, 1000), (torch.float16, 5, 77),
                                          (torch.bfloat16, 2, 8), (torch.float16, 4, 50001), (torch.float32, 2, 151936),
                                          (torch.bfloat16, 4, 400003)])
def test_argmax_rows_matches_torch(gpu_device, dtype, rows, n):
    """Against torch's argmax: ties resolved to the first index (also -0.0 against +0.0),
    NaN as the maximum, -inf rows, rows that take one batch of requests per thread and
    rows that loop over several, ragged tails, a strided row view, and the output
    written in place into a strided int64 column."""
    from qwendopamine_amd.ops import argmax_rows

    print(f"[case] argmax_rows dtype={dtype} rows={rows} n={n}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(rows * n)
    x = torch.randn(rows, n, generator=g).to(gpu_device, dtype)
    x[0, n // 3] = x[0, n // 2] = 100.0               # a tie: the first wins
    if rows > 1:
        x[1, n - 1] = float("nan")                    # NaN is the maximum
        x[1, 1] = float("nan")
    if rows > 2:
        x[2] = x[2].min()                             # all equal: index 0
    if rows > 3:
        x[3] = float("-inf")                          # all -inf: index 0
        x[3, n - 2] = -0.0                            # -0.0 then +0.0: equal, the first wins
        x[3, n - 1] = 0.0
    ref = x.argmax(-1, keepdim=True)
    got = argmax_rows(x)
    got_one = argmax_rows(x, split=False)             # one workgroup per row
    wide = torch.zeros(rows, 3, dtype=torch.int64, device=gpu_device)
    argmax_rows(x, out=wide[:, 1:2])
    big = torch.randn(rows, 2, n, generator=g).to(gpu_device, dtype)
    torch.cuda.synchronize()
    assert torch.equal(got, ref), (got.flatten().tolist(), ref.flatten().tolist())
    assert torch.equal(got_one, ref), (got_one.flatten().tolist(), ref.flatten().tolist())
    assert torch.equal(wide[:, 1:2], ref) and not bool(wide[:, 0].any()) and not bool(wide[:, 2].any())
    assert torch.equal(argmax_rows(big[:, 1]), big[:, 1].argmax(-1, keepdim=True))


@pytest.mark.parametrize("dtype,M,K,N", [(torch.bfloat16, 4, 1024, 6144), (torch.bfloat16, 1, 512, 100),
                                         (torch.float16, 3, 2048, 704), (torch.bfloat16, 5, 1024, 64),
                                         (torch.bfloat16, 2, 1024, 4112)])
def test_linear_addnorm_equals_add_norm_then_linear(gpu_device, dtype, M, K, N):
    """The residual add and RMSNorm formed while the few-row kernel stages its input:
    bit for bit ``add_rms_norm`` followed by ``linear`` for both outputs (the product
    and the residual sums); 5 rows run the two ops."""
    from qwendopamine_amd.ops import add_rms_norm, linear, linear_addnorm, silu_mul

    print(f"[case] linear_addnorm dtype={dtype} M={M} K={K} N={N}", flush=True)
    g = torch.Generator(device="cpu").manual_seed(M * K + N)
    x = (torch.randn(M, K, generator=g) * 2).to(gpu_device, dtype)
    h = torch.randn(M, K, generator=g).to(gpu_device, dtype)
    nw = (1 + 0.1 * torch.randn(K, generator=g)).to(gpu_device, dtype)
    w = (torch.randn(N, K, generator=g) * K ** -0.5).to(gpu_device, dtype)
    with torch.no_grad():
        y, s = linear_addnorm(x, h, nw, 1e-5, w)
        s_ref, n_ref = add_rms_norm(x, h, nw, 1e-5)
        y_ref = linear(n_ref, w)
        # SwiGLU epilogue (w as a stacked [w1; w2]): silu_mul of the same product
        # (where silu_mul's 16-byte pieces cover the width).
        yg, sg = linear_addnorm(x, h, nw, 1e-5, w, swiglu=True)
        yg_ref = silu_mul(y_ref) if (N // 2) % 8 == 0 else None
    torch.cuda.synchronize()
    _bits_equal(s, s_ref)
    _bits_equal(y, y_ref)
    _bits_equal(sg, s_ref)
    assert yg.shape == (M, N // 2)
    if yg_ref is not None:
        _bits_equal(yg, yg_ref)


def test_hybrid_decode_with_norm_in_projection(gpu_device, monkeypatch):
    """A bf16 host whose width the add-and-norm staging takes (512): decode-step logits
    with the fused passes equal the unfused host's bit for bit."""
    from qwendopamine_amd import ops
    from qwendopamine_amd.hybrid import HybridConfig, HybridDecoder

    print("[case] hybrid decode with the norm in the w1|w2 projection", flush=True)
    torch.manual_seed(29)
    cfg = HybridConfig(n_layer=3, n_embd=512, n_head=8, head_size=64, n_query_groups=4, intermediate_size=1024,
                       vocab_size=1000, gdn2_layers=[0, 1], block_size=256)
    m = HybridDecoder(cfg).to(gpu_device, torch.bfloat16).eval()
    idx = torch.randint(0, 1000, (3, 40), device=gpu_device)
    calls = {"n": 0}
    real = ops.linear_addnorm

    def counted(*a, **k):
        calls["n"] += 1
        return real(*a, **k)

    def run():
        with torch.no_grad():
            m.setup_caches(3, 42)
            m(idx, input_pos=torch.arange(40, device=gpu_device))
            out = [m(idx[:, -1:], input_pos=torch.tensor([40 + i], device=gpu_device)) for i in range(2)]
        torch.cuda.synchronize()
        return out

    monkeypatch.setattr(ops, "linear_addnorm", counted)
    fused = run()
    # Per decode step: norm_2 of each of the 3 blocks, and norm_1 of blocks 1 (gdn2)
    # and 2 (attention); block 0's norm_1 has no pending add.
    assert calls["n"] == 2 * (3 + 2)
    monkeypatch.setattr(ops, "add_rms_norm_supported", lambda x: False)
    plain = run()
    for f, p in zip(fused, plain):
        _bits_equal(f, p)
