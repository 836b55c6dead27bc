"""GPU parity of the HIP ops against the oracle on the committed golden fixtures,
at config 0, at the BASELINE full sizes, and for the two API variants that
change the arithmetic (negative eigenvalues, the bounded gate).

* Config 0 (fp32, B1 T512 H4 K=V=64, seed 0): both ops against the float64
  oracle and against ``tests/golden/gdn2_config0_fingerprint.npz``, at the
  fp32 bar (rel. L2 <= 1e-4).
* Golden fixtures (forward with a state, varlen with an empty sequence,
  backward with state gradients): through the HIP ops in fp32, at 1e-4.
* Full size, against the pinned float32 C port of the recurrence
  (``oracle/gdn2_cpu.c``, equal to the float64 oracle to 1e-5) on the same
  bf16-rounded inputs: config 1 (o and final state), config 2 (1024 in-place
  decode steps from the N(0, 0.02) state), config 4's forward, and config 4's
  backward on two (sequence, head) slices against the float64 oracle VJP.
  bf16 bar: rel. L2 <= 2e-2.
* ``allow_neg_eigval`` (b in [0, 2], reference ``gdn2.py:865-866``) and the
  bounded gate ``lower_bound * sigmoid(exp(A_log) (g + dt_bias))``
  (``safe_gate``, reference ``chunk_gdn2.py:1368-1376``, kernel form
  ``fused_recurrent_gdn2.py:266-268``) in both ops, forward and backward.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden"
NAMES = ("q", "k", "v", "g", "b", "w")


def _dev(x, dev, dt=torch.float32):
    return torch.from_numpy(np.ascontiguousarray(x)).to(dt).to(dev)


# --------------------------------------------------------------------- config 0
def test_config0_fp32_both_ops(gpu_device):
    """BASELINE config 0 on the HIP path in fp32, at the 1e-4 bar end to end."""
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    print("[case] config 0 fp32 B1 T512 H4 K=V=64, chunk and token-serial ops", flush=True)
    inp = orc.make_inputs(0, 1, 512, 4, 64, 64)
    fx = np.load(GOLDEN / "gdn2_config0_fingerprint.npz")
    sums = np.array([float(np.sum(inp[n])) for n in NAMES])
    np.testing.assert_allclose(sums, fx["input_sums"], rtol=1e-12, atol=1e-9)
    t = {n: _dev(inp[n], gpu_device) for n in NAMES}
    r = {n: t[n].double().cpu().numpy() for n in NAMES}
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES))
    with torch.no_grad():
        outs = {
            "chunk": chunk_gdn2(*(t[n] for n in NAMES), output_final_state=True,
                                use_qk_l2norm_in_kernel=True),
            "recurrent": fused_recurrent_gdn2(*(t[n] for n in NAMES), output_final_state=True,
                                              use_qk_l2norm_in_kernel=True),
        }
    torch.cuda.synchronize()
    for name, (o, ht) in outs.items():
        assert o.dtype == torch.float32 and ht.dtype == torch.float32
        o64, s64 = o.double().cpu().numpy(), ht.double().cpu().numpy()
        errs = dict(
            o=rel_l2(o64, o_ref), state=rel_l2(s64, s_ref),
            fx_ht=rel_l2(s64, fx["ht"]), fx_o=rel_l2(o64[0, :64, 0], fx["o_head0_first64"]),
            fx_tok=rel_l2(np.linalg.norm(o64[0], axis=(1, 2)), fx["o_token_norms"]),
        )
        print(f"  {name}: " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
        for k, e in errs.items():
            assert e <= 1e-4, (name, k, e)
        assert abs(np.linalg.norm(o64) / float(fx["o_norm"]) - 1.0) <= 1e-4


# ------------------------------------------------------------- golden fixtures
@pytest.mark.parametrize("op", ["chunk", "recurrent"])
def test_golden_forward_fixture(gpu_device, op):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    print(f"[case] golden forward fixture T100 H2 K32 V16 via {op}", flush=True)
    fx = np.load(GOLDEN / "gdn2_fwd_T100_H2_K32_V16.npz")
    t = {n: _dev(fx[n], gpu_device) for n in (*NAMES, "h0")}
    fn = chunk_gdn2 if op == "chunk" else fused_recurrent_gdn2
    with torch.no_grad():
        o, ht = fn(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                   use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    eo, es = rel_l2(o, fx["o"]), rel_l2(ht, fx["ht"])
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-4 and es <= 1e-4


@pytest.mark.parametrize("op", ["chunk", "recurrent"])
def test_golden_varlen_fixture(gpu_device, op):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    print(f"[case] golden varlen fixture T90 N4 via {op}", flush=True)
    fx = np.load(GOLDEN / "gdn2_varlen_T90_N4.npz")
    t = {n: _dev(fx[n], gpu_device) for n in (*NAMES, "h0")}
    cu = torch.tensor(fx["cu_seqlens"], dtype=torch.int64, device=gpu_device)
    fn = chunk_gdn2 if op == "chunk" else fused_recurrent_gdn2
    with torch.no_grad():
        o, ht = fn(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                   use_qk_l2norm_in_kernel=True, cu_seqlens=cu)
    torch.cuda.synchronize()
    eo, es = rel_l2(o, fx["o"]), rel_l2(ht, fx["ht"])
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-4 and es <= 1e-4
    # the empty sequence (cu 40 -> 40) hands its initial state through unchanged
    assert torch.equal(ht[2], t["h0"][2])


def test_golden_backward_fixture(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] golden backward fixture T24 H2 K8 V8 via chunk autograd", flush=True)
    fx = np.load(GOLDEN / "gdn2_bwd_T24_H2_K8_V8.npz")
    leaves = {n: _dev(fx[n], gpu_device).requires_grad_(True) for n in (*NAMES, "h0")}
    o, ht = chunk_gdn2(*(leaves[n] for n in NAMES), initial_state=leaves["h0"],
                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    ((o * _dev(fx["do"], gpu_device)).sum() + (ht * _dev(fx["dht"], gpu_device)).sum()).backward()
    torch.cuda.synchronize()
    errs = {f"d{n}": rel_l2(leaves[n].grad, fx[f"d{n}"]) for n in (*NAMES, "h0")}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= 1e-4, (k, e)


# ------------------------------------------------------------------ full sizes
def _bf16_inputs(dev, B, T, H, K, V, seed):
    """BASELINE recipe on the device (scalar beta and g per (b, t, h), broadcast)."""
    gen = torch.Generator(device=dev).manual_seed(seed)
    q = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    k = F.normalize(torch.randn(B, T, H, K, generator=gen, device=dev), dim=-1).to(torch.bfloat16)
    v = torch.randn(B, T, H, V, generator=gen, device=dev).to(torch.bfloat16)
    beta = torch.sigmoid(torch.randn(B, T, H, 1, generator=gen, device=dev))
    g = (-F.softplus(torch.randn(B, T, H, 1, generator=gen, device=dev) + 2.0)).expand(B, T, H, K).contiguous()
    b = beta.expand(B, T, H, K).to(torch.bfloat16).contiguous()
    w = beta.expand(B, T, H, V).to(torch.bfloat16).contiguous()
    return q, k, v, g, b, w


def _c_port(tensors, h0=None):
    """The float32 C port of the recurrence on the host cores, same (rounded) inputs."""
    from oracle import cpu_lib

    arrs = [x.float().cpu().numpy() for x in tensors]
    h = None if h0 is None else h0.float().cpu().numpy()
    return cpu_lib.recurrent_fwd_f32(*arrs, h0=h)


@pytest.mark.parametrize("shape", [(8, 4096, 16, 128, 128), (4, 8192, 16, 128, 128)], ids=["C1", "C4fwd"])
def test_full_size_chunk_vs_c_port(gpu_device, shape):
    from qwendopamine_amd.ops import chunk_gdn2

    B, T, H, K, V = shape
    print(f"[case] full-size chunk op vs float32 C port {shape} bf16", flush=True)
    x = _bf16_inputs(gpu_device, B, T, H, K, V, seed=11)
    with torch.no_grad():
        o, ht = chunk_gdn2(*x, output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = _c_port(x)
    eo, es = rel_l2(o.float().cpu().numpy(), o_ref), rel_l2(ht.cpu().numpy(), s_ref)
    print(f"  rel_l2 o={eo:.3e} state={es:.3e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2
    assert torch.isfinite(o.float()).all()


def test_full_size_decode_loop_vs_c_port(gpu_device):
    """Config 2: 1024 in-place decode steps on [64, 16, 128, 128] vs the C port over the same tokens."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2_fwd

    N, H, K, V, T = 64, 16, 128, 128, 1024
    print("[case] config 2: 1024 decode steps vs float32 C port", flush=True)
    x = _bf16_inputs(gpu_device, N, T, H, K, V, seed=12)
    gen = torch.Generator(device=gpu_device).manual_seed(13)
    h0 = torch.randn(N, H, K, V, generator=gen, device=gpu_device) * 0.02
    state = h0.clone()
    outs = torch.empty(N, T, H, V, dtype=torch.bfloat16, device=gpu_device)
    for t in range(T):
        o_t, _ = fused_recurrent_gdn2_fwd(*(a[:, t:t + 1] for a in x), initial_state=state,
                                          inplace_final_state=True, use_qk_l2norm_in_kernel=True)
        outs[:, t:t + 1] = o_t
        if t % 256 == 255:
            print(f"  step {t + 1}", flush=True)
    torch.cuda.synchronize()
    o_ref, s_ref = _c_port(x, h0)
    eo, es = rel_l2(outs.float().cpu().numpy(), o_ref), rel_l2(state.cpu().numpy(), s_ref)
    print(f"  rel_l2 o={eo:.3e} state={es:.3e}", flush=True)
    assert eo <= 2e-2 and es <= 2e-2


def test_full_size_backward_slices_vs_oracle_vjp(gpu_device):
    """Config 4 fwd + bwd in bf16 on the whole batch; two (sequence, head) slices of
    every gradient against the float64 oracle VJP over the full T = 8192."""
    from qwendopamine_amd.ops import chunk_gdn2

    B, T, H, K, V = 4, 8192, 16, 128, 128
    print("[case] config 4 backward, slices (0,3) and (3,12) vs float64 VJP", flush=True)
    x = _bf16_inputs(gpu_device, B, T, H, K, V, seed=14)
    gen = torch.Generator(device=gpu_device).manual_seed(15)
    do = torch.randn(B, T, H, V, generator=gen, device=gpu_device).to(torch.bfloat16)
    leaves = [a.detach().requires_grad_(True) for a in x]
    o, _ = chunk_gdn2(*leaves, use_qk_l2norm_in_kernel=True)
    (o.float() * do.float()).sum().backward()
    torch.cuda.synchronize()
    for bi, h in ((0, 3), (3, 12)):
        r = [a[bi:bi + 1, :, h:h + 1].double().cpu().numpy() for a in x]
        dr = do[bi:bi + 1, :, h:h + 1].double().cpu().numpy()
        ref = orc.recurrent_vjp(*r, dr)
        got = [lf.grad[bi:bi + 1, :, h:h + 1].double().cpu().numpy() for lf in leaves]
        errs = {f"d{n}": rel_l2(gv, rv) for n, gv, rv in zip(NAMES, got, ref)}
        # the scalar gates of the recipe: dbeta = sum_K db + sum_V dw, dg = sum_K dg
        errs["dbeta"] = rel_l2(got[4].sum(-1) + got[5].sum(-1), ref[4].sum(-1) + ref[5].sum(-1))
        errs["dg_scalar"] = rel_l2(got[3].sum(-1), ref[3].sum(-1))
        print(f"  slice ({bi},{h}) " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
        for k, e in errs.items():
            assert e <= 2e-2, (bi, h, k, e)


# ------------------------------------------- negative eigenvalues, bounded gate
def _neg_eig_inputs(B, T, H, K, V, seed, decay="paper"):
    inp = rand_inputs(B, T, H, K, V, seed=seed, decay=decay)
    inp["b"] = 2.0 * inp["b"]  # b = 2 sigmoid(.) in [0, 2] (gdn2.py:865-866)
    return inp


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("op,T,decay", [("chunk", 200, "paper"), ("chunk", 128, "extreme"),
                                        ("recurrent", 37, "paper"), ("recurrent", 1, "paper")])
def test_allow_neg_eigval_forward(gpu_device, dtype, op, T, decay):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    print(f"[case] allow_neg_eigval forward {op} T={T} {decay} {dtype}", flush=True)
    K = V = 128 if T == 1 else 64
    inp = _neg_eig_inputs(3 if T == 1 else 2, T, 2, K, V, seed=21, decay=decay)
    assert inp["b"].max() > 1.5
    t, r = to_device(inp, gpu_device, dtype)
    fn = chunk_gdn2 if op == "chunk" else fused_recurrent_gdn2
    with torch.no_grad():
        o, ht = fn(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                   use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= REL_TOL[dtype] and es <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_allow_neg_eigval_backward(gpu_device, dtype):
    from qwendopamine_amd.ops import chunk_gdn2

    print(f"[case] allow_neg_eigval backward {dtype}", flush=True)
    B, T, H, K, V = 2, 150, 2, 64, 64
    inp = _neg_eig_inputs(B, T, H, K, V, seed=23)
    rng = np.random.default_rng(24)
    inp["do"] = rng.standard_normal((B, T, H, V))
    t, r = to_device(inp, gpu_device, dtype)
    leaves = [t[n].detach().clone().requires_grad_(True) for n in NAMES]
    h0 = t["h0"].detach().clone().requires_grad_(True)
    o, _ = chunk_gdn2(*leaves, initial_state=h0, use_qk_l2norm_in_kernel=True)
    (o.float() * t["do"].float()).sum().backward()
    torch.cuda.synchronize()
    ref = orc.recurrent_vjp(*(r[n] for n in NAMES), r["do"], None, r["h0"])
    errs = {f"d{n}": rel_l2(x.grad, rv) for n, x, rv in zip((*NAMES, "h0"), (*leaves, h0), ref)}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= REL_TOL[dtype], (k, e)


def test_module_allow_neg_eigval(gpu_device):
    """The module with allow_neg_eigval=True: inference and training paths equal the
    oracle composition with b = 2 sigmoid(b_proj x)."""
    from qwendopamine_amd import GatedDeltaNet2

    print("[case] module allow_neg_eigval", flush=True)
    torch.manual_seed(3)
    m = GatedDeltaNet2(hidden_size=128, num_heads=4, head_dim=32, allow_neg_eigval=True).to(gpu_device)
    x = torch.randn(2, 100, 128, device=gpu_device)
    with torch.no_grad():
        xf = x.float()
        q, _ = m.q_conv1d(m.q_proj(xf))
        k, _ = m.k_conv1d(m.k_proj(xf))
        v, _ = m.v_conv1d(m.v_proj(xf))
        g = -m.A_log.exp().repeat_interleave(m.head_k_dim) * F.softplus(m.f_proj(xf) + m.dt_bias)
        b, w = 2.0 * m.b_proj(xf).sigmoid(), m.w_proj(xf).sigmoid()
        sp = lambda a: a.reshape(*a.shape[:-1], 4, 32).double().cpu().numpy()  # noqa: E731
        o, _ = orc.recurrent_fwd(sp(q), sp(k), sp(v), sp(g), sp(b), sp(w))
        o = torch.from_numpy(o).float().to(gpu_device)
        ref = m.o_proj(m.o_norm(o, m.g_proj(xf).reshape(*o.shape)).reshape(2, 100, -1))
    for training in (False, True):
        m.train(training)
        with torch.no_grad():
            out, _, _ = m(x)
        e = rel_l2(out, ref)
        print(f"  training={training} rel_l2={e:.2e}", flush=True)
        assert e <= 1e-4


def _bounded_gate(graw, A_log, dt_bias, lb):
    H, K = graw.shape[-2], graw.shape[-1]
    xx = graw + dt_bias.reshape(H, K)
    return lb / (1.0 + np.exp(-np.exp(A_log)[:, None] * xx))


@pytest.mark.parametrize("lb", [-5.0, -0.5])
@pytest.mark.parametrize("op,T", [("chunk", 150), ("recurrent", 21), ("recurrent", 1)])
def test_bounded_gate_forward(gpu_device, op, T, lb):
    from qwendopamine_amd.ops import chunk_gdn2, fused_recurrent_gdn2

    print(f"[case] safe_gate lower_bound={lb} forward {op} T={T}", flush=True)
    B, H = 2, 2
    K = V = 128 if T == 1 else 64
    inp = rand_inputs(B, T, H, K, V, seed=31)
    rng = np.random.default_rng(32)
    graw = rng.standard_normal((B, T, H, K)) * 2.0
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    g = _bounded_gate(r["g"], A_log, dt_bias, lb)
    extra = dict(A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
                 dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device),
                 use_gate_in_kernel=True, lower_bound=lb)
    with torch.no_grad():
        if op == "chunk":
            o, ht = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                               use_qk_l2norm_in_kernel=True, safe_gate=True, **extra)
        else:
            o, ht = fused_recurrent_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"],
                                         output_final_state=True, use_qk_l2norm_in_kernel=True, **extra)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, r["b"], r["w"], r["h0"])
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= 1e-4 and es <= 1e-4


def test_bounded_gate_ignored_without_safe_gate(gpu_device):
    """As in the reference (chunk_gdn2.py:1368-1376), the chunk op uses the bound only
    with safe_gate=True; without it the plain gate -exp(A_log) softplus(g + dt_bias) runs."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk lower_bound without safe_gate", flush=True)
    B, T, H, K, V = 1, 80, 2, 32, 32
    inp = rand_inputs(B, T, H, K, V, seed=33)
    rng = np.random.default_rng(34)
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, r["g"] + dt_bias.reshape(H, K))
    with torch.no_grad():
        o, ht = chunk_gdn2(*(t[n] for n in NAMES), initial_state=t["h0"], output_final_state=True,
                           use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True, lower_bound=-1.0,
                           A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
                           dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device))
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, r["b"], r["w"], r["h0"])
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4


def test_bounded_gate_backward(gpu_device):
    """Gradients through the bounded gate (dA_log, ddt_bias, and the input grads) against
    float64 torch autograd of the gate composed with the oracle VJP."""
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] safe_gate lower_bound=-3 backward", flush=True)
    B, T, H, K, V, lb = 1, 96, 2, 32, 32, -3.0
    inp = rand_inputs(B, T, H, K, V, seed=35)
    rng = np.random.default_rng(36)
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    inp["g"] = graw
    do = rng.standard_normal((B, T, H, V))
    t, r = to_device(inp, gpu_device, torch.float32)
    leaves = [t[n].detach().clone().requires_grad_(True) for n in NAMES]
    a_t = torch.tensor(A_log, dtype=torch.float32, device=gpu_device, requires_grad=True)
    d_t = torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device, requires_grad=True)
    o, _ = chunk_gdn2(*leaves, initial_state=t["h0"], use_qk_l2norm_in_kernel=True,
                      use_gate_in_kernel=True, safe_gate=True, lower_bound=lb, A_log=a_t, dt_bias=d_t)
    (o * _dev(do, gpu_device)).sum().backward()
    torch.cuda.synchronize()
    # reference: oracle VJP w.r.t. the activated g, then float64 autograd through the gate
    gr = torch.tensor(r["g"], dtype=torch.float64, requires_grad=True)
    ar = torch.tensor(A_log, dtype=torch.float64, requires_grad=True)
    dr = torch.tensor(dt_bias, dtype=torch.float64, requires_grad=True)
    gact = lb * torch.sigmoid(ar.exp().reshape(H, 1) * (gr + dr.reshape(H, K)))
    ref = orc.recurrent_vjp(r["q"], r["k"], r["v"], gact.detach().numpy(), r["b"], r["w"], do, None, r["h0"])
    gact.backward(torch.from_numpy(ref[3]))
    pairs = {"dq": (leaves[0].grad, ref[0]), "dk": (leaves[1].grad, ref[1]), "dv": (leaves[2].grad, ref[2]),
             "dgraw": (leaves[3].grad, gr.grad.numpy()), "db": (leaves[4].grad, ref[4]),
             "dw": (leaves[5].grad, ref[5]), "dA_log": (a_t.grad, ar.grad.numpy()),
             "ddt_bias": (d_t.grad, dr.grad.numpy())}
    errs = {k: rel_l2(a, b) for k, (a, b) in pairs.items()}
    print("  rel_l2 " + " ".join(f"{k}={v:.2e}" for k, v in errs.items()), flush=True)
    for k, e in errs.items():
        assert e <= 1e-4, (k, e)
