"""GPU parity of the fused module decode step (``ops.decode_step_fused``, C entry
``gdn2_decode_fused``): short convolution + gate / b / w activations + recurrence +
gated RMS norm in one kernel.

* **Oracle.** Against the float64 composition of ``oracle.short_conv`` (with the conv
  cache), the gate formula, ``oracle.recurrent_fwd`` (one token, from the state) and
  ``oracle.gated_rmsnorm``: rel. L2 <= 1e-4 in fp32, <= 2e-2 in bf16 on the same rounded
  inputs.  New conv caches are the last three inputs exactly.
* **Separate HIP passes.** Against ``ops.short_convolution`` -> ``fused_recurrent_gdn2``
  (in-kernel gate, b / w logits) -> ``ops.gated_rmsnorm`` on the same inputs.  At
  d = 128 the fused kernel keeps the decode kernel's thread mapping and summation order,
  so the results are bit-identical; at d = 64 it uses one wave per head (another
  summation order), so they agree to a bf16 rounding.
* **Module.** ``GatedDeltaNet2`` decode steps after a prefill, fused against the separate
  passes (``fused_decode = False``), with dict caches updated in place and not.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rel_l2

pytestmark = pytest.mark.gpu


def _case(dev, dtype, N, H, D, seed, with_cache=True, with_state=True, bias=True, nw_f32=False):
    """Raw inputs as the module produces them: q/k/v/b/w/f/g projections as column ranges
    of one [N, 7 * H * D] tensor (read in place), conv weights, caches, state, gate params."""
    gen = torch.Generator(device="cpu").manual_seed(seed)
    HD = H * D
    rnd = lambda *s, sc=1.0: (torch.randn(*s, generator=gen) * sc)  # noqa: E731
    y = rnd(N, 7 * HD).to(dtype).to(dev)
    qr, kr, vr, bl, wl, graw, z = y.split(HD, dim=-1)
    cw = [rnd(HD, 1, 4, sc=0.5).to(dtype).to(dev) for _ in range(3)]
    cb = [rnd(HD, sc=0.1).to(dtype).to(dev) for _ in range(3)] if bias else None
    caches = [rnd(N, HD, 3).to(dtype).to(dev) for _ in range(3)] if with_cache else None
    h0 = (rnd(N, H, D, D, sc=0.05)).to(dev) if with_state else None
    A_log = torch.log(torch.rand(H, generator=gen) * 15 + 1).to(dev)
    dt_bias = (rnd(HD, sc=0.5)).to(dev)
    nw = (rnd(D, sc=0.2) + 1.0).to(torch.float32 if nw_f32 else dtype).to(dev)
    return dict(x=[qr, kr, vr], cw=cw, cb=cb, caches=caches, h0=h0, bl=bl, wl=wl, graw=graw, z=z,
                A_log=A_log, dt_bias=dt_bias, nw=nw)


def _oracle(c, H, D, eps=1e-5):
    n64 = lambda t: t.detach().double().cpu().numpy()  # noqa: E731
    N = c["x"][0].shape[0]
    outs, new = [], []
    for t in range(3):
        y, nc = orc.short_conv(n64(c["x"][t]).reshape(N, 1, H * D), n64(c["cw"][t]),
                               None if c["cb"] is None else n64(c["cb"][t]),
                               None if c["caches"] is None else n64(c["caches"][t]),
                               output_final_state=True)
        outs.append(y.reshape(N, 1, H, D))
        new.append(nc)
    sig = lambda a: 1.0 / (1.0 + np.exp(-a))  # noqa: E731
    g = -np.exp(n64(c["A_log"]))[:, None] * np.logaddexp(0.0, n64(c["graw"]).reshape(N, H, D)
                                                          + n64(c["dt_bias"]).reshape(H, D))
    b = sig(n64(c["bl"])).reshape(N, 1, H, D)
    w = sig(n64(c["wl"])).reshape(N, 1, H, D)
    o, st = orc.recurrent_fwd(outs[0], outs[1], outs[2], g.reshape(N, 1, H, D), b, w,
                              None if c["h0"] is None else n64(c["h0"]))
    on = orc.gated_rmsnorm(o[:, 0], n64(c["z"]).reshape(N, H, D), n64(c["nw"]), eps)
    return on, st, new


def _fused(c, H, D, in_place=False):
    from qwendopamine_amd import ops

    return ops.decode_step_fused(c["x"], c["cw"], c["cb"], c["caches"], c["graw"], c["bl"], c["wl"], c["h0"],
                                 c["z"], c["nw"], 1e-5, num_heads=H, head_dim=D, A_log=c["A_log"],
                                 dt_bias=c["dt_bias"], update_cache_in_place=in_place)


@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("with_cache,with_state,bias", [(True, True, True), (False, False, False),
                                                         (True, False, False)])
def test_fused_decode_matches_oracle(gpu_device, D, dtype, with_cache, with_state, bias):
    N, H = 5, 3
    print(f"[case] fused decode vs oracle D={D} {dtype} cache={with_cache} state={with_state} "
          f"bias={bias}", flush=True)
    c = _case(gpu_device, dtype, N, H, D, seed=D + 7, with_cache=with_cache, with_state=with_state, bias=bias)
    o, st, new = _fused(c, H, D)
    torch.cuda.synchronize()
    o_ref, s_ref, new_ref = _oracle(c, H, D)
    eo, es = rel_l2(o, o_ref), rel_l2(st, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert o.dtype == dtype and o.shape == (N, H, D)
    assert eo <= REL_TOL[dtype] and es <= REL_TOL[dtype]
    for t in range(3):  # the new caches are the last three inputs, exactly
        np.testing.assert_array_equal(new[t].double().cpu().numpy(), new_ref[t])


def test_fused_decode_fp32_norm_weight_promotes(gpu_device):
    N, H, D = 4, 2, 64
    print("[case] fused decode, bf16 io with an fp32 norm weight", flush=True)
    c = _case(gpu_device, torch.bfloat16, N, H, D, seed=3, nw_f32=True)
    o, st, _ = _fused(c, H, D)
    torch.cuda.synchronize()
    o_ref, s_ref, _ = _oracle(c, H, D)
    assert o.dtype == torch.float32
    assert rel_l2(o, o_ref) <= 2e-2 and rel_l2(st, s_ref) <= 2e-2


@pytest.mark.parametrize("D", [64, 128])
def test_fused_decode_equals_separate_passes(gpu_device, D):
    from qwendopamine_amd import ops

    N, H = 6, 4
    print(f"[case] fused decode vs separate HIP passes D={D} bf16", flush=True)
    c = _case(gpu_device, torch.bfloat16, N, H, D, seed=11)
    o, st, new = _fused(c, H, D)
    (q, k, v), new_sep = ops.short_convolution([x.unsqueeze(1) for x in c["x"]], c["cw"], c["cb"], c["caches"],
                                               True, "silu")
    sp = lambda t: t.reshape(N, 1, H, D)  # noqa: E731
    o_sep, st_sep = ops.fused_recurrent_gdn2(
        sp(q), sp(k), sp(v), sp(c["graw"]), sp(c["bl"]), sp(c["wl"]), A_log=c["A_log"], dt_bias=c["dt_bias"],
        initial_state=c["h0"], output_final_state=True, use_qk_l2norm_in_kernel=True,
        use_gate_in_kernel=True, bw_logits=True)
    on_sep = ops.gated_rmsnorm(o_sep[:, 0], sp(c["z"])[:, 0], c["nw"], 1e-5)
    torch.cuda.synchronize()
    for t in range(3):
        assert torch.equal(new[t], new_sep[t])
    if D == 128:
        assert torch.equal(st, st_sep)
        assert torch.equal(o, on_sep)
    else:
        assert rel_l2(st, st_sep) <= 1e-5
        same = (o == on_sep).float().mean().item()
        worst = ((o.float() - on_sep.float()).abs() / (on_sep.float().abs() + 1e-2)).max().item()
        print(f"  bit-identical {same:.4f}, worst relative diff {worst:.2e}", flush=True)
        assert same >= 0.95 and worst <= 2.0 ** -6


@pytest.mark.parametrize("D", [64, 128])
def test_fused_decode_in_place(gpu_device, D):
    """In-place update of the caches and state equals the out-of-place results bit for bit."""
    N, H = 3, 2
    print(f"[case] fused decode in place D={D}", flush=True)
    c = _case(gpu_device, torch.bfloat16, N, H, D, seed=5)
    o1, st1, new1 = _fused(c, H, D, in_place=False)
    caches, h0 = c["caches"], c["h0"]
    o2, st2, new2 = _fused(c, H, D, in_place=True)
    torch.cuda.synchronize()
    assert st2.data_ptr() == h0.data_ptr() and all(a.data_ptr() == b.data_ptr() for a, b in zip(new2, caches))
    assert torch.equal(o1, o2) and torch.equal(st1, st2)
    for a, b in zip(new1, new2):
        assert torch.equal(a, b)


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("in_place", [False, True])
def test_module_fused_decode_equals_separate(gpu_device, head_dim, in_place):
    """Prefill, then decode steps: the fused path equals the separate passes (bit for bit at
    d = 128, to a bf16 rounding at d = 64), outputs and caches."""
    from qwendopamine_amd import GatedDeltaNet2

    print(f"[case] module fused decode head_dim={head_dim} in_place={in_place}", flush=True)
    torch.manual_seed(0)
    m = GatedDeltaNet2(hidden_size=256, num_heads=2, head_dim=head_dim).to(gpu_device).to(torch.bfloat16).eval()
    x = torch.randn(2, 40, 256, device=gpu_device).to(torch.bfloat16)
    steps = torch.randn(2, 4, 256, device=gpu_device).to(torch.bfloat16)
    res = {}
    for fused in (True, False):
        m.fused_decode = fused
        cache: dict = {}
        with torch.no_grad():
            m(x, past_key_values=cache, use_cache=True)
            outs = []
            for t in range(steps.shape[1]):
                o, _, cache = m(steps[:, t:t + 1], past_key_values=cache, use_cache=True,
                                update_cache_in_place=in_place)
                outs.append(o)
        torch.cuda.synchronize()
        res[fused] = (torch.cat(outs, 1), cache["recurrent_state"], cache["conv_state"])
    (of, sf, cf), (os_, ss, cs) = res[True], res[False]
    for a, b in zip(cf, cs):
        assert torch.equal(a, b)
    if head_dim == 128:
        assert torch.equal(sf, ss) and torch.equal(of, os_)
    else:
        e_o, e_s = rel_l2(of, os_), rel_l2(sf, ss)
        print(f"  rel_l2 o={e_o:.2e} state={e_s:.2e}", flush=True)
        assert e_o <= 1e-2 and e_s <= 1e-3
