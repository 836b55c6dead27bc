"""GPU parity of the HIP kernels against the float64 oracle (small, seeded cases).

Tolerances (north star): relative L2 <= 1e-4 for float32 inputs, <= 2e-2 for
bf16 / fp16 inputs against the oracle run on the same rounded inputs.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu


def _recurrent(dev, dtype, B, T, H, K, V, HV=None, seed=0, decay="paper", cu=None, h0_std=0.1):
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    inp = rand_inputs(B, T, H, K, V, HV=HV, seed=seed, decay=decay, h0_std=h0_std)
    if cu is not None:
        inp["h0"] = None if h0_std == 0 else np.random.default_rng(seed + 1).standard_normal(
            (len(cu) - 1, HV or H, K, V)) * h0_std
    t, r = to_device(inp, dev, dtype)
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int64, device=dev)
    o, ht = fused_recurrent_gdn2(
        t["q"], t["k"], t["v"], t["g"], t["b"], t["w"], initial_state=t["h0"],
        output_final_state=True, use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t,
    )
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], r["h0"],
                                     cu_seqlens=cu)
    return o, ht, o_ref, s_ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,V", [(32, 24), (128, 128), (64, 16), (100, 36)])
def test_recurrent_matches_oracle(gpu_device, dtype, K, V):
    print(f"[case] recurrent dtype={dtype} K={K} V={V}", flush=True)
    o, ht, o_ref, s_ref = _recurrent(gpu_device, dtype, 2, 19, 3, K, V)
    assert o.dtype == dtype and ht.dtype == torch.float32
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(ht, s_ref) <= REL_TOL[dtype]


def test_recurrent_gva_and_varlen(gpu_device):
    print("[case] recurrent GVA", flush=True)
    o, ht, o_ref, s_ref = _recurrent(gpu_device, torch.float32, 2, 11, 2, 32, 32, HV=4)
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4
    print("[case] recurrent varlen", flush=True)
    cu = [0, 5, 5, 17, 30]
    o, ht, o_ref, s_ref = _recurrent(gpu_device, torch.float32, 1, 30, 2, 32, 32, cu=cu)
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4


@pytest.mark.parametrize("B,H,HV,dtype", [(8, 4, 4, torch.bfloat16), (3, 1, 3, torch.float32),
                                           (5, 2, 4, torch.bfloat16)])
def test_recurrent_decode_inplace(gpu_device, B, H, HV, dtype):
    """Single-token decode step updating the state in place (serving path); odd
    slab counts and grouped value heads exercise the two-slab decode kernel."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2_fwd

    print(f"[case] recurrent decode in place B={B} H={H} HV={HV} {dtype}", flush=True)
    inp = rand_inputs(B, 1, H, 128, 128, HV=HV, seed=3, h0_std=0.02)
    t, r = to_device(inp, gpu_device, dtype)
    state = t["h0"].clone()
    o, ht = fused_recurrent_gdn2_fwd(t["q"], t["k"], t["v"], t["g"], t["b"], t["w"],
                                     initial_state=state, inplace_final_state=True,
                                     use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert ht.data_ptr() == state.data_ptr()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], r["h0"])
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(state, s_ref) <= REL_TOL[dtype]


def test_decode_zero_state_and_no_final_state(gpu_device):
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    inp = rand_inputs(4, 1, 2, 128, 128, seed=4, h0_std=0.0)
    t, r = to_device(inp, gpu_device, torch.float32)
    o, ht = fused_recurrent_gdn2(t["q"], t["k"], t["v"], t["g"], t["b"], t["w"],
                                 use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    assert ht is None
    o_ref, _ = orc.recurrent_fwd(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], None)
    assert rel_l2(o, o_ref) <= 1e-4


def test_recurrent_gate_in_kernel(gpu_device):
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    print("[case] recurrent gate in kernel", flush=True)
    B, T, H, K, V = 2, 9, 2, 32, 32
    inp = rand_inputs(B, T, H, K, V, seed=5)
    rng = np.random.default_rng(9)
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    x = graw + dt_bias.reshape(H, K)
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, x)
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    o, ht = fused_recurrent_gdn2(
        t["q"], t["k"], t["v"], t["g"], t["b"], t["w"],
        A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
        dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device),
        initial_state=t["h0"], output_final_state=True, use_qk_l2norm_in_kernel=True,
        use_gate_in_kernel=True,
    )
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, r["b"], r["w"], r["h0"])
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4


@pytest.mark.parametrize("T,K,V", [(9, 32, 32), (1, 128, 128)])
def test_recurrent_sigmoid_bw_logits(gpu_device, T, K, V):
    """b and w passed as logits (GDN2_FLAG_SIGMOID_BW), with the in-kernel gate: the
    module's fused decode path. T = 1 with K = V = 128 runs the decode-step kernel,
    the other case the generic one. The oracle gets sigmoid(b), sigmoid(w) in float64."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    print(f"[case] recurrent sigmoid b/w T={T} K={K} V={V}", flush=True)
    B, H = 3, 2
    inp = rand_inputs(B, T, H, K, V, seed=11)
    rng = np.random.default_rng(12)
    bl, wl = rng.standard_normal((B, T, H, K)) * 2, rng.standard_normal((B, T, H, V)) * 2
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, graw + dt_bias.reshape(H, K))
    inp.update(b=bl, w=wl, g=graw)
    t, r = to_device(inp, gpu_device, torch.float32)
    o, ht = fused_recurrent_gdn2(
        t["q"], t["k"], t["v"], t["g"], t["b"], t["w"],
        A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
        dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device),
        initial_state=t["h0"], output_final_state=True, use_qk_l2norm_in_kernel=True,
        use_gate_in_kernel=True, bw_logits=True,
    )
    torch.cuda.synchronize()
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))  # noqa: E731
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, sig(r["b"]), sig(r["w"]), r["h0"])
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4


def _chunk(dev, dtype, B, T, H, K, V, seed=0, decay="paper", h0_std=0.1, g_dtype=torch.float32):
    from qwendopamine_amd.ops import chunk_gdn2

    inp = rand_inputs(B, T, H, K, V, seed=seed, decay=decay, h0_std=h0_std)
    t, r = to_device(inp, dev, dtype, g_dtype=g_dtype)
    o, ht = chunk_gdn2(t["q"], t["k"], t["v"], t["g"], t["b"], t["w"], initial_state=t["h0"],
                       output_final_state=True, use_qk_l2norm_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], r["h0"])
    return o, ht, o_ref, s_ref


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("K,V,T", [(32, 32, 64), (64, 48, 130), (128, 128, 200), (40, 24, 77), (16, 16, 33)])
def test_chunk_matches_oracle(gpu_device, dtype, K, V, T):
    print(f"[case] chunk dtype={dtype} K={K} V={V} T={T}", flush=True)
    o, ht, o_ref, s_ref = _chunk(gpu_device, dtype, 2, T, 2, K, V)
    assert o.dtype == dtype and ht.dtype == torch.float32
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.3e} state={es:.3e}", flush=True)
    assert eo <= REL_TOL[dtype] and es <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("decay,K,T", [("extreme", 64, 128), ("extreme", 128, 128), ("sheer", 64, 128),
                                         ("sheer", 128, 128), ("extreme", 64, 77), ("sheer", 40, 77)])
def test_chunk_wide_decay_diagonal_blocks(gpu_device, dtype, decay, K, T):
    """Diagonal blocks whose decay span leaves the factored range.  "extreme" spans (> 115
    per 16 tokens, within it per 4-token quarter) take the four quarter-referred MFMA
    products; "sheer" ones (> 115 per quarter) add the exact pair sums inside each quarter.
    float32 storage and bf16 at d_k = 64 take these paths; bf16 at d_k = 128 sums every
    pair of a wide block exactly.  T = 77 ends in a partial chunk whose last 16-token block
    and last quarter are partial; K = 40 leaves channels of the padded width unused."""
    print(f"[case] chunk {decay} decay {dtype} K={K} T={T}", flush=True)
    o, ht, o_ref, s_ref = _chunk(gpu_device, dtype, 1, T, 2, K, 64, decay=decay)
    assert np.isfinite(o.float().cpu().numpy()).all()
    eo, es = rel_l2(o, o_ref), rel_l2(ht, s_ref)
    print(f"  rel_l2 o={eo:.2e} state={es:.2e}", flush=True)
    assert eo <= REL_TOL[dtype] and es <= REL_TOL[dtype]


def test_chunk_bf16_g_in_bf16(gpu_device):
    print("[case] chunk bf16 with bf16 g", flush=True)
    o, ht, o_ref, s_ref = _chunk(gpu_device, torch.bfloat16, 2, 96, 2, 64, 64, g_dtype=torch.bfloat16)
    assert rel_l2(o, o_ref) <= 2e-2 and rel_l2(ht, s_ref) <= 2e-2


def test_chunk_varlen_and_zero_state(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk varlen", flush=True)
    cu = [0, 70, 70, 71, 200, 264]
    T, H, K, V = cu[-1], 2, 64, 64
    inp = rand_inputs(1, T, H, K, V, seed=11, h0_std=0.0)
    t, r = to_device(inp, gpu_device, torch.float32)
    cu_t = torch.tensor(cu, dtype=torch.int64, device=gpu_device)
    o, ht = chunk_gdn2(t["q"], t["k"], t["v"], t["g"], t["b"], t["w"], output_final_state=True,
                       use_qk_l2norm_in_kernel=True, cu_seqlens=cu_t)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], r["g"], r["b"], r["w"], None, cu_seqlens=cu)
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4
    assert torch.all(ht[1] == 0)  # empty sequence keeps the zero state


def test_chunk_gate_in_kernel(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2

    print("[case] chunk gate in kernel", flush=True)
    B, T, H, K, V = 1, 100, 2, 64, 32
    inp = rand_inputs(B, T, H, K, V, seed=13)
    rng = np.random.default_rng(17)
    graw = rng.standard_normal((B, T, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, graw + dt_bias.reshape(H, K))
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    o, ht = chunk_gdn2(t["q"], t["k"], t["v"], t["g"], t["b"], t["w"], initial_state=t["h0"],
                       output_final_state=True, use_qk_l2norm_in_kernel=True,
                       use_gate_in_kernel=True,
                       A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
                       dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device))
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, r["b"], r["w"], r["h0"])
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4
