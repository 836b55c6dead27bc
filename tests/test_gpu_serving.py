"""GPU parity of the token-serial op's serving options against the float64 oracle
(``oracle.recurrent_fwd_pooled``): a state pool addressed by ``ssm_state_indices``
(continuous batching), ``num_accepted_tokens`` (speculative decoding), per-token
state stores, and the transposed state layout (reference
``fused_recurrent_gdn2.py:215-232, 311-333``).

Tolerances (north star): relative L2 <= 1e-4 for float32 inputs, <= 2e-2 for
bf16 inputs, against the oracle run on the same rounded inputs.  Pool slots the
op must not touch are compared bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gdn2_oracle as orc
from tests._helpers import REL_TOL, rand_inputs, rel_l2, to_device

pytestmark = pytest.mark.gpu

NAMES = ("q", "k", "v", "g", "b", "w")


def _pooled(dev, dtype, inp, pool, slots, accepted=None, cu=None, inplace=True, transpose=False,
            idx_dtype=torch.int64, final_rows=None):
    """Run the HIP op and the oracle on the same (rounded) inputs; returns both results."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2_fwd

    t, r = to_device({n: inp[n] for n in NAMES}, dev, dtype)
    pool_t = torch.tensor(pool, dtype=torch.float32, device=dev)
    idx_t = torch.tensor(slots, dtype=idx_dtype, device=dev)
    acc_t = None if accepted is None else torch.tensor(accepted, dtype=torch.int32, device=dev)
    cu_t = None if cu is None else torch.tensor(cu, dtype=torch.int64, device=dev)
    o, ht = fused_recurrent_gdn2_fwd(
        *(t[n] for n in NAMES), initial_state=pool_t, inplace_final_state=inplace,
        output_final_state=not inplace, cu_seqlens=cu_t, ssm_state_indices=idx_t,
        num_accepted_tokens=acc_t, use_qk_l2norm_in_kernel=True,
        transpose_state_layout=transpose,
    )
    torch.cuda.synchronize()
    o_ref, st_ref, written = orc.recurrent_fwd_pooled(
        *(r[n] for n in NAMES), pool, slots, accepted, inplace_final_state=inplace,
        cu_seqlens=cu, transpose_state_layout=transpose, final_rows=final_rows)
    return o, ht, o_ref, st_ref, written


def _check_pool(ht, st_ref, written, tol, untouched_from=None):
    got = ht.double().cpu().numpy()
    assert rel_l2(got[written], st_ref[written]) <= tol
    if untouched_from is not None:
        keep = [r for r in range(got.shape[0]) if r not in written]
        assert np.array_equal(got[keep], untouched_from[keep]), "untouched pool slots changed"


@pytest.mark.parametrize("dtype,K,V,idx_dtype", [(torch.bfloat16, 128, 128, torch.int32),
                                                 (torch.float32, 128, 128, torch.int64),
                                                 (torch.float32, 64, 32, torch.int32),
                                                 (torch.bfloat16, 40, 24, torch.int64)])
def test_decode_state_pool(gpu_device, dtype, K, V, idx_dtype):
    """One token per sequence, slots scattered over a larger pool, one padded entry (-1) and one
    slot past the pool end: both start from a zero state and store nothing."""
    print(f"[case] decode pool dtype={dtype} K={K} V={V} idx={idx_dtype}", flush=True)
    N, H, rows = 7, 4, 19
    inp = rand_inputs(N, 1, H, K, V, seed=31)
    rng = np.random.default_rng(32)
    pool = (rng.standard_normal((rows, H, K, V)) * 0.1).astype(np.float32).astype(np.float64)
    slots = np.array([11, 3, -1, 17, 0, rows + 4, 8])
    o, ht, o_ref, st_ref, written = _pooled(gpu_device, dtype, inp, pool, slots, idx_dtype=idx_dtype)
    assert written == sorted([11, 3, 17, 0, 8])
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    _check_pool(ht, st_ref, written, REL_TOL[dtype], untouched_from=pool)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_speculative_decoding_two_steps(gpu_device, dtype):
    """Step 1 stores the state after each draft token in slot idx[n, t]; step 2 resumes from
    slot idx[n, num_accepted - 1] (packed varlen sequences, [N, T_max] indices)."""
    print(f"[case] speculative decoding dtype={dtype}", flush=True)
    H, K, V, Tm = 2, 64, 64, 4
    rng = np.random.default_rng(41)
    slots = np.array([[3, 9, 1, 12], [0, 5, 7, 14], [2, 4, 6, 8]])
    pool = np.zeros((16, H, K, V))
    pool[slots[:, 0]] = rng.standard_normal((3, H, K, V)) * 0.1
    pool = pool.astype(np.float32).astype(np.float64)
    cu1 = [0, 4, 8, 12]
    inp1 = rand_inputs(1, 12, H, K, V, seed=42)
    o1, ht1, o1_ref, p1_ref, w1 = _pooled(gpu_device, dtype, inp1, pool, slots, [1, 1, 1], cu=cu1)
    assert rel_l2(o1, o1_ref) <= REL_TOL[dtype]
    _check_pool(ht1, p1_ref, w1, REL_TOL[dtype], untouched_from=pool)
    # Step 2 starts from the pool the GPU wrote (as a server would), rounded like its input.
    pool1 = ht1.double().cpu().numpy()
    cu2 = [0, 2, 5, 6]
    inp2 = rand_inputs(1, 6, H, K, V, seed=43)
    o2, ht2, o2_ref, p2_ref, w2 = _pooled(gpu_device, dtype, inp2, pool1, slots, [3, 1, 4], cu=cu2)
    assert rel_l2(o2, o2_ref) <= REL_TOL[dtype]
    _check_pool(ht2, p2_ref, w2, REL_TOL[dtype], untouched_from=pool1)


def test_pooled_token_rows_not_inplace(gpu_device):
    """Without in-place stores every token's state goes to its packed row of a new state."""
    print("[case] pooled per-token rows", flush=True)
    H, K, V = 2, 32, 32
    cu = [0, 3, 3, 8, 10]
    inp = rand_inputs(1, 10, H, K, V, seed=51)
    rng = np.random.default_rng(52)
    pool = (rng.standard_normal((6, H, K, V)) * 0.1).astype(np.float32).astype(np.float64)
    slots = np.array([4, 1, 0, 5])
    o, ht, o_ref, st_ref, written = _pooled(gpu_device, torch.float32, inp, pool, slots, cu=cu,
                                            inplace=False, final_rows=10)
    assert ht.shape[0] == 10 and written == list(range(10))
    assert rel_l2(o, o_ref) <= 1e-4
    _check_pool(ht, st_ref, written, 1e-4)


@pytest.mark.parametrize("dtype,K,V,T", [(torch.float32, 128, 128, 1), (torch.float32, 40, 24, 9),
                                         (torch.bfloat16, 128, 128, 5), (torch.float32, 16, 64, 3)])
def test_transposed_state_layout(gpu_device, dtype, K, V, T):
    """transpose_state_layout: states are [V, K]; results equal the [K, V] path's, transposed."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    print(f"[case] transposed state dtype={dtype} K={K} V={V} T={T}", flush=True)
    B, H = 3, 2
    inp = rand_inputs(B, T, H, K, V, seed=61)
    t, r = to_device(inp, gpu_device, dtype)
    h0_t = t["h0"].transpose(-1, -2).contiguous()
    o, ht = fused_recurrent_gdn2(*(t[n] for n in NAMES), initial_state=h0_t,
                                 output_final_state=True, use_qk_l2norm_in_kernel=True,
                                 transpose_state_layout=True)
    torch.cuda.synchronize()
    assert tuple(ht.shape) == (B, H, V, K)
    o_ref, s_ref = orc.recurrent_fwd(*(r[n] for n in NAMES), r["h0"])
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(ht, np.swapaxes(s_ref, -1, -2)) <= REL_TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_transposed_decode_step_no_state_gate_logits(gpu_device, dtype):
    """The [V, K] decode-step kernel without an initial state, with the in-kernel gate and b / w
    logits, an odd number of slabs (the last workgroup holds one)."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2

    print(f"[case] transposed decode step, no state, gate logits {dtype}", flush=True)
    B, H, K, V = 3, 3, 128, 128
    inp = rand_inputs(B, 1, H, K, V, seed=63, h0_std=0.0)
    rng = np.random.default_rng(64)
    bl, wl = rng.standard_normal((B, 1, H, K)) * 2, rng.standard_normal((B, 1, H, V)) * 2
    graw = rng.standard_normal((B, 1, H, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    g = -np.exp(A_log)[:, None] * np.logaddexp(0.0, graw + dt_bias.reshape(H, K))
    inp.update(b=bl, w=wl, g=graw)
    t, r = to_device(inp, gpu_device, dtype)
    t["g"] = torch.from_numpy(graw).to(gpu_device, torch.float32)
    with torch.no_grad():
        o, ht = fused_recurrent_gdn2(
            *(t[n] for n in NAMES), output_final_state=True, use_qk_l2norm_in_kernel=True,
            use_gate_in_kernel=True, A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
            dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device), bw_logits=True,
            transpose_state_layout=True)
    torch.cuda.synchronize()
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))  # noqa: E731
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, sig(r["b"]), sig(r["w"]), None)
    assert tuple(ht.shape) == (B, H, V, K)
    assert rel_l2(o, o_ref) <= REL_TOL[dtype]
    assert rel_l2(ht, np.swapaxes(s_ref, -1, -2)) <= REL_TOL[dtype]


def test_transposed_state_pool_decode(gpu_device):
    print("[case] transposed pooled decode", flush=True)
    N, H, K, V = 5, 4, 128, 128
    inp = rand_inputs(N, 1, H, K, V, seed=71)
    rng = np.random.default_rng(72)
    pool = (rng.standard_normal((8, H, V, K)) * 0.1).astype(np.float32).astype(np.float64)
    slots = np.array([6, 2, 7, -1, 0])
    o, ht, o_ref, st_ref, written = _pooled(gpu_device, torch.bfloat16, inp, pool, slots,
                                            transpose=True)
    assert written == [0, 2, 6, 7]
    assert rel_l2(o, o_ref) <= 2e-2
    _check_pool(ht, st_ref, written, 2e-2, untouched_from=pool)


@pytest.mark.parametrize("B,T,K,V", [(2, 6, 32, 32), (3, 1, 128, 128)])
def test_gva_gate_in_kernel_by_key_head(gpu_device, B, T, K, V):
    """Grouped value heads with the in-kernel gate: A_log / dt_bias are indexed by key head,
    as the reference kernel does (fused_recurrent_gdn2.py:259-265).  T = 1 with K = V = 128
    runs the decode-step kernel with an initial state (12 slabs over 6 workgroups)."""
    from qwendopamine_amd.ops import fused_recurrent_gdn2_fwd

    print(f"[case] GVA gate in kernel B={B} T={T} K={K} V={V}", flush=True)
    H, HV = 2, 4
    inp = rand_inputs(B, T, H, K, V, HV=HV, seed=81)
    rng = np.random.default_rng(82)
    graw = rng.standard_normal((B, T, HV, K))
    A_log = np.log(rng.uniform(1, 16, H))
    dt_bias = rng.standard_normal(H * K) * 0.5
    hk = np.arange(HV) // (HV // H)
    x = graw + dt_bias.reshape(H, K)[hk]
    g = -np.exp(A_log)[hk][:, None] * np.logaddexp(0.0, x)
    inp["g"] = graw
    t, r = to_device(inp, gpu_device, torch.float32)
    h0 = t["h0"].clone()
    o, ht = fused_recurrent_gdn2_fwd(
        *(t[n] for n in NAMES), A_log=torch.tensor(A_log, dtype=torch.float32, device=gpu_device),
        dt_bias=torch.tensor(dt_bias, dtype=torch.float32, device=gpu_device), initial_state=h0,
        inplace_final_state=True, use_qk_l2norm_in_kernel=True, use_gate_in_kernel=True)
    torch.cuda.synchronize()
    o_ref, s_ref = orc.recurrent_fwd(r["q"], r["k"], r["v"], g, r["b"], r["w"], r["h0"])
    assert ht.data_ptr() == h0.data_ptr()
    assert rel_l2(o, o_ref) <= 1e-4 and rel_l2(ht, s_ref) <= 1e-4
