"""The allocation-free chunk forward (C entry point ``gdn2_chunk_fwd_static``).

It must give exactly what ``gdn2_chunk_fwd`` gives on the same inputs (the same
kernels run; only the workspace differs), on consecutive calls that reuse the one
static array, the second call smaller and of another shape, so that whatever the
first call left behind in the array would show up in a wrong result.  Shapes
beyond the array's size are rejected before anything is launched.
"""

from __future__ import annotations


import numpy as np
import pytest
import torch

from tests._helpers import rand_inputs, to_device

NAMES = ("q", "k", "v", "g", "b", "w")


def test_static_rejects_oversize_before_launch():
    """A shape needing more than 72 MiB of blobs returns GDN2_ERR_SCRATCH (no GPU needed:
    the size is checked before any pointer is touched or any HIP call is made)."""
    from qwendopamine_amd import _native as nat

    lib = nat.load()
    B, T, H, K, V = 1, 8192, 16, 128, 128  # 2048 blobs of 66,048 B = 135 MB
    need = lib.gdn2_chunk_fwd_workspace_size(B, T, H, K, V, nat.DTYPE_BF16, None, B)
    assert need > nat.STATIC_SCRATCH_BYTES
    st = lib.gdn2_chunk_fwd_static(*([None] * 6), nat.DTYPE_BF16, nat.DTYPE_F32, None, None, None,
                                   None, None, 0.0, None, None, B, B, T, H, K, V, 1.0, 0, None)
    assert st == nat.ERR_SCRATCH
    assert b"static scratch" in lib.gdn2_status_string(st)
    # The largest shape of the stated limit fits: 4096 tokens x 16 heads at d_k = 128 in bf16.
    assert lib.gdn2_chunk_fwd_workspace_size(1, 4096, 16, 128, 128, nat.DTYPE_BF16, None, 1) \
        <= nat.STATIC_SCRATCH_BYTES
    # Training workspaces cannot live in the shared array.
    st = lib.gdn2_chunk_fwd_static(*([None] * 6), nat.DTYPE_BF16, nat.DTYPE_F32, None, None, None,
                                   None, None, 0.0, None, None, 1, 1, 64, 2, 32, 32, 1.0,
                                   nat.FLAG_SAVE_FOR_BWD, None)
    assert st == nat.ERR_INVALID


def _case(dev, dtype, B, T, H, K, V, seed, cu=None):
    from qwendopamine_amd.ops import chunk_gdn2_fwd, chunk_gdn2_static

    inp = rand_inputs(B, T, H, K, V, seed=seed, h0_std=0.1)
    if cu is not None:
        inp["h0"] = np.random.default_rng(seed + 1).standard_normal((len(cu) - 1, H, K, V)) * 0.1
    t, _ = to_device(inp, dev, dtype)
    cu_d = None if cu is None else torch.tensor(cu, dtype=torch.int64, device=dev)
    cu_h = None if cu is None else torch.tensor(cu, dtype=torch.int64)
    N = B if cu is None else len(cu) - 1
    with torch.no_grad():
        o_ref, s_ref = chunk_gdn2_fwd(*(t[n] for n in NAMES), K**-0.5, t["h0"], True,
                                      use_qk_l2norm_in_kernel=True, cu_seqlens=cu_d)
    out = torch.full_like(o_ref, float("nan"))
    fin = torch.full((N, H, K, V), float("nan"), dtype=torch.float32, device=dev)
    torch.cuda.synchronize()
    o, s = chunk_gdn2_static(*(t[n] for n in NAMES), out, fin, initial_state=t["h0"],
                             use_qk_l2norm_in_kernel=True, cu_seqlens=cu_d, cu_seqlens_cpu=cu_h)
    torch.cuda.synchronize()
    assert o is out and s is fin
    return o, s, o_ref, s_ref


@pytest.mark.gpu
def test_static_equals_workspace_entry_point(gpu_device):
    """Three calls in a row on the shared array, each smaller than the one before, each
    bit-identical to the workspace entry point on the same inputs."""
    cases = [
        ("bf16 B2 T700 H8 K=V=128", torch.bfloat16, 2, 700, 8, 128, 128, 1, None),
        ("fp32 B1 T150 H3 K=64 V=32", torch.float32, 1, 150, 3, 64, 32, 2, None),
        ("bf16 varlen T130 [0,1,60,60,130] H2 K=32 V=48", torch.bfloat16, 1, 130, 2, 32, 48, 3,
         [0, 1, 60, 60, 130]),
    ]
    for label, dtype, B, T, H, K, V, seed, cu in cases:
        print(f"[case] static chunk forward {label}", flush=True)
        o, s, o_ref, s_ref = _case(gpu_device, dtype, B, T, H, K, V, seed, cu)
        assert torch.equal(o, o_ref), label
        assert torch.equal(s, s_ref), label


@pytest.mark.gpu
def test_static_rejects_oversize_through_the_op(gpu_device):
    from qwendopamine_amd.ops import chunk_gdn2_static

    print("[case] static chunk forward, oversize shape", flush=True)
    B, T, H, K, V = 1, 8192, 16, 128, 128
    x = torch.zeros(B, T, H, K, dtype=torch.bfloat16, device=gpu_device)
    g = torch.zeros(B, T, H, K, dtype=torch.float32, device=gpu_device)
    with pytest.raises(ValueError, match="static scratch"):
        chunk_gdn2_static(x, x, x, g, x, x, torch.empty_like(x))
    torch.cuda.synchronize()
