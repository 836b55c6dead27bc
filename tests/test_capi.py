"""C-ABI checks that need no GPU: the library loads, exports every symbol that
include/gdn2_hip.h declares, and rejects bad arguments before launching."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "gdn2_hip.h"


def _declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(gdn2_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from qwendopamine_amd import _native as nat

    if not nat.LIB_PATH.exists():
        pytest.fail(f"{nat.LIB_PATH} not built (run python -m qwendopamine_amd.build)")
    return nat.load()


def test_header_declares_entry_points():
    names = _declared_functions()
    for n in ("gdn2_abi_version", "gdn2_status_string", "gdn2_recurrent_fwd",
              "gdn2_chunk_fwd", "gdn2_chunk_fwd_workspace_size"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    from qwendopamine_amd import _native as nat

    raw = ctypes.CDLL(str(nat.LIB_PATH))
    for name in _declared_functions():
        assert hasattr(raw, name), f"{name} declared in gdn2_hip.h but not exported"
        assert name in nat.SIGNATURES, f"{name} has no ctypes signature in _native.py"


def test_every_bound_entry_point_is_declared():
    """The reverse direction: every entry point the ctypes binding names (the
    library's public surface) is declared in gdn2_hip.h."""
    from qwendopamine_amd import _native as nat

    declared = set(_declared_functions())
    missing = sorted(n for n in nat.SIGNATURES if n not in declared)
    assert not missing, f"bound in _native.py but not declared in gdn2_hip.h: {missing}"


def test_abi_version_and_status_strings(lib):
    from qwendopamine_amd import _native as nat

    assert lib.gdn2_abi_version() == nat.ABI_VERSION == 2
    assert lib.gdn2_status_string(0) == b"ok"
    assert b"invalid" in lib.gdn2_status_string(-1)
    assert b"workspace" in lib.gdn2_status_string(-4)


def test_invalid_arguments_rejected_before_launch(lib):
    from qwendopamine_amd import _native as nat

    # bad dtype code
    st = lib.gdn2_recurrent_fwd(None, None, None, None, None, None, 7, 0, None, None, None, None,
                                None, 0.0, None, 1, 1, 1, 1, 1, 16, 16, 1.0, 0, None)
    assert st == nat.ERR_INVALID
    # value heads not a multiple of key heads
    st = lib.gdn2_recurrent_fwd(None, None, None, None, None, None, 0, 0, None, None, None, None,
                                None, 0.0, None, 1, 1, 1, 2, 3, 16, 16, 1.0, 0, None)
    assert st == nat.ERR_INVALID
    # key dim above 256 is unsupported (reference asserts K <= 256)
    st = lib.gdn2_recurrent_fwd(None, None, None, None, None, None, 0, 0, None, None, None, None,
                                None, 0.0, None, 1, 1, 1, 1, 1, 300, 16, 1.0, 0, None)
    assert st == nat.ERR_UNSUPPORTED
    # gate-in-kernel without A_log
    st = lib.gdn2_recurrent_fwd(None, None, None, None, None, None, 0, 0, None, None, None, None,
                                None, 0.0, None, 1, 1, 1, 1, 1, 16, 16, 1.0, nat.FLAG_GATE_IN_KERNEL, None)
    assert st == nat.ERR_INVALID
    # non-null tensors required when there are tokens
    st = lib.gdn2_chunk_fwd(None, None, None, None, None, None, 1, 0, None, None, None, None, None,
                            0.0, None, None, 1, 1, 8, 1, 16, 16, 1.0, 0, None, 0, None)
    assert st == nat.ERR_INVALID


def test_gated_norm_chunk_arguments_rejected_before_launch(lib):
    """The fused-norm chunk forward: bf16 only, V in {16, 32, 64}, inference only, and the
    gate / output alignment it reads with 8-byte accesses."""
    from qwendopamine_amd import _native as nat

    def call(io=1, V=64, flags=0, ld=64, gate=0x1000, o=0x2000, tensors=True):
        t = 0x3000 if tensors else None
        return lib.gdn2_chunk_fwd_gated_norm(t, t, t, t, t, t, io, 0, o, gate, ld, t, 1e-5, None, None,
                                             None, None, 0.0, None, None, 1, 1, 8, 1, 16, V, 1.0,
                                             flags, None, 0, None)

    assert call(io=0) == nat.ERR_UNSUPPORTED                  # float32
    assert call(io=2) == nat.ERR_UNSUPPORTED                  # float16
    assert call(V=128, ld=128) == nat.ERR_UNSUPPORTED         # a row spans several workgroups
    assert call(V=48, ld=48) == nat.ERR_UNSUPPORTED
    assert call(flags=nat.FLAG_SAVE_FOR_BWD) == nat.ERR_INVALID  # inference only
    assert call(ld=62) == nat.ERR_INVALID                     # row stride below H * V
    assert call(ld=66) == nat.ERR_INVALID                     # not a multiple of 4
    assert call(gate=0x1002) == nat.ERR_INVALID               # misaligned gate
    assert call(o=0x2004) == nat.ERR_INVALID                  # misaligned output
    assert call(tensors=False) == nat.ERR_INVALID             # null tensors with tokens


def test_serving_arguments_rejected_before_launch(lib):
    from qwendopamine_amd import _native as nat

    def call(h0=None, h0_rows=0, h0_stride=0, ht=None, ht_rows=0, ht_stride=0, idx=None,
             idx_dtype=nat.DTYPE_I64, acc=None, acc_dtype=nat.DTYPE_I32, K=16, V=16, flags=0,
             B=0, T=0):
        return lib.gdn2_recurrent_fwd_ex(None, None, None, None, None, None, 0, 0, None, h0, h0_rows,
                                         h0_stride, ht, ht_rows, ht_stride, None, None, 0.0, None, 0,
                                         idx, idx_dtype, 4, 1, acc, acc_dtype, B, T, 1, 1, K, V, 1.0,
                                         flags, None)

    # No sequences, valid arguments: nothing to launch.
    assert call(h0=256, h0_rows=1, h0_stride=256) == nat.OK
    # State rows overlapping the next row, or not 16-byte aligned.
    assert call(h0=256, h0_rows=1, h0_stride=128) == nat.ERR_INVALID
    assert call(h0=264, h0_rows=1, h0_stride=256) == nat.ERR_INVALID
    assert call(ht=256, ht_rows=1, ht_stride=258) == nat.ERR_INVALID
    # Without a state pool every sequence needs a row.
    assert call(h0=256, h0_rows=0, h0_stride=256, B=1) == nat.ERR_INVALID
    # Index tensors must be int32 / int64.
    assert call(idx=256, idx_dtype=nat.DTYPE_F32) == nat.ERR_INVALID
    assert call(idx=256, acc=512, acc_dtype=nat.DTYPE_BF16) == nat.ERR_INVALID
    # The transposed layout moves K in 16-byte groups.
    assert call(K=18, flags=nat.FLAG_TRANSPOSE_STATE) == nat.ERR_UNSUPPORTED
    # The plain entry point takes neither serving flag.
    st = lib.gdn2_recurrent_fwd(None, None, None, None, None, None, 0, 0, None, None, None, None,
                                None, 0.0, None, 1, 1, 0, 1, 1, 16, 16, 1.0,
                                nat.FLAG_TRANSPOSE_STATE, None)
    assert st == nat.ERR_INVALID


def test_chunk_workspace_size(lib):
    # bf16, K=V=128: 64 KiB of tiles + 512 B of decay per (chunk, head)
    n = lib.gdn2_chunk_fwd_workspace_size(8, 4096, 16, 128, 128, 1, None, 8)
    assert n == 8 * 64 * 16 * (65536 + 512)
    cu = (ctypes.c_int64 * 4)(0, 10, 10, 75)
    n2 = lib.gdn2_chunk_fwd_workspace_size(1, 75, 2, 64, 64, 0, ctypes.cast(cu, ctypes.c_void_p), 3)
    assert n2 == (1 + 0 + 2) * 2 * ((192 * 64 + 8192) * 4 + 64 * 4)
    # d_k in (128, 256]: KP = 256 blobs (X, Aqk 64x64; -W, Qbar 64x256; Ktilde^T 256x64; 256
    # decay floats) for 16-bit inputs.  float32 inputs there take the token-serial wide path:
    # no inference workspace; in training the chunk start states [nc, H, K, V] fp32, and a
    # backward scratch of 64 decayed states per (sequence, head, 128-column slice) plus, with
    # two slices, four [B*T*H, K] planes of the second slice's row sums.  d_k > 256: nothing.
    assert lib.gdn2_chunk_fwd_workspace_size(1, 64, 1, 200, 64, 1, None, 1) == (2 * 4096 + 3 * 16384) * 2 + 256 * 4
    assert lib.gdn2_chunk_fwd_workspace_size(1, 64, 1, 200, 64, 0, None, 1) == 0
    assert lib.gdn2_chunk_fwd_workspace_size(1, 64, 1, 257, 64, 1, None, 1) == 0
    assert lib.gdn2_chunk_train_workspace_size(2, 130, 3, 200, 64, 0, None, 2) == 2 * 3 * 3 * 200 * 64 * 4
    assert lib.gdn2_chunk_bwd_workspace_size(2, 130, 3, 200, 64, 0, None, 2) == 2 * 3 * 64 * 4 * 16 * 64 * 16
    assert lib.gdn2_chunk_bwd_workspace_size(2, 130, 3, 200, 200, 0, None, 2) == (
        2 * 3 * 2 * 64 * 8 * 16 * 64 * 16 + 4 * 2 * 130 * 3 * 200 * 4)


def test_gate_argument_checks(lib):
    """The gate entry points reject bad arguments before any launch (no GPU needed)."""
    from qwendopamine_amd import _native as nat

    assert lib.gdn2_gate_bwd_workspace_size(1000, 3, 257, 1) == 0
    # 16 blocks of 64 tokens: dA_log partials [16, 3] and ddt_bias partials [16, 3, 100], 256-byte aligned
    assert lib.gdn2_gate_bwd_workspace_size(1000, 3, 100, 1) == 256 + 16 * 3 * 100 * 4
    assert lib.gdn2_gate_bwd_workspace_size(1000, 3, 100, 0) == 256
    fake = ctypes.c_void_p(256)  # never dereferenced: each call returns before launching
    assert lib.gdn2_gate_fwd(fake, 0, fake, None, 0.0, 0, fake, 10, 3, 257, None) == nat.ERR_UNSUPPORTED
    assert lib.gdn2_gate_fwd(None, 0, fake, None, 0.0, 0, fake, 10, 3, 100, None) == nat.ERR_INVALID
    assert lib.gdn2_gate_fwd(fake, 0, None, None, 0.0, 0, fake, 10, 3, 100, None) == nat.ERR_INVALID
    assert lib.gdn2_gate_fwd(fake, 0, fake, None, 0.0, nat.FLAG_L2NORM_QK, fake, 10, 3, 100, None) == nat.ERR_INVALID
    assert lib.gdn2_gate_bwd(fake, 0, fake, fake, 0.0, 0, fake, fake, fake, None, 10, 3, 100, fake, 1 << 20,
                             None) == nat.ERR_INVALID
    assert lib.gdn2_gate_bwd(fake, 0, fake, None, 0.0, 0, fake, fake, fake, None, 10, 3, 100, fake, 8,
                             None) == nat.ERR_WORKSPACE

