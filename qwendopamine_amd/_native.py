"""ctypes binding of ``libgdn2_hip.so`` (C ABI declared in ``include/gdn2_hip.h``).

The library is the only compute path of this package: there is no CPU or
PyTorch fallback, and every failure to load it or to launch a kernel raises.
``torch`` is imported before the library is opened so that the library binds
to the HIP runtime torch already loaded (one runtime per process).
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch  # noqa: F401  (must precede dlopen of the HIP library)

LIB_PATH = Path(os.environ.get("GDN2_HIP_LIB", Path(__file__).with_name("libgdn2_hip.so")))
ABI_VERSION = 2

DTYPE_F32 = 0
DTYPE_BF16 = 1
DTYPE_F16 = 2
DTYPE_I32 = 3
DTYPE_I64 = 4

FLAG_L2NORM_QK = 1
FLAG_GATE_IN_KERNEL = 2
FLAG_LOWER_BOUND = 4
FLAG_SAVE_FOR_BWD = 8
FLAG_TRANSPOSE_STATE = 16
FLAG_INPLACE_FINAL_STATE = 32
FLAG_SIGMOID_BW = 64

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_LAUNCH = -3
ERR_WORKSPACE = -4
ERR_SCRATCH = -5
STATIC_SCRATCH_BYTES = 75497472  # GDN2_STATIC_SCRATCH_BYTES

_vp = ctypes.c_void_p
_i = ctypes.c_int
_f = ctypes.c_float
_u = ctypes.c_uint
_sz = ctypes.c_size_t
_i64 = ctypes.c_int64

# Every exported symbol with its ctypes signature (restype, argtypes).
SIGNATURES: dict[str, tuple] = {
    "gdn2_abi_version": (_i, []),
    "gdn2_status_string": (ctypes.c_char_p, [_i]),
    "gdn2_recurrent_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _f, _vp, _i,
         _i, _i, _i, _i, _i, _i, _f, _u, _vp],
    ),
    "gdn2_recurrent_fwd_ex": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _i64, _i64, _vp, _i64, _i64, _vp, _vp,
         _f, _vp, _i, _vp, _i, _i64, _i64, _vp, _i, _i, _i, _i, _i, _i, _i, _f, _u, _vp],
    ),
    "gdn2_short_conv_fwd": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    ),
    "gdn2_short_conv_fwd_ex": (
        _i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _vp],
    ),
    "gdn2_gated_rmsnorm_fwd": (_i, [_vp, _vp, _vp, _i, _vp, _i, _i64, _i, _f, _vp]),
    "gdn2_add_rms_norm_fwd": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _i64, _i, _f, _vp]),
    "gdn2_silu_mul_fwd": (_i, [_vp, _i64, _vp, _i, _i64, _i, _vp]),
    "gdn2_skinny_linear": (_i, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i, _i, _i, _i, _vp]),
    "gdn2_skinny_linear_addnorm": (_i, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _f, _vp, _i64, _vp, _vp, _i64, _i, _i,
                                        _i, _i, _vp]),
    "gdn2_skinny_linear_addnorm_swiglu": (_i, [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _f, _vp, _i64, _vp, _vp, _i64,
                                               _i, _i, _i, _i, _vp]),
    "gdn2_small_linear_pair": (_i, [_vp, _i64, _vp, _vp, _vp, _i64, _i, _vp, _i64, _vp, _vp, _vp, _i64, _i, _i, _i,
                                    _i, _vp]),
    "gdn2_argmax_rows_workspace_size": (_sz, [_i64, _i64, _i]),
    "gdn2_argmax_rows": (_i, [_vp, _i64, _i, _i64, _i64, _vp, _i64, _vp, _sz, _vp]),
    "gdn2_attn_decode_workspace_size": (_sz, [_i, _i, _i, _i, _i64]),
    "gdn2_attn_decode": (_i, [_vp, _vp, _vp, _i, _i64, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i64, _f, _vp, _sz, _vp]),
    "gdn2_decode_fused": (
        _i,
        [_vp, _vp, _vp, _i64, _i, _vp, _i64, _vp, _i64, _vp, _vp, _i, _vp, _vp, _vp, _i64, _vp, _i64,
         _vp, _vp, _f, _vp, _i64, _vp, _i, _f, _vp, _i, _i, _i, _i, _i, _f, _u, _vp],
    ),
    "gdn2_chunk_states": (_i, [_vp, _sz, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "gdn2_chunk_fwd_workspace_size": (_sz, [_i, _i, _i, _i, _i, _i, _vp, _i]),
    "gdn2_chunk_fwd": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp,
         _i, _i, _i, _i, _i, _i, _f, _u, _vp, _sz, _vp],
    ),
    "gdn2_gate_bwd_workspace_size": (_sz, [_i64, _i, _i, _i]),
    "gdn2_gate_fwd": (_i, [_vp, _i, _vp, _vp, _f, _u, _vp, _i64, _i, _i, _vp]),
    "gdn2_gate_bwd": (
        _i,
        [_vp, _i, _vp, _vp, _f, _u, _vp, _vp, _vp, _vp, _i64, _i, _i, _vp, _sz, _vp],
    ),
    "gdn2_short_conv_bwd_workspace_size": (_sz, [_i, _i, _i, _i]),
    "gdn2_short_conv_bwd": (
        _i,
        [_vp, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp],
    ),
    "gdn2_gated_rmsnorm_bwd_workspace_size": (_sz, [_i64, _i]),
    "gdn2_gated_rmsnorm_bwd": (
        _i,
        [_vp, _vp, _vp, _i, _vp, _vp, _vp, _vp, _i, _i64, _i, _f, _vp, _sz, _vp],
    ),
    "gdn2_chunk_fwd_gated_norm": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _i64, _vp, _f, _vp, _vp, _vp, _vp, _f,
         _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _u, _vp, _sz, _vp],
    ),
    "gdn2_chunk_fwd_conv": (
        _i,
        [_vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _i, _i, _vp, _vp, _i64,
         _vp, _f, _vp, _vp, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _u, _vp, _sz, _vp],
    ),
    "gdn2_chunk_fwd_static": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _f, _vp, _vp,
         _i, _i, _i, _i, _i, _i, _f, _u, _vp],
    ),
    "gdn2_chunk_fwd_prep": (
        _i,
        [_vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _f, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _u,
         _vp, _sz, _vp],
    ),
    "gdn2_chunk_fwd_scan": (
        _i,
        [_vp, _vp, _i, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp, _sz, _vp],
    ),
    "gdn2_chunk_train_workspace_size": (_sz, [_i, _i, _i, _i, _i, _i, _vp, _i]),
    "gdn2_chunk_bwd_workspace_size": (_sz, [_i, _i, _i, _i, _i, _i, _vp, _i]),
    "gdn2_chunk_bwd": (
        _i,
        [_vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
         _vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _f, _u, _vp, _sz, _vp, _sz, _vp],
    ),
}

_LIB: ctypes.CDLL | None = None


class GDN2KernelError(RuntimeError):
    """A gdn2 HIP entry point returned a non-zero status."""


def load() -> ctypes.CDLL:
    """Open the HIP library once and declare every entry point."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"gdn2 HIP library not found at {LIB_PATH}; build it with "
            "`python -m qwendopamine_amd.build` (hipcc, gfx950). This package has no "
            "CPU fallback."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.gdn2_abi_version()
    if ver != ABI_VERSION:
        raise RuntimeError(f"gdn2 HIP library ABI {ver} != expected {ABI_VERSION}")
    _LIB = lib
    return lib


def check(status: int, what: str) -> None:
    """Map a gdn2_status to the reference's exception types."""
    if status == OK:
        return
    msg = load().gdn2_status_string(status).decode()
    if status in (ERR_INVALID, ERR_SCRATCH):
        raise ValueError(f"{what}: {msg}")
    if status == ERR_UNSUPPORTED:
        raise NotImplementedError(f"{what}: {msg}")
    raise GDN2KernelError(f"{what}: {msg} (status {status})")


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    if dt == torch.float16:
        return DTYPE_F16
    raise NotImplementedError(f"gdn2 HIP kernels support float32/bfloat16/float16, not {dt}")


def index_dtype_code(t: torch.Tensor | None) -> int:
    """Dtype code of an index tensor (int32 / int64); int64 when absent."""
    if t is None or t.dtype == torch.int64:
        return DTYPE_I64
    if t.dtype == torch.int32:
        return DTYPE_I32
    raise NotImplementedError(f"gdn2 index tensors must be int32/int64, not {t.dtype}")


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream
