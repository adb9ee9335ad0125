"""ctypes binding of the in-tree HIP library ``libboundflow_hip.so``.

The library is loaded after ``import torch`` so that it binds to the HIP
runtime torch already mapped (both carry the SONAME ``libamdhip64.so.7``); one
runtime per process.  There is no CPU fallback: if the library is missing or a
call fails, the error is raised to the caller.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path
from typing import Optional

import torch

from . import profiling

LIB_PATH = Path(__file__).resolve().parent / "libboundflow_hip.so"

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int
F32 = ctypes.c_float
F64 = ctypes.c_double

# name -> (restype, argtypes); every entry point listed in include/boundflow_hip.h
SIGNATURES = {
    "bf_abi_version": (I32, []),
    "bf_last_error": (ctypes.c_char_p, []),
    "bf_gemm_tile_config": (I32, [I64, I64, I32, I32, I32, I32]),
    "bf_gemm": (I32, [P, I64, P, I64, I32, I32, P, I64, I64, I64, I64, P]),
    "bf_gemm_rank1": (I32, [P, I64, P, I64, I32, P, I64, I64, I64, I64, I64, P, P, I64, P, I64, P]),
    "bf_gemm_rank1_workspace": (I64, [I64, I64, I64]),
    "bf_relu_relax_table": (I32, [P, P, P, I64, I64, I64, P, P]),
    "bf_relu_relax_table_multi": (I32, [I32, P, P, P, P, I64, P, P, P]),
    "bf_crown_relu_linear_fwd": (I32, [P, P, I64, I64, I64, I64, P, P, I64, P, I64, I32, P, P, P, P, P, P, P, P]),
    "bf_relu_relax_table_from_planes": (I32, [P, P, P, P, I64, P, P]),
    "bf_crown_relu_planes_conv_transpose": (I32, [P, P, I64, I64, I32, I32, I32, P, P, P, P, P, P, P, P, P, I32, I32,
                                                  I32, I32, I32, I32, I32, I32, I32, P, P, P, P, P]),
    "bf_crown_relu_linear_concretize": (I32, [P, P, I64, I64, I64, I64, P, P, I64, P, I64, I32, P, P, P, F32, I32, P,
                                              P, P, P, P, P, P, P]),
    "bf_crown_relu_linear_concretize_workspace": (I64, [I64, I64, I64]),
    "bf_crown_relu_linear_concretize_noalloc": (I32, [P, P, I64, I64, I64, I64, P, P, I64, P, I64, I32, P, P, P, F32,
                                                      I32, P, P, P, P, P, P, P]),
    "bf_crown_relu_linear_relu_fwd": (I32, [P, P, I64, I64, I64, I64, P, P, I64, P, I64, P, P, P, P, P, I64, P, P,
                                            I64, P, P, P, P, P, P, P, P, P, P]),
    "bf_crown_relu_linear_relu_fwd_workspace": (I64, [I64, I64, I64]),
    "bf_crown_linear_concretize": (I32, [P, P, I64, I64, I64, I64, P, I64, P, F32, I32, P, P, P, P, P, P, P, P, P,
                                         P]),
    "bf_crown_linear_concretize_workspace": (I64, [I64, I64, I64]),
    "bf_crown_relu_relax": (I32, [P, P, I64, I64, I64, I64, P, P, I64, P, P, P, P, P, P, P, P, P, P, P]),
    "bf_crown_relu_relax_lu": (I32, [P, P, I64, I64, I64, I64, P, P, P, I64, P, I64, P, P, P, P, P, P, P, P, P, P,
                                     P]),
    "bf_concretize_dense": (I32, [P, I64, I64, I64, P, P, F32, I32, P, I32, P, P]),
    "bf_concretize_dense_grad": (I32, [P, I64, I64, I64, P, P, F32, I32, P, P, P]),
    "bf_rows_abs_max": (I32, [P, P, I64, I64, I64, P, P]),
    "bf_rows_add": (I32, [P, P, I64, I64, I64, P, P, I64, P, P]),
    "bf_ibp_linear": (I32, [P, P, I64, I64, I32, F32, I32, P, P, I64, P, I64, P, P, P, P, P, P, P]),
    "bf_ibp_linear_workspace": (I64, [I64, I64, I64]),
    "bf_interval_clip": (I32, [P, P, P, P, P, I64, I64, I64, P, P]),
    "bf_interval_relu": (I32, [P, P, I64, P, P, P]),
    "bf_interval_center_radius": (I32, [P, P, I64, I32, P, P, P]),
    "bf_interval_add": (I32, [P, P, P, P, I64, P, P, P]),
    "bf_interval_mul": (I32, [P, P, P, P, I64, P, P, P]),
    "bf_spec_linear": (I32, [P, P, P, I64, I64, I64, P, P, P]),
    "bf_ibp_batched_linear": (I32, [P, P, I64, I64, P, P, I64, P, P, P]),
    "bf_branch_update": (I32, [P, P, I64, I64, I32, P, P, P, P]),
    "bf_alpha_adaptive": (I32, [P, P, I64, P, P]),
    "bf_objective_step": (I32, [P, P, I64, I64, I32, I32, F32, F32, F32, F32, P, P, P, P, P, P, P, I32, P]),
    "bf_scale_rows": (I32, [P, I64, I64, P, P]),
    "bf_branch_update_native": (I32, [P, P, P, I64, I64, I64, I32, P, P, P, P, P, P]),
    "bf_split_certificate": (I32, [P, I64, P, P, I64, P, I64, P, I64, F32, I32, I64, I64, I64, I32, F64, F64, P, P,
                                   P]),
    "bf_adam_clamp_step": (I32, [P, P, P, P, I64, F64, F64, F64, F32, I32, F32, F32, I32, P]),
    "bf_adam_clamp_multi": (I32, [I32, P, P, P, P, P, P, P, P, F64, F64, F64, F32, I32, P, P, I64, P]),
    "bf_conv2d_rows": (I32, [P, I64, I64, I32, I32, I32, P, I32, I32, I32, I32, I32, I32, I32, I32, I32, I32, P, P, P,
                             I64, I64, P]),
    "bf_conv_transpose_rows": (I32, [P, P, I64, I32, I32, I32, P, I32, I32, I32, I32, I32, I32, I32, I32, I32, P, P,
                                     I64, P, I64, I32, P, P, P, P, P]),
    "bf_conv_transpose_hwc_supported": (I32, [I32] * 12),
    "bf_crown_relu_conv_transpose": (I32, [P, P, I64, I64, I32, I32, I32, P, P, P, I64, P, I64, P, P, P, P, P, I32, I32,
                                           I32, I32, I32, I32, I32, I32, I32, P, P, P, P, P, P, P]),
    "bf_conv_transpose_small_supported": (I32, [I32] * 12),
    "bf_crown_relu_conv_transpose_concretize": (I32, [P, P, I64, I64, I32, I32, I32, P, P, P, I64, P, I64, P, P, P, P, P]
                                                + [I32] * 9 + [P, I64, I32, P, P, P, P, P, P, P, P, P, P, F32, P, P,
                                                               P]),
    "bf_conv_transpose_packed_floats": (I64, [I32] * 12),
    "bf_conv_transpose_pack_weights": (I32, [P] + [I32] * 12 + [P, P]),
    "bf_ibp_conv2d": (I32, [P, P, I64, I32, I32, I32, I32, F32, I32, P, P, I32, I32, I32, I32, I32, I32, I32, I32, I32,
                            P, I64, P, P, P, P, P, P]),
    "bf_ibp_conv2d_workspace": (I64, [I64, I64, I64]),
    "bf_relu_grad": (I32, [P, P, I64, I64, I64, I64, P, P, P, I64, P, P, I64, P, P, P, P]),
    "bf_beta_coeff": (I32, [P, I64, P, I64, I64, I64, P, P]),
    "bf_beta_coeff_multi": (I32, [I32, P, P, P, P, P, I64, P, P]),
    "bf_best_update": (I32, [P, P, I64, I64, P, P, P, P, I32, P]),
    "bf_masked_copy_rows": (I32, [P, P, I64, I64, P, P]),
    "bf_masked_copy_rows_multi": (I32, [I32, P, P, P, I64, P, P]),
    "bf_sum_rows": (I32, [P, I64, I64, P, P]),
    "bf_concretize_finalize": (I32, [P, P, I32, I64, P, P, P, P, F32, I32, P, P, P]),
    "bf_alpha_from_crown": (I32, [P, P, I64, P, P]),
    "bf_domain_status": (I32, [P, I64, I64, P, F32, F32, P, P]),
}

_lib: Optional[ctypes.CDLL] = None


class HipError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Load (once) and return the library; raise if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise HipError(
            f"{LIB_PATH} is missing: build it with `python -m boundflow_amd.build` "
            "(the HIP backend has no CPU fallback)")
    lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.bf_abi_version() != 1:
        raise HipError("libboundflow_hip ABI version mismatch")
    _lib = lib
    return lib


class DevicePtr(ctypes.c_void_p):
    """A tensor's address that keeps the tensor alive.  Arguments such as
    ``ptr(x.contiguous())`` may be temporaries; held here, they survive until
    the call that receives them has enqueued its kernels, so the caching
    allocator cannot hand their memory to a later argument of the same call
    (later reuse is ordered after the launch on the stream)."""

    def __init__(self, t: torch.Tensor):
        super().__init__(t.data_ptr())
        self.tensor = t


def ptr(t: Optional[torch.Tensor]):
    if t is None:
        return None
    return DevicePtr(t)


class HostArray:
    """A host array argument of a multi-tensor entry point (device pointers or
    sizes); keeps the tensors whose addresses it holds alive."""

    def __init__(self, ctype, values, keep=()):
        self.buf = (ctype * max(1, len(values)))(*values)
        self.keep = tuple(keep)

    @property
    def _as_parameter_(self):
        return ctypes.cast(self.buf, ctypes.c_void_p)


def ptr_array(tensors) -> HostArray:
    """Host array of the device addresses of ``tensors`` (None -> NULL)."""
    return HostArray(ctypes.c_void_p, [None if t is None else t.data_ptr() for t in tensors],
                     keep=[t for t in tensors if t is not None])


def i64_array(values) -> HostArray:
    return HostArray(ctypes.c_int64, [int(v) for v in values])


def i32_array(values) -> HostArray:
    return HostArray(ctypes.c_int32, [int(v) for v in values])


def f32_array(values) -> HostArray:
    return HostArray(ctypes.c_float, [float(v) for v in values])


def stream_handle(stream: Optional[torch.cuda.Stream] = None):
    s = stream if stream is not None else torch.cuda.current_stream()
    return ctypes.c_void_p(s.cuda_stream)


def call(name: str, *args) -> int:
    """Invoke an entry point and raise HipError with bf_last_error() on failure."""
    lib = load()
    fn = getattr(lib, name)
    profiling.begin_call()
    rc = fn(*args)
    profiling.end_call()
    if SIGNATURES[name][0] is I32 and name != "bf_abi_version" and rc != 0:
        msg = lib.bf_last_error().decode(errors="replace")
        raise HipError(f"{name} failed (status {rc}): {msg}")
    return rc


def require_device(t: torch.Tensor, name: str) -> None:
    if not t.is_cuda:
        raise HipError(f"{name} must be a HIP device tensor (the backend has no CPU path)")
    if t.dtype != torch.float32 and t.dtype not in (torch.int8, torch.int32):
        raise HipError(f"{name} must be float32, got {t.dtype}")
    if not t.is_contiguous():
        raise HipError(f"{name} must be contiguous")


def loaded_path() -> str:
    return str(LIB_PATH)


def library_exports(path: Optional[str] = None):
    """Names of SIGNATURES that the shared object exports (no device call)."""
    lib = ctypes.CDLL(str(path or LIB_PATH))
    return [n for n in SIGNATURES if hasattr(lib, n)]


def env_flag(name: str) -> bool:
    return os.environ.get(name, "") not in ("", "0", "false", "False")
