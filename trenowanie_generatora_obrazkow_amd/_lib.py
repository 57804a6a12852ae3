"""ctypes binding of libhmoe.so (the C ABI declared in include/hmoe.h).

The library is built in-tree (trenowanie_generatora_obrazkow_amd/_lib/libhmoe.so, by build.py).  There is no CPU
or PyTorch fallback: if the library is missing, every call raises.
"""
from __future__ import annotations

import ctypes
import os

import torch

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_lib", "libhmoe.so")

DT_BF16, DT_F16, DT_F32, DT_I32, DT_I64, DT_I8 = 0, 1, 2, 3, 4, 5
_DT = {torch.bfloat16: DT_BF16, torch.float16: DT_F16, torch.float32: DT_F32, torch.int32: DT_I32,
       torch.int64: DT_I64, torch.int8: DT_I8}

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/hmoe.h
SIGNATURES = {
    "hmoe_abi_version": (_I32, []),
    "hmoe_error_string": (ctypes.c_char_p, [_I32]),
    "hmoe_route_topk": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I32, _I32, _I32, _F32, _P, _P, _P, _P]),
    "hmoe_route_sigmoid_group": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I32, _I32, _I32, _I32, _F32, _P, _P, _P,
                                        _P]),
    "hmoe_dispatch_workspace_size": (_SZ, [_I64, _I32, _I32]),
    "hmoe_dispatch": (_I32, [_P, _I32, _P, _I32, _I64, _I32, _I32, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P, _P,
                             _P, _P, _SZ, _I32, _P]),
    "hmoe_dispatch_noalloc": (_I32, [_P, _I32, _P, _I32, _I64, _I32, _I32, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                                     _P, _P, _I32, _P]),
    "hmoe_make_schedule": (_I32, [_P, _I32, _I32, _I64, _I32, _P, _P, _P, _P]),
    "hmoe_grouped_mm": (_I32, [_P, _I64, _I32, _P, _I32, _I64, _I64, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P,
                               _I32, _P, _I32, _P, _I64, _P]),
    "hmoe_gate_up_swiglu": (_I32, [_P, _I64, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _I32, _P]),
    "hmoe_gate_up_swiglu_tiles": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _I32, _P]),
    "hmoe_xs_tiles_bytes": (_SZ, [_I64, _I32, _I64]),
    "hmoe_dispatch_tiles": (_I32, [_P, _I32, _P, _I32, _I64, _I32, _I32, _P, _I64, _I64, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _P, _P, _P, _SZ, _I32, _P]),
    "hmoe_down_scatter": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P, _P, _I32, _P]),
    "hmoe_gate_up_swiglu_i8": (_I32, [_P, _I64, _P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P, _I32, _P]),
    "hmoe_down_scatter_i8": (_I32, [_P, _P, _P, _I32, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P, _I32, _P]),
    "hmoe_combine": (_I32, [_P, _P, _I64, _I32, _I64, _P, _I32, _P]),
    "hmoe_moe_forward_workspace_size": (_SZ, [_I64, _I64, _I32, _I32, _I64]),
    "hmoe_moe_experts_workspace_size": (_SZ, [_I64, _I64, _I32, _I32, _I64, _I32, _I32]),
    "hmoe_moe_experts": (_I32, [_P, _I64, _P, _I32, _P, _I32, _P, _P, _I32, _P, _P, _I32, _I32, _I64, _I64, _I32,
                                _I32, _I64, _P, _P, _P, _P, _SZ, _I32, _P]),
    "hmoe_moe_forward": (_I32, [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I32, _I32, _I64, _I32, _F32, _P, _P, _P, _P,
                                _P, _SZ, _P]),
    "hmoe_combine_add": (_I32, [_P, _P, _I64, _I32, _I64, _P, _P, _I32, _P]),
    "hmoe_combine_bwd": (_I32, [_P, _P, _P, _P, _P, _I64, _I32, _I64, _P, _P, _P]),
    "hmoe_down_dgrad_swiglu": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P]),
    "hmoe_down_dgrad_dw_workspace_size": (_SZ, [_I64, _I64]),
    "hmoe_down_dgrad_swiglu_dw": (_I32, [_P, _P, _P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _P, _P, _P, _P, _SZ,
                                         _P]),
    "hmoe_gate_up_dgrad": (_I32, [_P, _P, _I64, _I64, _I64, _P, _I32, _I64, _P, _I32, _P]),
    "hmoe_grouped_wgrad": (_I32, [_P, _I64, _P, _I64, _I64, _I64, _I64, _P, _I32, _I64, _P, _I32, _P]),
    "hmoe_router_bwd_workspace_size": (_SZ, [_I64, _I32, _I64]),
    "hmoe_router_bwd": (_I32, [_P, _P, _P, _I64, _I32, _I32, _I32, _F32, _P, _I64, _I64, _P, _P, _I32, _P, _SZ,
                               _P]),
    "hmoe_unpermute_bwd": (_I32, [_P, _I32, _P, _P, _P, _I64, _I32, _I64, _I32, _P, _P]),
}

_lib = None


def lib():
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"hmoe HIP library not built ({LIB_PATH}); run `python -c \"import __graft_entry__ as g; "
                               f"g.build()\"` or trenowanie_generatora_obrazkow_amd/build.py")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class HmoeError(RuntimeError):
    def __init__(self, name, code):
        msg = lib().hmoe_error_string(code).decode()
        super().__init__(f"{name} failed with code {code}: {msg}")
        self.code = code


def call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != 0:
        raise HmoeError(name, rc)


def dt(t_or_dtype) -> int:
    d = t_or_dtype.dtype if isinstance(t_or_dtype, torch.Tensor) else t_or_dtype
    if d not in _DT:
        raise TypeError(f"unsupported dtype {d}")
    return _DT[d]


def ptr(t):
    return None if t is None else t.data_ptr()


# torch's raw current-stream lookup (what its generated kernels launch on), without building a Stream object: the
# per-op stream query is otherwise a visible part of the host time of a small layer call
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream(device=None):
    """Handle of the current stream of `device` (a torch.device, an index or None for the current device)."""
    if _raw_stream is not None:
        if isinstance(device, torch.device):
            device = device.index
        return _raw_stream(torch.cuda.current_device() if device is None else device)
    return torch.cuda.current_stream(device).cuda_stream


def require_gpu(t: torch.Tensor, name: str):
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a ROCm GPU tensor: the hmoe kernels have no CPU path")
