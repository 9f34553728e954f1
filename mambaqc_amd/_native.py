"""ctypes binding of libmambaqc_hip.so (declared in include/mambaqc_hip.h).

The library is the only compute path of this package: there is no CPU or
torch fallback. Loading fails loudly with the build command if the library is
absent, and every entry point checks that its tensors live on a ROCm device.

torch is imported before the library is opened so that the HIP runtime torch
ships (soname libamdhip64.so.7) is the one the library binds to; streams and
device pointers handed across are then valid on both sides.
"""
from __future__ import annotations

import ctypes
import weakref
import os
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "lib" / "libmambaqc_hip.so"

F32, BF16, F16 = 0, 1, 2
_DTYPES = {torch.float32: F32, torch.bfloat16: BF16, torch.float16: F16}

_vp = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> argtypes (all return int status)
SIGNATURES = {
    "mqc_quaternion_multiply": [_vp, _vp, _vp, _i64, _int, _vp],
    "mqc_quaternion_conjugate": [_vp, _vp, _i64, _int, _vp],
    "mqc_quaternion_inverse": [_vp, _vp, _i64, _f32, _int, _vp],
    "mqc_quaternion_norm": [_vp, _vp, _i64, _int, _vp],
    "mqc_cayley_fwd": [_vp, _vp, _i64, _f32, _int, _vp],
    "mqc_cumprod_scan_fwd": [_vp, _vp, _i64, _i64, _i64, _int, _vp],
    "mqc_ssm_q_fwd": [_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp,
                      _i64, _i64, _i64, _i64, _int, _vp],
    "mqc_ssm_fused_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                          _i64, _i64, _i64, _i64, _f32, _int, _vp],
    "mqc_qln_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _vp],
    "mqc_out_gate_fwd": [_vp, _vp, _i64, _vp, _vp, _i64, _i64, _int, _vp],
    "mqc_ssm_bwd_ckpt_every": [_int],
    "mqc_ssm_fused_fwd_train": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64,
                                _i64, _i64, _i64, _i64, _f32, _int, _vp],
    "mqc_ssm_fused_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _vp,
                          _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _int, _vp],
    "mqc_qln_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _int, _vp],
    "mqc_out_gate_bwd": [_vp, _vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp],
    "mqc_ssm_front_fwd": [_vp, _vp, _vp, _vp, _vp, _i64, _int, _vp],
    "mqc_ssm_front_bwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _int, _vp],
    "mqc_causal_conv_silu_fwd": [_vp, _i64, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _vp],
    "mqc_conv_run_length": [],
    "mqc_causal_conv_silu_bwd": [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _i64,
                                 _i64, _i64, _int, _vp],
    "mqc_causal_conv_silu_step": [_vp, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _int, _vp],
    "mqc_ssm_fused_fwd_chunked": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                  _i64, _i64, _i64, _i64, _i64, _f32, _int, _vp, _i64, _vp],
    "mqc_gemm_nt": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp],
    "mqc_gemm_skinny_nt": [_vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp, _vp, _i64, _int, _vp],
    "mqc_ssm_fused_fwd_train_chunked": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                        _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _vp,
                                        _i64, _vp],
    "mqc_ssm_fused_bwd_chunked": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                                  _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                  _i64, _i64, _f32, _int, _vp, _i64, _vp],
    "mqc_ssm_fused_fwd_chunked_noalloc": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                          _i64, _i64, _i64, _i64, _i64, _f32, _int, _vp],
    "mqc_ssm_noalloc_prepare": [],
    "mqc_ssm_fused_bc_fwd": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                             _i64, _i64, _i64, _i64, _f32, _int, _vp],
    "mqc_ssm_fused_bc_fwd_split": [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp,
                                   _i64, _i64, _i64, _i64, _f32, _int, _vp, _i64, _vp],
    "mqc_out_proj_gate_fwd": [_vp, _vp, _vp, _vp, _vp, _i64, _vp, _i64, _i64, _i64, _int, _vp],
}

# name -> argtypes of the entry points that return int64_t (a size, or a
# negative status code)
SIGNATURES_I64 = {
    "mqc_ssm_chunk_len_auto": [_i64, _i64, _i64, _i64, _int],
    "mqc_ssm_chunked_workspace_bytes": [_i64, _i64, _i64, _i64, _i64],
    "mqc_ssm_chunked_scratch_bytes": [],
    "mqc_ssm_fused_bc_split_workspace_bytes": [_i64, _i64, _i64, _i64],
}

ABI_VERSION = 8

_lock = threading.Lock()
_lib = None


class NativeLibraryMissing(RuntimeError):
    pass


def load(path: os.PathLike | str | None = None) -> ctypes.CDLL:
    """Open the library once per process and declare every entry point."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    with _lock:
        if _lib is not None and path is None:
            return _lib
        p = Path(path) if path is not None else LIB_PATH
        if not p.exists():
            raise NativeLibraryMissing(
                f"{p} is missing: build it with `python -m mambaqc_amd.build` "
                "(mambaqc_amd has no CPU fallback)")
        lib = ctypes.CDLL(str(p))
        for name, argtypes in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _int
        for name, argtypes in SIGNATURES_I64.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = _i64
        lib.mqc_status_string.argtypes = [_int]
        lib.mqc_status_string.restype = ctypes.c_char_p
        lib.mqc_abi_version.argtypes = []
        lib.mqc_abi_version.restype = _int
        if lib.mqc_abi_version() != ABI_VERSION:
            raise NativeLibraryMissing(
                f"{p}: ABI version {lib.mqc_abi_version()} != {ABI_VERSION}; rebuild")
        if path is None:
            _lib = lib
        return lib


def status_string(status: int) -> str:
    return load().mqc_status_string(status).decode()


def check(status: int, name: str) -> None:
    if status != 0:
        raise RuntimeError(f"{name} failed with status {status}: {status_string(status)}")


def dtype_code(t: torch.Tensor) -> int:
    try:
        return _DTYPES[t.dtype]
    except KeyError:
        raise TypeError(f"unsupported dtype {t.dtype}; expected float32, bfloat16 or float16") from None


def require_device(name: str, *tensors: torch.Tensor) -> None:
    for t in tensors:
        if not t.is_cuda:
            raise RuntimeError(
                f"mambaqc_amd.{name}: expected tensors on a ROCm device, got {t.device}; "
                "this package runs only on the GPU")
    dev = tensors[0].device
    for t in tensors[1:]:
        if t.device != dev:
            raise RuntimeError(f"mambaqc_amd.{name}: tensors on different devices ({dev}, {t.device})")


def compiling() -> bool:
    """True while torch.compile traces: the Python API then calls the
    registered torch.ops.mambaqc.* operators (traceable through their fake
    kernels) instead of ctypes."""
    return torch.compiler.is_compiling()


def stream_of(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def aligned16(t: torch.Tensor) -> torch.Tensor:
    """Contiguous and 16-byte aligned (the kernels' vector width)."""
    t = t.contiguous()
    if t.data_ptr() % 16 != 0:
        t = t.clone()
    return t


# Converted copies of parameters by id(), dropped when the parameter object
# dies (kept off the tensor itself so that pickling a module does not carry them).
_F32_CACHE: dict = {}


def param_f32(t: torch.Tensor) -> torch.Tensor:
    """fp32, contiguous, 16-byte aligned form of a parameter-like tensor (the
    kernels read Lambda, D, gamma, beta and conv weights in fp32 whatever the
    model dtype). An fp32 tensor that already qualifies is used as is; other
    conversions are cached and redone when the tensor's data pointer, shape or
    version counter (bumped by every in-place update) changes. Inference
    tensors (made in inference mode) have no version counter and are converted
    on every call. The cached conversions are made with inference mode off,
    also when the call comes from inside it: a conversion made in inference
    mode would be an inference tensor, which autograd could not save if the
    cache handed it to a later training step."""
    if t.dtype == torch.float32 and t.is_contiguous() and t.data_ptr() % 16 == 0:
        return t.detach()
    if t.is_inference():
        return aligned16(t.detach().float())
    key = (t._version, t.data_ptr(), t.dtype, tuple(t.shape))
    hit = _F32_CACHE.get(id(t))
    if hit is not None and hit[0]() is t and hit[1] == key:
        return hit[2]
    with torch.inference_mode(False):
        conv = aligned16(t.detach().float())
    if hit is None or hit[0]() is not t:
        weakref.finalize(t, _F32_CACHE.pop, id(t), None)
    _F32_CACHE[id(t)] = (weakref.ref(t), key, conv)
    return conv


def call(name: str, device_tensor: torch.Tensor, *args) -> None:
    """Call entry point `name` with the tensor's device current (the library
    launches on the device that is current; the stream argument must belong to
    it). The device switch is skipped when it is current already."""
    fn = getattr(load(), name)
    idx = device_tensor.device.index
    if idx is None or idx == torch.cuda.current_device():
        status = fn(*args)
    else:
        with torch.cuda.device(idx):
            status = fn(*args)
    check(status, name)
