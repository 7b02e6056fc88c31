"""ctypes boundary to ``libq3t_amd.so`` (the C ABI declared in include/qwen3tts_amd.h).

PyTorch supplies device memory and the current HIP stream; every computation happens in
the HIP kernels behind this library.  There is no CPU or eager-torch fallback: if the
library is missing or a call is rejected, the wrappers raise.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIBRARY_PATH = Path(__file__).resolve().parent / "libq3t_amd.so"

Q3T_OK = 0
Q3T_EINVAL = -1
Q3T_EUNSUPPORTED = -2
Q3T_EWORKSPACE = -3

Q3T_BF16, Q3T_F16, Q3T_F32, Q3T_BOOL = 0, 1, 2, 3
DTYPE_CODES = {torch.bfloat16: Q3T_BF16, torch.float16: Q3T_F16, torch.float32: Q3T_F32,
               torch.bool: Q3T_BOOL}

c_i64 = ctypes.c_int64
c_vp = ctypes.c_void_p
I64x3 = c_i64 * 3


class DecodeArgs(ctypes.Structure):
    """Mirror of ``q3t_decode_args``."""
    _fields_ = [
        ("batch", c_i64), ("query_len", c_i64), ("q_heads", c_i64), ("kv_heads", c_i64),
        ("head_dim", c_i64), ("ctx", c_i64), ("dtype", c_i64), ("scale", ctypes.c_float),
        ("fused", ctypes.c_int32),
        ("query", c_vp), ("q_stride_b", c_i64), ("q_stride_s", c_i64), ("q_stride_h", c_i64),
        ("keys", c_vp), ("values", c_vp),
        ("k_stride_b", c_i64), ("k_stride_h", c_i64), ("k_stride_t", c_i64),
        ("v_stride_b", c_i64), ("v_stride_h", c_i64), ("v_stride_t", c_i64),
        ("kv_offsets", c_vp), ("positions", c_vp),
        ("mask", c_vp), ("mask_dtype", c_i64), ("mask_stride_b", c_i64),
        ("mask_stride_s", c_i64), ("mask_stride_t", c_i64),
        ("out", c_vp), ("o_stride_b", c_i64), ("o_stride_s", c_i64), ("o_stride_h", c_i64),
        ("new_key", c_vp), ("new_value", c_vp),
        ("nk_stride_b", c_i64), ("nk_stride_h", c_i64), ("nv_stride_b", c_i64), ("nv_stride_h", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("cs_stride_b", c_i64),
        ("workspace", c_vp), ("workspace_bytes", c_i64), ("max_chunks", c_i64),
        ("q_norm_weight", c_vp), ("k_norm_weight", c_vp), ("norm_eps", ctypes.c_float),
        ("nk_stride_s", c_i64), ("nv_stride_s", c_i64), ("cs_stride_s", c_i64),
        ("splits", c_i64),
        ("grid", c_i64),
        ("plan", c_vp),
    ]


class PrefillArgs(ctypes.Structure):
    """Mirror of ``q3t_prefill_args``."""
    _fields_ = [
        ("batch", c_i64), ("total_tokens", c_i64), ("max_seqlen", c_i64), ("q_heads", c_i64),
        ("kv_heads", c_i64), ("head_dim", c_i64), ("scale", ctypes.c_float),
        ("cu_seqlens", c_vp), ("query", c_vp), ("q_stride_t", c_i64), ("q_stride_h", c_i64),
        ("keys", c_vp), ("values", c_vp),
        ("k_stride_b", c_i64), ("k_stride_h", c_i64), ("k_stride_t", c_i64),
        ("v_stride_b", c_i64), ("v_stride_h", c_i64), ("v_stride_t", c_i64),
        ("kv_slots", c_vp), ("out", c_vp), ("o_stride_t", c_i64), ("o_stride_h", c_i64),
        ("capacity", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("cs_stride_t", c_i64),
        ("kv_lens", c_vp), ("mask", c_vp), ("mask_dtype", c_i64), ("mask_stride_b", c_i64),
        ("mask_stride_q", c_i64), ("new_values", c_vp), ("nv_stride_t", c_i64), ("nv_stride_h", c_i64),
    ]


class PrefillRopeWriteArgs(ctypes.Structure):
    """Mirror of ``q3t_prefill_rope_write_args``."""
    _fields_ = [
        ("batch", c_i64), ("total_tokens", c_i64), ("q_heads", c_i64), ("kv_heads", c_i64),
        ("head_dim", c_i64), ("capacity", c_i64), ("cu_seqlens", c_vp),
        ("query", c_vp), ("q_stride_t", c_i64), ("q_stride_h", c_i64),
        ("key", c_vp), ("k_stride_t", c_i64), ("k_stride_h", c_i64),
        ("value", c_vp), ("v_stride_t", c_i64), ("v_stride_h", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("cs_stride_t", c_i64),
        ("q_out", c_vp), ("qo_stride_t", c_i64), ("qo_stride_h", c_i64),
        ("arena_keys", c_vp), ("arena_values", c_vp),
        ("a_stride_b", c_i64), ("a_stride_h", c_i64), ("a_stride_t", c_i64),
        ("kv_slots", c_vp),
    ]


# Every exported entry point with its ctypes signature.
SIGNATURES = {
    "q3t_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "q3t_abi_version": (ctypes.c_int, []),
    "q3t_kv_write": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64,
                                    c_i64, I64x3, I64x3, I64x3, c_i64, c_vp]),
    "q3t_copy_strided": (ctypes.c_int, [c_vp, c_vp, c_i64, ctypes.c_int, ctypes.POINTER(c_i64),
                                        ctypes.POINTER(c_i64), ctypes.POINTER(c_i64), c_vp]),
    "q3t_copy_bytes": (ctypes.c_int, [c_vp, c_vp, c_i64, c_vp]),
    "q3t_rotary": (ctypes.c_int, [c_vp, c_vp, c_vp, c_vp, c_i64, c_i64, c_i64, c_i64, c_vp]),
    "q3t_rope_tables": (ctypes.c_int, [c_vp, c_i64, c_vp, c_i64, ctypes.c_float, c_i64, c_vp,
                                       c_vp, c_vp]),
    "q3t_decode_workspace_bytes": (c_i64, [ctypes.POINTER(DecodeArgs)]),
    "q3t_decode_grid": (ctypes.c_int, [ctypes.POINTER(DecodeArgs)]),
    "q3t_decode_attention": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "q3t_decode_reset_workspace": (ctypes.c_int, [c_vp, c_i64, c_vp]),
    "q3t_decode_plan": (ctypes.c_int, [c_vp, c_i64, c_i64, c_i64, c_i64, c_vp, c_vp]),
    "q3t_decode_plan_bytes": (ctypes.c_int64, [c_i64, c_i64, c_i64]),
    "q3t_decode_attention_static": (ctypes.c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "q3t_prefill_attention": (ctypes.c_int, [ctypes.POINTER(PrefillArgs), c_vp]),
    "q3t_prefill_rope_write": (ctypes.c_int, [ctypes.POINTER(PrefillRopeWriteArgs), c_vp]),
}

_lock = threading.Lock()
_lib = None


class KernelError(RuntimeError):
    """A HIP launch failed after host validation passed."""


ABI_VERSION = 8  # q3t_abi_version() of the header these structures mirror


def library() -> ctypes.CDLL:
    """Load the HIP library once; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIBRARY_PATH.exists():
                raise RuntimeError(
                    f"{LIBRARY_PATH.name} is not built; run __graft_entry__.build() first")
            lib = ctypes.CDLL(str(LIBRARY_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = restype
                fn.argtypes = argtypes
            if lib.q3t_abi_version() != ABI_VERSION:
                raise RuntimeError(f"{LIBRARY_PATH.name} implements ABI {lib.q3t_abi_version()}, "
                                   f"these bindings ABI {ABI_VERSION}; rebuild it")
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    """Map a status code to the reference's exception convention."""
    if status == Q3T_OK:
        return
    text = library().q3t_status_string(status).decode()
    if status < 0:
        raise ValueError(f"{what}: {text}")
    raise KernelError(f"{what}: HIP launch failed: {text}")


def stream_handle(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


_HIP = None


def capture_id(stream: int) -> int:
    """Id of the graph capture ``stream`` is recording into (hipStreamGetCaptureInfo), 0 when
    it is not capturing."""
    global _HIP
    if _HIP is None:
        hip = ctypes.CDLL('libamdhip64.so')  # the HIP runtime torch has loaded
        hip.hipStreamGetCaptureInfo.argtypes = [ctypes.c_void_p, ctypes.POINTER(ctypes.c_int),
                                                ctypes.POINTER(ctypes.c_ulonglong)]
        hip.hipStreamGetCaptureInfo.restype = ctypes.c_int
        _HIP = hip
    status, cid = ctypes.c_int(0), ctypes.c_ulonglong(0)
    err = _HIP.hipStreamGetCaptureInfo(ctypes.c_void_p(stream), ctypes.byref(status), ctypes.byref(cid))
    if err != 0:
        raise KernelError(f'hipStreamGetCaptureInfo failed: error {err}')
    return int(cid.value) if status.value == 1 else 0  # hipStreamCaptureStatusActive


def require_gpu(*tensors: torch.Tensor) -> torch.device:
    """All tensors on one ROCm device; the HIP kernels are the only implementation."""
    device = tensors[0].device
    if device.type != "cuda":
        raise ValueError("expected tensors on a ROCm GPU device")
    for t in tensors:
        if t.device != device:
            raise ValueError("tensors must share one device")
    return device


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def i64x3(values) -> ctypes.Array:
    return I64x3(*[int(v) for v in values])
