"""ctypes binding of libflywheel_hip.so (the C-ABI declared in
include/flywheel_hip.h).

The library is the only compute path: there is no CPU fallback.  Loading fails
with a RuntimeError naming the missing file; a call without a HIP device fails
with a RuntimeError before anything is launched.
"""

import ctypes
import os
import threading

import torch

_LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "lib", "libflywheel_hip.so")
_lock = threading.Lock()
_lib = None

FW_OK, FW_ERR_VALUE, FW_ERR_NOT_IMPLEMENTED, FW_ERR_RUNTIME = 0, 1, 2, 3
FW_BF16, FW_FP8_E4M3, FW_FP8_E5M2 = 0, 1, 2
FW_KV_DENSE, FW_KV_VARLEN, FW_KV_PAGED = 0, 1, 2
FW_DECODE_SCRATCH_BYTES = 64 << 20  # include/flywheel_hip.h

_c_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float


class DecodeParams(ctypes.Structure):
    _fields_ = [
        ("q", _c_p), ("kv_cache", _c_p), ("k_new", _c_p), ("v_new", _c_p),
        ("cache_seqlens", _c_p), ("block_table", _c_p), ("num_active", _c_p),
        ("sinks", _c_p), ("out", _c_p), ("lse", _c_p), ("workspace", _c_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("batch", _i32), ("seqlen_q", _i32), ("nheads", _i32), ("nheads_k", _i32),
        ("head_dim", _i32), ("page_size", _i32), ("num_pages", _i32), ("max_pages", _i32),
        ("kv_dtype", _i32), ("seqlen_add", _i32),
        ("softmax_scale", _f32), ("softcap", _f32),
        ("causal", _i32), ("window_left", _i32),
        ("k_descale", _f32), ("v_descale", _f32),
        ("num_splits", _i32),
        ("v_cache", _c_p),
        ("k_descale_ptr", _c_p), ("v_descale_ptr", _c_p),
    ]


class PrefillParams(ctypes.Structure):
    _fields_ = [
        ("kv_mode", _i32),
        ("q", _c_p), ("out", _c_p), ("lse", _c_p), ("k", _c_p), ("v", _c_p),
        ("cu_seqlens_q", _c_p), ("cu_seqlens_k", _c_p), ("seqused_k", _c_p),
        ("block_table", _c_p), ("num_active", _c_p), ("sinks", _c_p),
        ("workspace", _c_p), ("workspace_bytes", ctypes.c_size_t),
        ("q_stride_b", _i64), ("q_stride_h", _i64), ("q_stride_t", _i64),
        ("o_stride_b", _i64), ("o_stride_h", _i64), ("o_stride_t", _i64),
        ("k_stride_b", _i64), ("k_stride_h", _i64), ("k_stride_t", _i64),
        ("v_stride_b", _i64), ("v_stride_h", _i64), ("v_stride_t", _i64),
        ("lse_stride_b", _i64), ("lse_stride_h", _i64),
        ("batch", _i32), ("nheads", _i32), ("nheads_k", _i32), ("head_dim", _i32),
        ("seqlen_q", _i32), ("seqlen_k", _i32), ("max_seqlen_q", _i32),
        ("page_size", _i32), ("num_pages", _i32), ("max_pages", _i32),
        ("kv_dtype", _i32),
        ("softmax_scale", _f32), ("softcap", _f32),
        ("causal", _i32), ("window_left", _i32), ("window_right", _i32),
        ("k_descale", _f32), ("v_descale", _f32),
        ("rotary_cos", _c_p), ("rotary_sin", _c_p),
        ("rotary_rows", _i32), ("rotary_f32", _i32), ("rotary_interleaved", _i32),
        ("seqused_k_excludes_q", _i32),
        ("k_descale_ptr", _c_p), ("v_descale_ptr", _c_p),
        ("head_dim_v", _i32),
        ("k_new", _c_p), ("v_new", _c_p),
    ]


class AttnBwdParams(ctypes.Structure):
    _fields_ = [
        ("q", _c_p), ("k", _c_p), ("v", _c_p), ("out", _c_p), ("dout", _c_p), ("lse", _c_p),
        ("dq", _c_p), ("dk", _c_p), ("dv", _c_p),
        ("workspace", _c_p), ("workspace_bytes", ctypes.c_size_t),
        ("q_stride_b", _i64), ("q_stride_h", _i64), ("q_stride_t", _i64),
        ("k_stride_b", _i64), ("k_stride_h", _i64), ("k_stride_t", _i64),
        ("v_stride_b", _i64), ("v_stride_h", _i64), ("v_stride_t", _i64),
        ("lse_stride_b", _i64), ("lse_stride_h", _i64),
        ("batch", _i32), ("nheads", _i32), ("nheads_k", _i32), ("head_dim", _i32),
        ("seqlen_q", _i32), ("seqlen_k", _i32),
        ("softmax_scale", _f32), ("causal", _i32),
        ("head_dim_v", _i32),
        ("o_stride_b", _i64), ("o_stride_h", _i64), ("o_stride_t", _i64),
    ]


class RotaryParams(ctypes.Structure):
    _fields_ = [
        ("x", _c_p), ("y", _c_p), ("cos_table", _c_p), ("sin_table", _c_p),
        ("cu_seqlens", _c_p), ("kv_cu", _c_p), ("kv_lens", _c_p), ("num_active", _c_p),
        ("x_stride_b", _i64), ("x_stride_h", _i64), ("x_stride_t", _i64),
        ("y_stride_b", _i64), ("y_stride_h", _i64), ("y_stride_t", _i64),
        ("batch_rows", _i32), ("nheads", _i32), ("ntokens", _i32), ("head_dim", _i32),
        ("table_rows", _i32), ("table_f32", _i32), ("interleaved", _i32),
        ("pos_offset", _i32), ("nseq", _i32),
    ]


# name -> (restype, argtypes); the full exported surface of include/flywheel_hip.h
SIGNATURES = {
    "fw_last_error": (ctypes.c_char_p, []),
    "fw_abi_version": (ctypes.c_int, []),
    "fw_paged_decode_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(DecodeParams)]),
    "fw_paged_decode": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _c_p]),
    "fw_paged_decode_noalloc": (ctypes.c_int, [ctypes.POINTER(DecodeParams), _c_p]),
    "fw_append_ragged": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _c_p, _c_p, _c_p,
                                        _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _c_p]),
    "fw_write_kv_cache_pages": (ctypes.c_int, [_c_p, _c_p, _c_p, _c_p, _i32, _c_p,
                                               _i32, _i32, _i32, _i32, _i32, _c_p]),
    "fw_prefill_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(PrefillParams)]),
    "fw_prefill": (ctypes.c_int, [ctypes.POINTER(PrefillParams), _c_p]),
    "fw_rotary": (ctypes.c_int, [ctypes.POINTER(RotaryParams), _c_p]),
    "fw_clock_probe": (ctypes.c_int, [_c_p, _i32, _i32, _c_p]),
    "fw_attn_bwd_workspace_bytes": (ctypes.c_size_t, [ctypes.POINTER(AttnBwdParams)]),
    "fw_attn_bwd": (ctypes.c_int, [ctypes.POINTER(AttnBwdParams), _c_p]),
}


def library_path():
    return _LIB_PATH


def lib():
    """The loaded library; RuntimeError if it was never built."""
    global _lib
    if _lib is None:
        with _lock:
            if _lib is None:
                if not os.path.exists(_LIB_PATH):
                    raise RuntimeError(
                        f"libflywheel_hip.so is not built ({_LIB_PATH}); run"
                        " `python flywheel-tpu_amd/build.py` (or __graft_entry__.build())."
                    )
                handle = ctypes.CDLL(_LIB_PATH)
                for name, (res, args) in SIGNATURES.items():
                    fn = getattr(handle, name)
                    fn.restype = res
                    fn.argtypes = args
                _lib = handle
    return _lib


def check(status):
    if status == FW_OK:
        return
    msg = lib().fw_last_error().decode()
    if status == FW_ERR_VALUE:
        raise ValueError(msg)
    if status == FW_ERR_NOT_IMPLEMENTED:
        raise NotImplementedError(msg)
    raise RuntimeError(msg)


def require_device(*tensors):
    """RuntimeError unless every tensor lives on a HIP device."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "flywheel_tpu runs on an AMD GPU (HIP) only; got a tensor on"
                f" {t.device}. There is no CPU fallback."
            )


def stream_of(tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


KV_DTYPES = {
    torch.bfloat16: FW_BF16,
    torch.float8_e4m3fn: FW_FP8_E4M3,
    torch.float8_e5m2: FW_FP8_E5M2,
}
