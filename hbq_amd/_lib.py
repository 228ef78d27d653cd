"""Loader of libhbq_amd.so, the C-ABI library declared in include/hbq_amd.h.

There is no fallback: if the library is missing or no GPU is present, the
calls raise RuntimeError.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_lib", "libhbq_amd.so")

DTYPE_CODE = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}

_lib = None

_P, _I, _I64, _D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
SIGNATURES = {
    "hbq_last_error": ([], ctypes.c_char_p),
    "hbq_abi_version": ([], _I),
    "hbq_set_generic_only": ([_I], _I),
    "hbq_mxfp_qdq": ([_P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _D, _I, _P], _I),
    "hbq_hbq_qdq": ([_P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "hbq_elem_quant": ([_P, _P, _P, _I64, _I, _I, _I, _I, _P], _I),
    "hbq_scale_quant": ([_P, _P, _I64, _I, _I, _I, _I, _I, _I, _P], _I),
    "hbq_gemm_fp32_accum_workspace": ([_I64, _I64, _I64, _I], _I64),
    "hbq_gemm_fp32_accum_ws": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I, _P], _I),
    "hbq_gemm_fp32_accum_noalloc": ([_P, _P, _P, _I64, _I64, _I64, _I, _P], _I),
    "hbq_gemm_fp32_accum_batched": ([_P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _P], _I),
    "hbq_gemm_fp32_accum_batched_ex": ([_P, _P, _P] + [_I64] * 9 + [_P], _I),
    "hbq_gemm_fp32_accum": ([_P, _P, _P, _I64, _I64, _I64, _I, _P], _I),
    "hbq_gemm_fp16_accum": ([_P, _P, _P, _I64, _I64, _I64, _I, _P], _I),
    "hbq_gemm_fp16_grouped_accum": ([_P, _P, _P, _I64, _I64, _I64, _I, _I, _P], _I),
    "hbq_gemm_blockquant_mxint8": ([_P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P], _I),
    "hbq_gemm_blockquant_mxfp8": ([_P, _P, _P, _I64, _I64, _I64, _I, _I, _I, _P], _I),
    "hbq_gemm_group_partials": ([_P, _P, _P, _I64, _I64, _I64, _I, _I, _P], _I),
    "hbq_transpose16": ([_P, _P, _I64, _I64, _P], _I),
    "hbq_flag_nonfinite": ([_P, _I64, _I64, _I64, _I, _P, _P], _I),
    "hbq_scale_causal_mask": ([_P, _I64, _I64, ctypes.c_double, _I, _P], _I),
    "hbq_causal_softmax": ([_P, _P, _I64, _I64, ctypes.c_double, _I, _P], _I),
    "hbq_hbq_qdq_causal": ([_P, _I64, _I64, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
    "hbq_rms_prep": ([_P, _P, _P, _P, _I64, _I, _P], _I),
    "hbq_rms_apply": ([_P, _P, _P, _P, _I64, _I64, _I, _P], _I),
    "hbq_silu_mul": ([_P, _P, _P, _I64, _I, _P], _I),
    "hbq_rms_apply_hbq_qdq": ([_P, _P, _P, _P, _I64, _I64] + [_I] * 12 + [_P], _I),
    "hbq_silu_mul_hbq_qdq": ([_P, _P, _P, _I64, _I64] + [_I] * 12 + [_P], _I),
    "hbq_rope": ([_P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _I64, _I64, _I, _P], _I),
    "hbq_hbq_packed_strides": ([_I64, _I, _I, _I, _I, _I, _P], _I),
    "hbq_hbq_pack": ([_P, _P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _P], _I),
    "hbq_hbq_unpack": ([_P, _P, _P, _P, _P, _I64, _I64, _I, _I, _I, _I, _I, _I, _P], _I),
    "hbq_gemm_packed_w": ([_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P], _I),
}


def lib():
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"HBQ HIP library not found at {LIB_PATH}; build it with `python -m hbq_amd.build`")
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            if hasattr(L, name):
                fn = getattr(L, name)
                fn.argtypes = args
                fn.restype = res
        _lib = L
    return _lib


# return codes of the C-ABI (include/hbq_amd.h)
ERR_INVALID, ERR_UNSUPPORTED, ERR_HIP = 1, 2, 3


def check(rc, exc=RuntimeError):
    if rc != 0:
        msg = lib().hbq_last_error().decode(errors="replace")
        raise exc(msg or f"HBQ call failed with code {rc}")


def ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def stream_of(t):
    """HIP stream handle of torch's current stream on t's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(t, what):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{what}: expected a torch.Tensor")
    if not t.is_cuda:
        raise RuntimeError(f"{what}: the HBQ HIP path needs a GPU tensor, got device {t.device}")
