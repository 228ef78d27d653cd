"""ctypes front end of the CPU oracle (oracle/hbq_oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, ``__graft_entry__.smoke()`` and bench.py's
cpu_baseline leg use it as the checker.  The product package ``hbq_amd`` never
imports it.

Arrays are numpy: fp16 and bf16 tensors travel as uint16 bit patterns, fp32
as float32.  Each wrapper names the reference code it restates.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libhbq_oracle.so")

DT = {"f16": 0, "bf16": 1, "f32": 2}
SCHEMES = ["PoT", "INT", "SIG-1", "FP-1", "FP1", "FP-10", "FP-100", "Mix"]

_lib = None


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, I, I64, D = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_double
        sig = {
            "orc_elem_quant": [P, P, I64, I, I, I, I, I],
            "orc_fp_quant": [P, P, I64, I, I, I, I, I],
            "orc_floor_log2": [P, P, I64, I],
            "orc_mx_scale": [P, P, I64, I, I, I, I, I, I, I, I],
            "orc_mxfp_qdq": [P, P, P, I64, I64, I, I, I, I, I, I, I, I, I, I, D, I],
            "orc_hbq_l2_table": [I, I, I, P],
            "orc_hbq_qdq": [P, P, P, P, P, P, I64, I64, I, I, I, I, I, I, I, I, I, I, I, I],
            "orc_gemm_fp32acc": [P, P, P, I, I, I],
            "orc_gemm_fp16acc": [P, P, P, I, I, I],
            "orc_gemm_grouped": [P, P, P, I, I, I, I],
            "orc_gemm_mxint8": [P, P, P, I, I, I, I, I],
            "orc_gemm_mxfp8": [P, P, P, I, I, I, I, I],
            "orc_group_partials": [P, P, P, I, I, I, I],
            "orc_epilogue": [P, P, I, I, I, I, I],
        }
        L.orc_cascade_sum.argtypes = [P, I64, I64]
        L.orc_cascade_sum.restype = ctypes.c_float
        L.orc_row_sum.argtypes = [P, I64]
        L.orc_row_sum.restype = ctypes.c_float
        L.orc_group_partial_one.argtypes = [P, P, I, I, I, I, I, I]
        L.orc_group_partial_one.restype = ctypes.c_float
        for name, args in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = I
        _lib = L
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def _bits(x, dt):
    if dt == "f32":
        return np.ascontiguousarray(x, dtype=np.float32)
    return np.ascontiguousarray(x, dtype=np.uint16)


def _empty(shape, dt):
    return np.empty(shape, np.float32 if dt == "f32" else np.uint16)


def _check(rc, name):
    if rc != 0:
        raise RuntimeError(f"oracle {name} failed with code {rc}")


def elem_quant(x, dt, ebit, mbit, use_ceil=False, compiled=False):
    """make_fp_quant(ebit, mbit) elementwise (src/quantizer.py:187-257).

    compiled=True gives the torch.compile'd form GLOBAL_FP_QUANT_CACHE serves
    (src/quantizer.py:38-63): every step in fp32, the sum |m| + 0.5004 not
    rounded to T."""
    x = _bits(x, dt)
    y = _empty(x.shape, dt)
    _check(lib().orc_elem_quant(_p(x), _p(y), x.size, DT[dt], ebit, mbit, int(use_ceil), int(compiled)),
           "elem_quant")
    return y


def fp_quant(x, dt, ebit, mbit, allow_subnormal=True, use_ceil=False):
    """fp_quant (src/quantizer.py:259-328)."""
    x = _bits(x, dt)
    y = _empty(x.shape, dt)
    _check(lib().orc_fp_quant(_p(x), _p(y), x.size, DT[dt], ebit, mbit, int(allow_subnormal), int(use_ceil)),
           "fp_quant")
    return y


def floor_log2(x, dt):
    """floor(R_T(log2 |x|)) as used at src/quantizer.py:217,291,493-499."""
    x = _bits(x, dt)
    y = np.empty(x.shape, np.float32)
    _check(lib().orc_floor_log2(_p(x), _p(y), x.size, DT[dt]), "floor_log2")
    return y


def mx_scale(amax, dt, ebit, mbit, sc_ebit, sc_mbit, allow_subnormal=False, use_round=False, use_ceil=False):
    """MXFPQuantizer.get_shared_scale given the block amax (src/quantizer.py:481-511)."""
    a = _bits(amax, dt)
    y = _empty(a.shape, dt)
    _check(lib().orc_mx_scale(_p(a), _p(y), a.size, DT[dt], ebit, mbit, sc_ebit, sc_mbit, int(allow_subnormal),
                              int(use_round), int(use_ceil)), "mx_scale")
    return y


def mxfp_qdq(x, dt, block_size, ebit, mbit, sc_ebit, sc_mbit, scale_allow_subnormal=False, use_round=False,
             use_ceil=False, tensor_scale=None, compiled=False):
    """MXFPQuantizer.q (src/quantizer.py:513-539) on a 2-D array; blocks along the last dim.

    compiled selects the element rule of activate_dynamo=True.  Returns
    (dequantized, per-block scales)."""
    x = _bits(x, dt)
    rows, cols = x.shape
    nblk = -(-cols // block_size)
    y = _empty(x.shape, dt)
    s = _empty((rows, nblk), dt)
    per = tensor_scale is not None
    _check(lib().orc_mxfp_qdq(_p(x), _p(y), _p(s), rows, cols, DT[dt], block_size, ebit, mbit, sc_ebit, sc_mbit,
                              int(scale_allow_subnormal), int(use_round), int(use_ceil), int(per),
                              float(tensor_scale) if per else 1.0, int(compiled)), "mxfp_qdq")
    return y, s


def l2_table(scheme, l2_sc_bit, dt):
    tab = np.zeros(64, np.float32)
    S = lib().orc_hbq_l2_table(SCHEMES.index(scheme), l2_sc_bit, DT[dt], _p(tab))
    _check(0 if S > 0 else S, "l2_table")
    return tab[: (1 << l2_sc_bit) * S].reshape(1 << l2_sc_bit, S)


def hbq_qdq(x, dt, block_size=128, ebit=2, mbit=3, sc_ebit=5, sc_mbit=3, l2_block_size=4, l2_sc_bit=1,
            l2_scheme="PoT", scale_allow_subnormal=False, use_ceil=False, use_quant_kernel=True):
    """HBQQuantizer.q (src/quantizer.py:741-859) on a 2-D array.

    use_quant_kernel selects the element rule as the reference's flag does, with
    the same default: True is the torch.compile'd lpfp_quant
    (src/quantizer.py:468-469,724), False the eager one.
    Returns dict(y, l1, l2idx, scheme, l2val) mirroring the keep_l2_scale
    attributes shared_scale, l2_scale, blk_l2_scheme, real_l2_scale."""
    x = _bits(x, dt)
    rows, cols = x.shape
    nblk = -(-cols // block_size)
    nsub = block_size // l2_block_size
    y = _empty(x.shape, dt)
    l1 = _empty((rows, nblk), dt)
    l2i = np.empty((rows, nblk, nsub), np.uint8)
    sch = np.empty((rows, nblk), np.uint8)
    l2v = _empty((rows, nblk, nsub), dt)
    _check(lib().orc_hbq_qdq(_p(x), _p(y), _p(l1), _p(l2i), _p(sch), _p(l2v), rows, cols, DT[dt], block_size, ebit,
                             mbit, sc_ebit, sc_mbit, l2_block_size, l2_sc_bit, SCHEMES.index(l2_scheme),
                             int(scale_allow_subnormal), int(use_ceil), int(use_quant_kernel)), "hbq_qdq")
    return {"y": y, "l1": l1, "l2idx": l2i, "scheme": sch, "l2val": l2v}


def cascade_sum(v):
    """torch's fp32 order for a Half sum over one strided column (sub-block errors)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return float(lib().orc_cascade_sum(_p(v), v.size, 1))


def row_sum(v):
    """torch's fp32 order for a Half sum over a contiguous row read with a stride (scheme errors)."""
    v = np.ascontiguousarray(v, dtype=np.float32)
    return float(lib().orc_row_sum(_p(v), v.size))


def _gemm_in(A, B):
    A = np.ascontiguousarray(A, dtype=np.uint16)
    B = np.ascontiguousarray(B, dtype=np.uint16)
    assert A.ndim == 2 and B.ndim == 2 and A.shape[1] == B.shape[0]
    return A, B, np.empty((A.shape[0], B.shape[1]), np.uint16)


def gemm_fp32_accum(A, B):
    """gemm_core_kernel<false> (blockquant_ext_src/gemm.cu:96-303)."""
    A, B, C = _gemm_in(A, B)
    _check(lib().orc_gemm_fp32acc(_p(A), _p(B), _p(C), A.shape[0], B.shape[1], A.shape[1]), "gemm_fp32acc")
    return C


def gemm_fp16_accum(A, B):
    """gemm_core_kernel<true> (blockquant_ext_src/gemm.cu:96-303)."""
    A, B, C = _gemm_in(A, B)
    _check(lib().orc_gemm_fp16acc(_p(A), _p(B), _p(C), A.shape[0], B.shape[1], A.shape[1]), "gemm_fp16acc")
    return C


def gemm_fp16_grouped_accum(A, B, group_k):
    """gemm_core_kernel_grouped<GK> (blockquant_ext_src/gemm.cu:305-553)."""
    A, B, C = _gemm_in(A, B)
    _check(lib().orc_gemm_grouped(_p(A), _p(B), _p(C), A.shape[0], B.shape[1], A.shape[1], group_k), "grouped")
    return C


def gemm_blockquant_mxint8(A, B, group_k, group_n):
    """gemm_blockquant_mxint8_core_kernel (blockquant_ext_src/gemm.cu:1145-1396)."""
    A, B, C = _gemm_in(A, B)
    _check(lib().orc_gemm_mxint8(_p(A), _p(B), _p(C), A.shape[0], B.shape[1], A.shape[1], group_k, group_n),
           "mxint8")
    return C


def gemm_blockquant_mxfp8(A, B, group_k, group_n):
    """gemm_blockquant_mxfp8_core_kernel (blockquant_ext_src/gemm.cu:669-1035)."""
    A, B, C = _gemm_in(A, B)
    _check(lib().orc_gemm_mxfp8(_p(A), _p(B), _p(C), A.shape[0], B.shape[1], A.shape[1], group_k, group_n),
           "mxfp8")
    return C


def group_partials(A, B, group_k):
    """fp32 group partials P[g, m, n] (sequential fmaf within each K group)."""
    A, B, _ = _gemm_in(A, B)
    M, K = A.shape
    N = B.shape[1]
    G = -(-K // group_k)
    P = np.empty((G, M, N), np.float32)
    _check(lib().orc_group_partials(_p(A), _p(B), _p(P), M, N, K, group_k), "group_partials")
    return P


def group_partial_one(A, B, m, n, k0, k1):
    """One fp32 partial, the sequential chain written per output (for checking group_partials)."""
    A, B, _ = _gemm_in(A, B)
    return float(lib().orc_group_partial_one(_p(A), _p(B), B.shape[1], A.shape[1], m, n, k0, k1))


def epilogue(P, mode, group_n=0):
    """Cross-group epilogue on given partials: mode 'grouped', 'mxint8' or 'mxfp8'."""
    P = np.ascontiguousarray(P, dtype=np.float32)
    G, M, N = P.shape
    C = np.empty((M, N), np.uint16)
    m = {"grouped": 0, "mxint8": 1, "mxfp8": 2}[mode]
    _check(lib().orc_epilogue(_p(P), _p(C), G, M, N, m, group_n), "epilogue")
    return C
