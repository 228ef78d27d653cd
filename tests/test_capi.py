"""The C-ABI library loads and exports every entry point include/hbq_amd.h declares (no GPU calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "hbq_amd.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\s*\*?\s*(hbq_\w+)\s*\(", text, flags=re.M)))


@pytest.fixture(scope="module")
def lib():
    from hbq_amd import _lib
    if not os.path.exists(_lib.LIB_PATH):
        from hbq_amd import build
        build.build(verbose=False)
    return ctypes.CDLL(_lib.LIB_PATH)


def test_header_declares_entry_points():
    syms = declared_symbols()
    for s in ("hbq_mxfp_qdq", "hbq_hbq_qdq", "hbq_elem_quant", "hbq_scale_quant", "hbq_gemm_fp32_accum",
              "hbq_gemm_fp16_accum", "hbq_gemm_fp16_grouped_accum", "hbq_gemm_blockquant_mxint8",
              "hbq_gemm_blockquant_mxfp8", "hbq_gemm_group_partials", "hbq_last_error", "hbq_abi_version"):
        assert s in syms


def test_library_exports_every_declared_symbol(lib):
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing


def test_python_signatures_cover_header():
    from hbq_amd import _lib
    assert set(declared_symbols()) <= set(_lib.SIGNATURES)


def test_abi_version_and_error_string(lib):
    lib.hbq_abi_version.restype = ctypes.c_int
    assert lib.hbq_abi_version() == 2
    lib.hbq_last_error.restype = ctypes.c_char_p
    assert lib.hbq_last_error() == b""


def test_argument_errors_without_gpu(lib):
    """Argument checks fail before any HIP call, with the reference's messages."""
    from hbq_amd import _lib
    L = _lib.lib()
    rc = L.hbq_gemm_fp16_grouped_accum(None, None, None, 4, 4, 4, 48, 0, None)
    assert rc == 1 and L.hbq_last_error() == b"group_k must be one of {16,32,64,128}"
    rc = L.hbq_gemm_blockquant_mxint8(None, None, None, 4, 4, 4, 128, 7, 0, None)
    assert rc == 1 and b"group_n must be one of {4,8,16,32}" in L.hbq_last_error()
    fake = ctypes.c_void_p(256)            # never dereferenced: the shape check fails first
    rc = L.hbq_gemm_blockquant_mxint8(fake, fake, fake, 4, 32, 100, 128, 32, 0, None)
    assert rc == 1 and L.hbq_last_error() == b"K must be divisible by group_k"
    rc = L.hbq_hbq_qdq(None, None, None, None, None, None, 1, 128, 0, 128, 2, 2, 5, 3, 8, 2, 9, 0, 0, 1, None)
    assert rc == 1
    rc = L.hbq_mxfp_qdq(ctypes.c_void_p(16), ctypes.c_void_p(16), None, None, 1, 96, 0, 48, 2, 1, 5, 0, 0, 0, 0,
                        0, 1.0, 1, None)
    assert rc == 2 and b"block_size" in L.hbq_last_error()


def test_packed_argument_errors_without_gpu(lib):
    """hbq_hbq_pack / hbq_hbq_unpack / hbq_hbq_flag_nonfinite check their arguments before any HIP call."""
    from hbq_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(256)            # never dereferenced: the checks fail first
    # cols not a multiple of the block
    rc = L.hbq_hbq_pack(fake, fake, fake, fake, fake, fake, fake, fake, 4, 100, 0, 128, 1, 8, 2, 7, None)
    assert rc == 2 and b"cols % block_size" in L.hbq_last_error()
    # mbit outside 1..3
    rc = L.hbq_hbq_unpack(fake, fake, fake, fake, fake, 4, 128, 0, 128, 5, 8, 2, 2, None)
    assert rc == 2 and b"mbit" in L.hbq_last_error()
    # Mix needs the scheme strings
    rc = L.hbq_hbq_unpack(fake, fake, fake, None, ctypes.c_void_p(1024), 4, 128, 0, 128, 1, 8, 2, 7, None)
    assert rc == 1 and b"scheme" in L.hbq_last_error()
    # l2_sc_bit > 0 needs the L2 strings
    rc = L.hbq_hbq_pack(fake, fake, None, None, fake, fake, None, None, 4, 128, 0, 128, 2, 8, 2, 2, None)
    assert rc == 1 and b"L2" in L.hbq_last_error()
    # misaligned output
    rc = L.hbq_hbq_unpack(fake, fake, fake, None, ctypes.c_void_p(1026), 4, 128, 0, 128, 2, 8, 2, 2, None)
    assert rc == 1 and b"misaligned" in L.hbq_last_error()
    # empty tensors are a no-op
    assert L.hbq_hbq_unpack(None, None, None, None, None, 0, 128, 0, 128, 2, 8, 2, 2, None) == 0
    # non-finite flag: bad stride
    rc = L.hbq_flag_nonfinite(fake, 4, 8, 4, 0, fake, None)
    assert rc == 1


def test_decoder_kernel_argument_errors_without_gpu(lib):
    """The decoder entry points (causal softmax, causal attention-weight quantizer, RMSNorm
    halves, SiLU product) check their arguments before any HIP call; empty inputs are no-ops."""
    from hbq_amd import _lib
    L = _lib.lib()
    fake = ctypes.c_void_p(256)
    # causal softmax: t outside 64..2048 powers of two, bad dtype
    assert L.hbq_causal_softmax(fake, fake, 2, 96, 1.0, 0, None) == 2
    assert L.hbq_causal_softmax(fake, fake, 2, 128, 1.0, 2, None) == 2
    assert L.hbq_causal_softmax(None, None, 0, 128, 1.0, 0, None) == 0
    # causal quantizer: t % 128, block size, fp32, the quantizer's own checks (ebit)
    args = (0, 128, 2, 2, 5, 3, 8, 2, 2, 0, 0, 1, None)
    assert L.hbq_hbq_qdq_causal(fake, 2, 192, *args) == 2
    assert L.hbq_hbq_qdq_causal(fake, 2, 256, 0, 64, *args[2:]) == 2
    assert L.hbq_hbq_qdq_causal(fake, 2, 256, 2, *args[1:]) == 2
    assert L.hbq_hbq_qdq_causal(fake, 2, 256, 0, 128, 3, *args[3:]) == 2 and b"exponent" in L.hbq_last_error()
    # RMSNorm halves and SiLU product: element counts and row lengths of 8, alignment, dtype
    assert L.hbq_rms_prep(fake, None, None, fake, 12, 0, None) == 2
    assert L.hbq_rms_prep(ctypes.c_void_p(258), None, None, fake, 16, 0, None) == 1
    assert L.hbq_rms_prep(fake, fake, None, fake, 16, 0, None) == 1          # res without sum
    assert L.hbq_rms_apply(fake, fake, fake, fake, 2, 12, 0, None) == 2
    assert L.hbq_rms_apply(None, None, None, None, 0, 16, 0, None) == 0
    assert L.hbq_silu_mul(fake, fake, fake, 16, 2, None) == 2
    assert L.hbq_silu_mul(fake, fake, fake, 20, 0, None) == 2
    assert L.hbq_silu_mul(None, None, None, 0, 1, None) == 0
    # batched GEMM with shared W groups and a C row stride: argument checks before any launch
    bx = L.hbq_gemm_fp32_accum_batched_ex
    assert bx(fake, fake, fake, 8, 256, 128, 256, 65536, 32768, 0, 128, 1024, None) == 1      # w_group 0
    assert bx(fake, fake, fake, 8, 256, 128, 256, 65536, 32768, 4, 128, 64, None) == 1       # ldc < N
    assert bx(fake, fake, fake, 8, 256, 128, 256, 65536, 32768, 4, 64, 1024, None) == 1      # outputs overlap
    assert bx(fake, fake, fake, 8, 256, 128, 256, 100, 32768, 4, 128, 1024, None) == 1       # stride_a < M K
    assert bx(fake, fake, fake, 0, 256, 128, 256, 65536, 32768, 4, 128, 1024, None) == 0     # no problems
    assert L.hbq_gemm_fp32_accum_batched(fake, fake, fake, 2, 4, 8, 64, 256, 512, 16, None) == 1   # stride_c < M N
    # quantizer fused into the RMSNorm apply / SiLU product: only E2M2, one scheme, block 128
    q = [128, 2, 2, 5, 3, 32, 2, 2, 0, 0, 1]                  # HBQ-E act (SIG-1), compiled rule

    def with_(**kw):
        names = ["block", "ebit", "mbit", "sc_ebit", "sc_mbit", "l2b", "l2bit", "scheme", "sub", "ceil", "comp"]
        return [kw.get(n, v) for n, v in zip(names, q)]
    for fn, lead in ((L.hbq_rms_apply_hbq_qdq, (fake, fake, fake, fake)), (L.hbq_silu_mul_hbq_qdq, (fake, fake, fake))):
        assert fn(*lead, 4, 256, 2, *q, None) == 2                       # fp32
        assert fn(*lead, 4, 256, 0, *with_(mbit=1), None) == 2
        assert fn(*lead, 4, 256, 0, *with_(scheme=7), None) == 2        # Mix
        assert fn(*lead, 4, 256, 0, *with_(block=64), None) == 2
        assert fn(*lead, 4, 256, 0, *with_(ebit=3), None) == 2
        assert fn(*lead, 4, 200, 0, *q, None) != 0                       # cols % 128
        assert fn(*((None,) * len(lead)), 0, 256, 0, *q, None) == 0      # empty: no-op
        assert fn(*((None,) * len(lead)), 4, 256, 0, *q, None) == 1
