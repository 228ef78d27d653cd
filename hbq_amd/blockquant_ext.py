"""HIP-backed drop-in for the reference's `blockquant_ext` module.

The five ops keep the pybind signatures of blockquant_ext_src/blockquant_ext.cpp:51-72
and the checks and messages of blockquant_ext.cpp:12-19 and gemm.cu:558-566,
618-621, 1040-1054, 1399-1411 (all raise RuntimeError).  A is [M, K] and B is
[K, N], both fp16 on one GPU; C is a new [M, N] fp16 tensor.  Kernels run on
torch's current stream.

Additions beyond the reference (same arithmetic, other operand layout):
the *_nk variants take the weight as W[N, K] (nn.Linear layout), which avoids
the caller's W.t().contiguous() copy, and group_partials() exposes the fp32
per-K-group partial sums for checking the fused epilogues.
"""
import torch

from . import _lib


def _check_inputs(A, B, b_is_nk=False):
    if not isinstance(A, torch.Tensor) or not isinstance(B, torch.Tensor):
        raise TypeError("A and B must be tensors")
    if A.dtype != torch.float16:
        raise RuntimeError("A must be fp16")
    if B.dtype != torch.float16:
        raise RuntimeError("B must be fp16")
    if A.dim() != 2 or B.dim() != 2:
        raise RuntimeError("A and B must be 2D")
    if not (A.is_cuda and B.is_cuda):
        raise RuntimeError("A and B must be CUDA tensors")
    if A.device != B.device:
        raise RuntimeError("A and B must be on the same CUDA device")
    kb = B.size(1) if b_is_nk else B.size(0)
    if A.size(1) != kb:
        raise RuntimeError("A's K dimension must match B's K dimension")


# B[K, N] operands of at least this many multiply-adds are transposed to W[N, K]
# first: the 256x256-tile kernel reads W[N, K] (K contiguous), and the copy costs
# a few percent of such a GEMM.  Both layouts give bit-identical results (the
# same MFMA sequence per output element).
TRANSPOSE_MIN_MNK = 1 << 30


def _prep(A, B, b_is_nk, group_k=64):
    _check_inputs(A, B, b_is_nk)
    A = A.contiguous()
    M, K = A.shape
    N = B.size(0) if b_is_nk else B.size(1)
    if not b_is_nk and M * N * K >= TRANSPOSE_MIN_MNK and K % 64 == 0 and N % 8 == 0 and group_k >= 64:
        B = B.contiguous()
        W = torch.empty((N, K), dtype=B.dtype, device=B.device)
        _call(_lib.lib().hbq_transpose16, _lib.ptr(B), _lib.ptr(W), K, N, _lib.stream_of(B))
        B, b_is_nk = W, True
    else:
        B = B.contiguous()
    C = torch.empty((M, N), dtype=torch.float16, device=A.device)
    return A, B, C, M, N, K, b_is_nk


def _call(fn, *args):
    _lib.check(fn(*args))


def gemm_fp32_accum(A, B, b_is_nk=False):
    """fp32 accumulation over all of K, one rounding to fp16 (gemm.cu:593-616)."""
    A, B, C, M, N, K, b_is_nk = _prep(A, B, b_is_nk)
    _call(_lib.lib().hbq_gemm_fp32_accum, _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), M, N, K, int(b_is_nk),
          _lib.stream_of(A))
    return C


def gemm_fp16_accum(A, B, b_is_nk=False):
    """fp16 fused multiply-add chain over ascending k (gemm.cu:568-591)."""
    A, B, C, M, N, K, b_is_nk = _prep(A, B, b_is_nk, group_k=0)
    _call(_lib.lib().hbq_gemm_fp16_accum, _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), M, N, K, int(b_is_nk),
          _lib.stream_of(A))
    return C


def gemm_fp16_grouped_accum(A, B, group_k, b_is_nk=False):
    """fp32 within each group_k-wide K group, fp16 accumulation across groups (gemm.cu:618-667)."""
    A, B, C, M, N, K, b_is_nk = _prep(A, B, b_is_nk, group_k)
    _call(_lib.lib().hbq_gemm_fp16_grouped_accum, _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), M, N, K, int(group_k),
          int(b_is_nk), _lib.stream_of(A))
    return C


def gemm_blockquant_mxfp8(A, B, group_k, group_n, b_is_nk=False):
    """Per-K-group partials quantized to E3M4 per (row, group_n columns), fp16 accumulation (gemm.cu:1040-1135)."""
    A, B, C, M, N, K, b_is_nk = _prep(A, B, b_is_nk, group_k)
    _call(_lib.lib().hbq_gemm_blockquant_mxfp8, _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), M, N, K, int(group_k),
          int(group_n), int(b_is_nk), _lib.stream_of(A))
    return C


def gemm_blockquant_mxint8(A, B, group_k, group_n, b_is_nk=False):
    """Per-K-group partials quantized to INT8 with a power-of-two scale per (row, group_n columns),
    fp16 accumulation across groups (gemm.cu:1399-1478)."""
    A, B, C, M, N, K, b_is_nk = _prep(A, B, b_is_nk, group_k)
    _call(_lib.lib().hbq_gemm_blockquant_mxint8, _lib.ptr(A), _lib.ptr(B), _lib.ptr(C), M, N, K, int(group_k),
          int(group_n), int(b_is_nk), _lib.stream_of(A))
    return C


def gemm_fp32_accum_nk(A, W):
    return gemm_fp32_accum(A, W, b_is_nk=True)


_WORKSPACE = {}


def gemm_fp32_accum_nk_split(A, W):
    """gemm_fp32_accum_nk that may split K: for long K on grids of at most one round of
    tiles it sums two K halves' fp32 partials (each the kernel's own group partial for
    group_k = K / 2) before the fp16 rounding.  The split-K workspace is cached per device
    and stream (calls on one stream run in order, so they can share it).  Same
    fp32-accumulation contract, another summation order."""
    A, W, C, M, N, K, _ = _prep(A, W, True)
    need = _lib.lib().hbq_gemm_fp32_accum_workspace(M, N, K, 1)
    ws = None
    if need > 0:
        key = (A.device, torch.cuda.current_stream(A.device).cuda_stream)
        ws = _WORKSPACE.get(key)
        if ws is None or ws.numel() * 4 < need:
            ws = _WORKSPACE[key] = torch.empty((need + 3) // 4, dtype=torch.float32, device=A.device)
    _call(_lib.lib().hbq_gemm_fp32_accum_ws, _lib.ptr(A), _lib.ptr(W), _lib.ptr(C), _lib.ptr(ws),
          ws.numel() * 4 if ws is not None else 0, M, N, K, 1, _lib.stream_of(A))
    return C


def gemm_fp16_accum_nk(A, W):
    return gemm_fp16_accum(A, W, b_is_nk=True)


def gemm_fp16_grouped_accum_nk(A, W, group_k):
    return gemm_fp16_grouped_accum(A, W, group_k, b_is_nk=True)


def gemm_blockquant_mxfp8_nk(A, W, group_k, group_n):
    return gemm_blockquant_mxfp8(A, W, group_k, group_n, b_is_nk=True)


def gemm_blockquant_mxint8_nk(A, W, group_k, group_n):
    return gemm_blockquant_mxint8(A, W, group_k, group_n, b_is_nk=True)


def group_partials(A, B, group_k, b_is_nk=False):
    """fp32 partial sums of every group_k-wide K group, [ceil(K/group_k), M, N], computed by the
    same MFMA accumulation as the GEMM kernels."""
    _check_inputs(A, B, b_is_nk)
    A = A.contiguous()
    B = B.contiguous()
    M, K = A.shape
    N = B.size(0) if b_is_nk else B.size(1)
    G = -(-K // group_k)
    P = torch.empty((G, M, N), dtype=torch.float32, device=A.device)
    _call(_lib.lib().hbq_gemm_group_partials, _lib.ptr(A), _lib.ptr(B), _lib.ptr(P), M, N, K, int(group_k),
          int(b_is_nk), _lib.stream_of(A))
    return P
