"""Packed HBQ tensors and linears whose weights stay packed in HBM.

The reference keeps fake-quantized fp16 weights (src/ptq.py:338-358); the HBQ
hardware emits the same quantization as bit fields: E2Mm element codes, an E5M3
L1 scale byte per block, L2 indices and a scheme bit
(hardware/HBQ_accelerator/hbq_e_quantizer/top.sv:14-45).  `pack` stores a
tensor in that form (0.54 B per element for HBQ-A weights instead of 2), and
`unpack` decodes it on the GPU to exactly the fake-quantized values, so a GEMM on
the decoded weight gives the same bits as one on the fake-quantized weight.

`pack_linear_weights` quantizes a model's linear weights into packed form and
frees the fp16 copies; each forward decodes the weight into a scratch buffer shared
by all layers of that shape, right before its GEMM (`_QBaseLinear.forward_quantized`).
"""
from dataclasses import dataclass
from typing import Optional, Tuple

import torch

from . import _lib
from .quantizer import HBQQuantizer

_SCHEMES = HBQQuantizer.L2_SCHEME


def packed_strides(cols, block_size, mbit, l2_block_size, l2_sc_bit, l2_scheme):
    """Row strides in bytes of the four packed strings (codes, l1, l2, scheme; 0 if absent)."""
    import ctypes
    out = (ctypes.c_int64 * 4)()
    _lib.check(_lib.lib().hbq_hbq_packed_strides(cols, block_size, mbit, l2_block_size, l2_sc_bit,
                                                 _SCHEMES.index(l2_scheme), ctypes.addressof(out)), ValueError)
    return tuple(out)


@dataclass
class PackedHBQ:
    """An HBQ-quantized tensor as bit fields (rows = all leading dims, blocks along the last)."""
    codes: torch.Tensor                 # uint8 [rows, cols * (mbit + 3) / 8]
    l1: torch.Tensor                    # uint8 [rows, cols / block_size], E5M3 bytes
    l2: Optional[torch.Tensor]          # uint8 [rows, ceil(nsub * l2_sc_bit / 8)] or None
    scheme: Optional[torch.Tensor]      # uint8 [rows, ceil(nblk / 8)] (Mix) or None
    shape: Tuple[int, ...]
    dtype: torch.dtype
    block_size: int
    mbit: int
    l2_block_size: int
    l2_sc_bit: int
    l2_scheme: str

    @property
    def nbytes(self) -> int:
        return sum(t.numel() for t in (self.codes, self.l1, self.l2, self.scheme) if t is not None)

    def unpack(self, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        return unpack(self, out)


def pack(quantizer: HBQQuantizer, x: torch.Tensor) -> PackedHBQ:
    """Quantize x with an HBQQuantizer (as quantizer.q(x) does) and pack the result.
    The last dimension must be a multiple of the block size (and of 8)."""
    if not isinstance(quantizer, HBQQuantizer):
        raise TypeError("pack needs an HBQQuantizer")
    _lib.require_gpu(x, "pack")
    cols = x.shape[-1]
    rows = x.numel() // cols if cols else 0
    st = packed_strides(cols, quantizer.block_size, quantizer.mbit, quantizer.l2_block_size, quantizer.l2_sc_bit,
                        quantizer.l2_scheme)
    qo = quantizer.quantize(x)
    dev = x.device
    pc = torch.empty((rows, st[0]), dtype=torch.uint8, device=dev)
    pl1 = torch.empty((rows, st[1]), dtype=torch.uint8, device=dev)
    pl2 = torch.empty((rows, st[2]), dtype=torch.uint8, device=dev) if st[2] else None
    ps = torch.empty((rows, st[3]), dtype=torch.uint8, device=dev) if st[3] else None
    if rows:
        _lib.check(_lib.lib().hbq_hbq_pack(
            _lib.ptr(qo.codes), _lib.ptr(qo.scales), _lib.ptr(qo.l2_index), _lib.ptr(qo.scheme), _lib.ptr(pc),
            _lib.ptr(pl1), _lib.ptr(pl2), _lib.ptr(ps), rows, cols, _lib.DTYPE_CODE[x.dtype], quantizer.block_size,
            quantizer.mbit, quantizer.l2_block_size, quantizer.l2_sc_bit, _SCHEMES.index(quantizer.l2_scheme),
            _lib.stream_of(x)), ValueError)
    return PackedHBQ(pc, pl1, pl2, ps, tuple(x.shape), x.dtype, quantizer.block_size, quantizer.mbit,
                     quantizer.l2_block_size, quantizer.l2_sc_bit, quantizer.l2_scheme)


def unpack(p: PackedHBQ, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Decode a packed tensor to its fake-quantized values (the quantizer's q(x), bit for bit)."""
    cols = p.shape[-1]
    rows = p.codes.shape[0]
    if out is None:
        out = torch.empty(p.shape, dtype=p.dtype, device=p.codes.device)
    elif out.shape != torch.Size(p.shape) or out.dtype != p.dtype or not out.is_contiguous():
        raise ValueError("out must be a contiguous tensor of the packed shape and dtype")
    if rows and cols:
        _lib.check(_lib.lib().hbq_hbq_unpack(
            _lib.ptr(p.codes), _lib.ptr(p.l1), _lib.ptr(p.l2), _lib.ptr(p.scheme), _lib.ptr(out), rows, cols,
            _lib.DTYPE_CODE[p.dtype], p.block_size, p.mbit, p.l2_block_size, p.l2_sc_bit,
            _SCHEMES.index(p.l2_scheme), _lib.stream_of(out)), ValueError)
    return out


# ---- GEMM on a packed weight -------------------------------------------------------------------

ACC_MODES = {"fp32": 0, "grouped": 1, "mxint8": 2, "mxfp8": 3}


def packed_gemm_supported(p: PackedHBQ, rows: int) -> bool:
    """True when hbq_gemm_packed_w takes this weight and row count (E2M1 fp16 weights in blocks
    of 128, l2 blocks of 8..32 with at most 4 L2 factors below 4, N % 32 == 0, K % 256 == 0, 1..32 rows)."""
    N, K = p.shape[0], p.shape[-1]
    return (len(p.shape) == 2 and p.dtype == torch.float16 and p.mbit == 1 and p.block_size == 128
            and p.l2_block_size in (8, 16, 32) and p.l2_sc_bit <= 2 and p.l2_scheme not in ("PoT", "INT")
            and 1 <= rows <= 32 and N % 32 == 0 and K % 256 == 0)


def packed_gemm(x2d: torch.Tensor, p: PackedHBQ, mode: str = "fp32", group_k: int = 0, group_n: int = 0):
    """C[M, N] fp16 = x2d[M, K] fp16 @ unpack(p)^T with the accumulation of `mode` (the
    blockquant_ext op of that name), decoding the codes in registers ahead of MFMA: the same bits
    as the GEMM on the unpacked weight.  For decode-sized M (1..32 rows)."""
    _lib.require_gpu(x2d, "packed_gemm")
    if x2d.dtype != torch.float16 or x2d.dim() != 2 or x2d.shape[1] != p.shape[-1]:
        raise RuntimeError("x2d must be a 2-D fp16 tensor with the weight's K")
    x2d = x2d.contiguous()
    M, K = x2d.shape
    N = p.shape[0]
    C = torch.empty((M, N), dtype=torch.float16, device=x2d.device)
    _lib.check(_lib.lib().hbq_gemm_packed_w(
        _lib.ptr(x2d), _lib.ptr(p.codes), _lib.ptr(p.l1), _lib.ptr(p.l2), _lib.ptr(p.scheme), _lib.ptr(C), M, N, K,
        p.block_size, p.mbit, p.l2_block_size, p.l2_sc_bit, _SCHEMES.index(p.l2_scheme), ACC_MODES[mode], group_k,
        group_n, _lib.stream_of(x2d)))
    return C


def linear_packed(xq: torch.Tensor, p: PackedHBQ, ops, bias=None):
    """ops(xq, unpack(p), bias) for the HIP accumulation operators, on the packed weight directly when
    the row count is decode-sized; None when the caller should decode the weight and call ops."""
    from .ops import FP16AccumMatMul, FP32AccumMatMul
    rows = xq.numel() // xq.shape[-1] if xq.shape[-1] else 0
    if not packed_gemm_supported(p, rows) or not xq.is_cuda:
        return None
    if isinstance(ops, FP32AccumMatMul):
        mode, gk, gn = "fp32", 0, 0
    elif isinstance(ops, FP16AccumMatMul) and ops.quant_block_size is not None:
        if ops.group_size not in (64, 128) or ops.quant_block_size not in (4, 8, 16, 32):
            return None     # ops raises the reference's ValueError, or the kernel does not take the group
        mode, gk, gn = "mxint8", ops.group_size, ops.quant_block_size
    elif isinstance(ops, FP16AccumMatMul) and ops.group_size in (16, 32, 64, 128):
        mode, gk, gn = "grouped", ops.group_size, 0
    else:
        return None
    x2d = xq.reshape(-1, xq.shape[-1])
    if x2d.dtype != torch.float16:
        x2d = x2d.half()
    y = packed_gemm(x2d, p, mode, gk, gn)
    if bias is not None:
        y = y + bias
    return y.view(*xq.shape[:-1], -1)


# ---- linears with packed weights ---------------------------------------------------------------

_SCRATCH = {}


def _scratch(shape, dtype, device):
    """One decode buffer per (shape, dtype, device, stream), reused by every layer of that
    shape: calls on one stream run in order, so a buffer is free again once the GEMM that
    read it has been issued after it; another stream gets its own buffer."""
    key = (tuple(shape), dtype, device, torch.cuda.current_stream(device).cuda_stream)
    buf = _SCRATCH.get(key)
    if buf is None:
        buf = _SCRATCH[key] = torch.empty(shape, dtype=dtype, device=device)
    return buf


def decoded_weight(p: PackedHBQ, copy: bool = False) -> torch.Tensor:
    """The fake-quantized weight of a packed linear, decoded into the shared scratch buffer
    of its shape and stream: valid until the next decode of that shape on that stream
    (copy=True returns a tensor of its own)."""
    w = unpack(p, _scratch(p.shape, p.dtype, p.codes.device))
    return w.clone() if copy else w


def decoded_stack(ps) -> torch.Tensor:
    """Packed weights with one K decoded into consecutive row ranges of one shared scratch
    [sum N, K] buffer (for one GEMM over several linears that read the same input)."""
    n = sum(p.shape[0] for p in ps)
    W = _scratch((n, ps[0].shape[1]), ps[0].dtype, ps[0].codes.device)
    off = 0
    for p in ps:
        unpack(p, W[off:off + p.shape[0]])
        off += p.shape[0]
    return W


def pack_linear_weights(model) -> int:
    """Quantize every _QBaseLinear weight with its HBQ weight quantizer into packed form
    (instead of PTQ.static_quant_wgt's in-place fake quantization, src/ptq.py:338-358: the
    weights must not be quantized yet) and free the fp16 weight; forwards decode it into a
    shared scratch buffer before the GEMM, which then sees exactly the fake-quantized weight.
    The packed strings are plain attributes: move the model before packing.  Returns the
    number of linears packed."""
    from .module import _QBaseLinear
    n = 0
    for mod in model.modules():
        if not isinstance(mod, _QBaseLinear) or not isinstance(mod.wq, HBQQuantizer):
            continue
        w = mod.weight
        if w.shape[-1] % mod.wq.block_size or not w.is_cuda:
            continue
        with torch.no_grad():
            mod.packed_weight = pack(mod.wq, w.detach())
        mod._parameters["weight"] = torch.nn.Parameter(torch.empty(0, dtype=w.dtype, device=w.device),
                                                       requires_grad=False)
        n += 1
    return n
