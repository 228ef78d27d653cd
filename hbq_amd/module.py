"""Quantized linear layer: the caller of the HBQ quantizers and GEMMs.

Mirrors `_QBaseLinear` (src/module.py:20-67): an nn.Linear with three
quantizer slots (`wq` weight, `aq` input activation, `yq` output) and an optional
GEMM operator `ops` (an `FP16AccumMatMul`).  The weight is quantized once, in
place, by `PTQ.static_quant_linear_weight`; `forward` quantizes the input, runs
the GEMM (torch's `F.linear` when `ops` is None, as in the reference), raises on
a non-finite result and applies `yq`.
"""
import contextlib

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _lib
from .quantizer import _QBase

# Active deferred-check scopes (see deferred_finite_checks).
_DEFERRED = []


class _FlagBuffer:
    """Device int32 flags, one per checked output, set to 1 by hbq_flag_nonfinite when
    the output holds a NaN or inf (one fused pass over the output, no host sync)."""

    CHUNK = 512

    def __init__(self):
        self.chunks = []
        self.mods = []

    def check(self, mod, y):
        i = len(self.mods)
        if i % self.CHUNK == 0:
            self.chunks.append(torch.zeros(self.CHUNK, dtype=torch.int32, device=y.device))
        flag = self.chunks[-1][i % self.CHUNK:]
        y2 = y.reshape(-1, y.shape[-1]) if y.dim() != 2 else y   # a column slice of a wider output stays a view
        if y2.stride(-1) != 1:
            y2 = y2.contiguous()
        _lib.check(_lib.lib().hbq_flag_nonfinite(_lib.ptr(y2), y2.shape[0], y2.shape[1], y2.stride(0),
                                                 _lib.DTYPE_CODE[y2.dtype], _lib.ptr(flag), _lib.stream_of(y2)))
        self.mods.append(mod)

    def bad(self):
        """The modules whose output was not finite, in call order."""
        if not self.mods:
            return []
        flags = torch.cat(self.chunks).cpu().tolist()
        return [m for m, f in zip(self.mods, flags) if f]


@contextlib.contextmanager
def deferred_finite_checks():
    """Inside this scope _QBaseLinear records each output's finiteness on the device
    instead of synchronizing per layer, and the scope raises on exit if any output was
    not finite.  The reference raises per layer (src/module.py:51-66); the error still
    reaches the caller before the forward returns, without a host sync per layer."""
    flags = _FlagBuffer()
    _DEFERRED.append(flags)
    try:
        yield
    finally:
        _DEFERRED.pop()
    bad = flags.bad()
    if bad:
        mod = bad[0]
        raise RuntimeError(
            f"Non-finite output from {type(mod).__name__}({mod.in_features} -> {mod.out_features}) "
            f"(found after the forward).\n"
            f"  activation quantizer: {type(mod.aq).__name__}\n"
            f"  weight quantizer:     {type(mod.wq).__name__}\n"
            f"  matmul:               {type(mod.ops).__name__ if mod.ops is not None else 'F.linear'}\n"
            "The quantization format cannot represent this layer's dynamic range: check the element and "
            "scale exponent bits and the block size of the quantization config.")


def same_quantizer(a, b):
    """True when two quantizers compute the same function (same class and settings), so one
    quantized copy of an input can serve both."""
    if type(a) is not type(b):
        return False
    keys = ("ebit", "mbit", "sc_ebit", "sc_mbit", "block_size", "per_tensor_scale", "scale_allow_subnormal",
            "use_round", "use_ceil", "l2_block_size", "l2_sc_bit", "l2_scheme", "_fused")
    return all(getattr(a, k, None) == getattr(b, k, None) for k in keys)


def _fusable(mods):
    """True when linears fed one quantized input can run as one GEMM over their stacked weights
    and give each output column the same bits as their own GEMMs: a HIP operator of one type and
    settings on all of them (each output column of those kernels depends only on its own weight
    row), fp16 weights with one K on one GPU, no bias, and partial-sum blocks (quant_block_size
    columns) that never straddle two linears."""
    from .ops import FP16AccumMatMul, FP32AccumMatMul
    o = mods[0].ops
    if type(o) not in (FP16AccumMatMul, FP32AccumMatMul):
        return False
    packed = ["packed_weight" in m.__dict__ for m in mods]
    if any(packed) and not all(packed):
        return False
    w0 = _weight_meta(mods[0])
    for m in mods:
        if type(m.ops) is not type(o) or any(getattr(m.ops, k, None) != getattr(o, k, None)
                                             for k in ("group_size", "quant_block_size")):
            return False
        shape, dtype, device, contiguous = _weight_meta(m)
        if m.bias is not None or dtype != torch.float16 or device.type != "cuda" or device != w0[2] \
                or len(shape) != 2 or shape[1] != w0[0][1] or not contiguous:
            return False
    qb = getattr(o, "quant_block_size", None)
    return qb is None or all(m.out_features % qb == 0 for m in mods[:-1])


def _weight_meta(m):
    """(shape, dtype, device, contiguous) of the weight the GEMM reads (a packed one decodes contiguous)."""
    p = m.__dict__.get("packed_weight")
    if p is not None:
        return tuple(p.shape), p.dtype, p.codes.device, True
    w = m.weight
    return tuple(w.shape), w.dtype, w.device, w.is_contiguous()


def _stacked_weight(mods):
    """The weights of `mods` as consecutive row ranges of one [sum N, K] tensor.  Built on first
    use by moving each weight into the stack (its parameter then views its rows: no memory is
    added, and in-place updates of a weight land in the stack); built again when a weight has
    been replaced (assignment to .data, .to(), a new Parameter).  Packed weights are decoded
    into consecutive row ranges of a shared scratch stack instead."""
    if "packed_weight" in mods[0].__dict__:
        from .packed import decoded_stack
        return decoded_stack([m.packed_weight for m in mods])
    W = mods[0].__dict__.get("_hbq_stack")
    if W is not None:
        off = 0
        for m in mods:
            w = m.weight
            if w.data_ptr() != W.data_ptr() + off * W.stride(0) * W.element_size() or w.shape[0] != m.out_features \
                    or w.shape[1] != W.shape[1] or w.device != W.device:
                break
            off += w.shape[0]
        else:
            if off == W.shape[0]:
                return W
    with torch.no_grad():
        W = torch.cat([m.weight.detach() for m in mods])
        off = 0
        for m in mods:
            n = m.weight.shape[0]
            m.weight.data = W[off:off + n]
            off += n
    mods[0].__dict__["_hbq_stack"] = W
    return W


def forward_quantized_stacked(mods, xq):
    """[m.forward_quantized(xq) for m in mods] as one GEMM over the stacked weights when the
    linears allow it (same bits per output column), else one GEMM each.  The outputs are
    column slices of the one result; each gets its module's finiteness check and yq."""
    if len(mods) < 2 or not _fusable(mods):
        return [m.forward_quantized(xq) for m in mods]
    y = mods[0].ops(xq, _stacked_weight(mods), None)
    outs, off = [], 0
    for m in mods:
        ym = y[..., off:off + m.out_features]
        off += m.out_features
        m._check_finite(ym)
        outs.append(m.yq(ym))
    return outs


class _QBaseLinear(nn.Linear):
    """Low-precision linear layer (src/module.py:20-67)."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, ops=None):
        super().__init__(in_features, out_features, bias)
        self.wq = _QBase()
        self.aq = _QBase()
        self.yq = _QBase()
        self.ops = ops

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # the weight was quantized in place before inference (src/ptq.py:338-358)
        return self.forward_quantized(self.aq(x))

    def gemm_weight(self, copy: bool = False) -> torch.Tensor:
        """The weight the GEMM reads: the parameter, or for a packed weight
        (hbq_amd.packed.pack_linear_weights) its decoded fake-quantized values, which live
        in a scratch buffer that the next decode of that shape on the stream overwrites
        (copy=True: a tensor of its own, for use outside the forward)."""
        p = self.__dict__.get("packed_weight")
        if p is None:
            return self.weight
        from .packed import decoded_weight
        return decoded_weight(p, copy=copy)

    def forward_quantized(self, xq: torch.Tensor) -> torch.Tensor:
        """forward() on an input already quantized by a quantizer equal to self.aq."""
        y = None
        p = self.__dict__.get("packed_weight")
        if p is not None and self.ops is not None:
            from .packed import linear_packed
            y = linear_packed(xq, p, self.ops, self.bias)   # decode-sized inputs: codes decoded in the GEMM
        if y is None:
            w = self.gemm_weight()
            if self.ops is None:
                y = F.linear(xq, w, self.bias)
            else:
                y = self.ops(xq, w, self.bias)
        self._check_finite(y)
        return self.yq(y)

    def _check_finite(self, y):
        # src/module.py:51-66: a non-finite GEMM output is an error of the format choice
        if _DEFERRED and y.is_cuda and y.dtype in _lib.DTYPE_CODE:
            _DEFERRED[-1].check(self, y)
            return
        if bool(torch.isfinite(y).all()):
            return
        ops_name = type(self.ops).__name__ if self.ops is not None else "F.linear"
        raise RuntimeError(
            f"Non-finite output from {type(self).__name__}({self.in_features} -> {self.out_features}): "
            f"{int(y.isnan().sum())} NaN and {int(y.isinf().sum())} Inf out of {y.numel()} elements.\n"
            f"  activation quantizer: {type(self.aq).__name__}\n"
            f"  weight quantizer:     {type(self.wq).__name__}\n"
            f"  matmul:               {ops_name}\n"
            "The quantization format cannot represent this layer's dynamic range: check the element and "
            "scale exponent bits and the block size of the quantization config.")
