"""Quantized linear layer: the caller of the HBQ quantizers and GEMMs.

Mirrors `_QBaseLinear` (src/module.py:20-67): an nn.Linear with three
quantizer slots (`wq` weight, `aq` input activation, `yq` output) and an optional
GEMM operator `ops` (an `FP16AccumMatMul`).  The weight is quantized once, in
place, by `PTQ.static_quant_linear_weight`; `forward` quantizes the input, runs
the GEMM (torch's `F.linear` when `ops` is None, as in the reference), raises on
a non-finite result and applies `yq`.
"""
import torch
import torch.nn as nn
import torch.nn.functional as F

from .quantizer import _QBase


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
        xq = self.aq(x)
        if self.ops is None:
            y = F.linear(xq, self.weight, self.bias)
        else:
            y = self.ops(xq, self.weight, self.bias)
        self._check_finite(y)
        return self.yq(y)

    def _check_finite(self, y):
        # src/module.py:51-66: a non-finite GEMM output is an error of the format choice
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
