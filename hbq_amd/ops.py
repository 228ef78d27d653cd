"""Drop-in for the reference's src/ops.py: FP16AccumMatMul on the HIP GEMMs.

Same constructor, forward(x, w, bias) signature, group-size validation
(ValueError) and dispatch as src/ops.py:16-62.  The weight is handed to the
kernel in its nn.Linear layout W[N, K] instead of materializing w.t() on
every call (src/ops.py:41); the arithmetic is the same.
"""
import torch
import torch.nn as nn

from . import blockquant_ext as ext


class FP16AccumMatMul(nn.Module):
    """Low-precision-accumulation matmul: psum-quantized (quant_block_size set),
    grouped fp16 (group_size set) or pure fp16 accumulation."""

    def __init__(self, group_size: int = None, quant_block_size: int = None):
        super().__init__()
        self.group_size = group_size
        self.quant_block_size = quant_block_size

    def forward(self, x, w, bias=None) -> torch.Tensor:
        orig_shape = x.shape
        x2d = x.reshape(-1, x.shape[-1])
        if x2d.dtype != torch.float16:
            x2d = x2d.half()
        x2d = x2d.to(w.device, non_blocking=True)
        w16 = w if w.dtype == torch.float16 else w.half()
        if self.quant_block_size is not None:
            if self.group_size not in [4, 8, 16, 32, 64, 128]:
                raise ValueError(f"Invalid group size: {self.group_size}")
            if self.quant_block_size not in [4, 8, 16, 32]:
                raise ValueError(f"Invalid quant block size: {self.quant_block_size}")
            out2d = ext.gemm_blockquant_mxint8_nk(x2d, w16, self.group_size, self.quant_block_size)
        elif self.group_size is not None:
            if self.group_size not in [4, 8, 16, 32, 64, 128]:
                raise ValueError(f"Invalid group size: {self.group_size}")
            out2d = ext.gemm_fp16_grouped_accum_nk(x2d, w16, self.group_size)
        else:
            out2d = ext.gemm_fp16_accum_nk(x2d, w16)
        if bias is not None:
            out2d = out2d + bias
        return out2d.view(*orig_shape[:-1], -1)


class FP32AccumMatMul(nn.Module):
    """fp32-accumulation matmul on the HIP GEMM (one fp16 rounding at the end).

    No counterpart in src/ops.py: the reference leaves fp32 accumulation to
    F.linear (cuBLAS).  This operator puts those linears on the same MFMA kernel as
    the other accumulation modes (x [.., K] fp16 against W [N, K], bias added in
    fp16); the fp32 sum order inside a K range differs from any library's, as it
    does between libraries, and long K may be summed as two halves (split K)."""

    def forward(self, x, w, bias=None) -> torch.Tensor:
        orig_shape = x.shape
        x2d = x.reshape(-1, x.shape[-1])
        if x2d.dtype != torch.float16:
            x2d = x2d.half()
        w16 = w if w.dtype == torch.float16 else w.half()
        out2d = ext.gemm_fp32_accum_nk_split(x2d, w16)
        if bias is not None:
            out2d = out2d + bias
        return out2d.view(*orig_shape[:-1], -1)


def use_hip_fp32_gemm(model):
    """Route every fp32-accumulation _QBaseLinear (ops None) of a model's decoder layers
    through FP32AccumMatMul."""
    from .module import _QBaseLinear
    n = 0
    for layer in [m for _, m in model.named_modules() if hasattr(m, "self_attn") and hasattr(m, "mlp")]:
        for mod in layer.modules():
            if isinstance(mod, _QBaseLinear) and mod.ops is None:
                mod.ops = FP32AccumMatMul()
                n += 1
    return n


def stack_qkv_gemms(model):
    """Let every attention block of a model run q, k and v as one GEMM over their stacked
    weights (N = q + k + v outputs) where their operators allow it with the same bits per
    output column; the parameters then view row ranges of the stack.  Returns the number of
    attention blocks switched."""
    n = 0
    for mod in model.modules():
        if hasattr(mod, "stack_qkv"):
            mod.stack_qkv = True
            n += 1
    return n


def fuse_input_quantizers(model, on=True):
    """Let every decoder layer of a model compute its linears' input quantizers inside the
    passes that produce their inputs (RMSNorm -> q/k/v and gate/up, SiLU product -> down),
    where those quantizers are HBQQuantizers that the fused kernels take; the outputs keep
    their bits.  Returns the number of layers switched."""
    n = 0
    for mod in model.modules():
        if hasattr(mod, "fuse_input_quant"):
            mod.fuse_input_quant = bool(on)
            n += 1
    return n
