"""HIP-backed drop-in for the reference quantizer module (src/quantizer.py).

Class names, constructor signatures and defaults, the q()/forward() interface
and the keep_l2_scale attributes follow src/quantizer.py; the arithmetic runs
in the fused gfx950 kernels of libhbq_amd.so (include/hbq_amd.h).  Inputs
must be GPU tensors: there is no CPU path.

Differences a caller can observe:
  * quantize() is an addition: it returns the element codes and block scales
    that q() computes but discards.
  * The GPU kernels cover element formats E2M1/E2M2/E2M3 (HBQ) and
    E2M1/E2M2/E2M3/E2M5 (MXFP), power-of-two block sizes 16..1024 and L2
    block sizes 4..32; other settings raise NotImplementedError.
  * MXINTQuantizer, MXExQuantizer and VSQQuantizer exist so that callers
    importing them keep working; they are not part of this GPU path and
    raise NotImplementedError when constructed.
"""
from collections import namedtuple
from dataclasses import dataclass
from typing import Callable, Dict

import torch
import torch.nn as nn

from . import _lib

FP32_EXPONENT_BIAS = 127
FP16_EXPONENT_BIAS = 15
FP32_MIN_NORMAL = 2 ** (-FP32_EXPONENT_BIAS + 1)
FP16_MIN_NORMAL = 2 ** (-FP16_EXPONENT_BIAS + 1)
FP32_MAX_NORMAL = 2 ** (-FP32_EXPONENT_BIAS + 2 ** 10)
FP16_MAX_NORMAL = 2 ** (-FP16_EXPONENT_BIAS + 2 ** 5)

QuantOutput = namedtuple("QuantOutput", ["y", "codes", "scales", "l2_index", "scheme"])


# ---------------------------------------------------------------------------
# format constants (src/quantizer.py:148-185)
# ---------------------------------------------------------------------------
def get_max_norm(ebit: int, mbit: int, unsigned: bool = False):
    """Largest normal value of E(ebit)M(mbit); INT(mbit) when ebit == 0."""
    if ebit == 0:
        return 2 ** mbit - 1 if unsigned else 2 ** (mbit - 1) - 1
    if (ebit, mbit) == (4, 3):
        return 448
    emax = 15 if ebit == 5 else 2 ** (ebit - 1)
    return 2 ** emax * float(2 ** (mbit + 1) - 1) / 2 ** mbit


def get_min_norm(ebit: int, mbit: int):
    """Smallest normal value of E(ebit)M(mbit) (0 for integers)."""
    if ebit == 0:
        return 0
    if ebit == 1:
        return 1
    return 2 ** (2 - 2 ** (ebit - 1))


def get_min_subnorm(ebit: int, mbit: int):
    """Smallest subnormal value of E(ebit)M(mbit)."""
    return 2 ** (2 - 2 ** (ebit - 1)) * 2 ** (-mbit)


# ---------------------------------------------------------------------------
# block view helpers (src/quantizer.py:67-146)
# ---------------------------------------------------------------------------
def _reshape_to_blocks(A, axes, block_size):
    """View A with every axis in `axes` split into (n_blocks, block_size),
    zero padding each such axis to a multiple of block_size.

    Returns (blocked view, shifted axes, shape before padding, padded shape)."""
    if axes is None:
        raise Exception("axes required in order to determine which dimension to apply block size to")
    if block_size == 0:
        raise Exception("block_size == 0 in _reshape_to_blocks")
    axes = sorted(a + A.dim() if a < 0 else a for a in axes)
    shifted = []
    for i, ax in enumerate(axes):
        ax = ax + i
        A = A.unsqueeze(ax + 1)
        shifted.append(ax)
    orig_shape = A.size()
    pad = [0] * (2 * A.dim())
    need_pad = False
    for ax in shifted:
        rem = orig_shape[ax] % block_size
        if rem:
            # F.pad lists the last dimension first
            pad[2 * (A.dim() - 1 - ax) + 1] = block_size - rem
            need_pad = True
    if need_pad:
        A = torch.nn.functional.pad(A, pad, mode="constant")
    padded_shape = A.size()
    shape = list(padded_shape)
    for ax in shifted:
        n = shape[ax]
        if n >= block_size:
            shape[ax], shape[ax + 1] = n // block_size, block_size
        else:
            shape[ax], shape[ax + 1] = 1, n
    return A.view(shape), shifted, orig_shape, padded_shape


def _undo_reshape_to_blocks(A, padded_shape, orig_shape, axes):
    """Inverse of _reshape_to_blocks: merge blocks, drop the padding, squeeze."""
    A = A.view(padded_shape)
    if list(padded_shape) != list(orig_shape):
        A = A[tuple(slice(0, n) for n in orig_shape)]
    for ax in reversed(axes):
        A = torch.squeeze(A, dim=ax + 1)
    return A


# ---------------------------------------------------------------------------
# scalar quantizers
# ---------------------------------------------------------------------------
def _as_rows(x):
    xc = x.contiguous()
    cols = xc.shape[-1] if xc.dim() > 0 else 1
    rows = xc.numel() // cols if cols else 0
    return xc, rows, cols


def make_fp_quant(ebit: int, mbit: int, allow_subnormal: bool = True, detailed_output: bool = False,
                  use_ceil: bool = False, emax: int = None, emin: int = None):
    """Element quantizer of E(ebit)M(mbit) (src/quantizer.py:187-257) as a GPU callable,
    with the rounding of the eager op chain (each step rounded to the tensor dtype)."""
    return _elem_quantizer(ebit, mbit, allow_subnormal, detailed_output, use_ceil, emax, emin, compiled=False)


def _elem_quantizer(ebit, mbit, allow_subnormal, detailed_output, use_ceil, emax, emin, compiled):
    if ebit != 2 or not allow_subnormal or detailed_output or use_ceil or emax is not None or emin is not None:
        raise NotImplementedError(
            "the GPU element quantizer implements E2Mm with subnormals and nearest rounding only")

    def lpfp_quant(x: torch.Tensor):
        _lib.require_gpu(x, "lpfp_quant")
        if x.dtype not in _lib.DTYPE_CODE:
            raise NotImplementedError(f"Non-supported data type: {x.dtype}")
        xc = x.contiguous()
        y = torch.empty_like(xc)
        _lib.check(_lib.lib().hbq_elem_quant(_lib.ptr(xc), _lib.ptr(y), None, xc.numel(), _lib.DTYPE_CODE[x.dtype],
                                             ebit, mbit, int(compiled), _lib.stream_of(xc)), NotImplementedError)
        return y

    lpfp_quant.compiled = compiled
    return lpfp_quant


@dataclass(frozen=True)
class FPQuantConfig:
    ebit: int
    mbit: int
    allow_subnormal: bool = True
    detailed_output: bool = False
    use_ceil: bool = False
    emax: int = None
    emin: int = None

    @property
    def key(self):
        return (self.ebit, self.mbit, self.allow_subnormal, self.detailed_output, self.use_ceil, self.emax,
                self.emin)


class FPQuantCompilerCache:
    """Cache of element quantizers by format (src/quantizer.py:38-65).

    The reference serves make_fp_quant's function compiled with torch.compile,
    which fuses the op chain into one fp32 kernel: the sum |m| + 0.5004 is not
    rounded to the tensor dtype, unlike the eager chain.  Every entry here is the
    HIP element kernel with that fused rounding, so there is nothing to compile
    or warm up."""

    def __init__(self):
        self._cache: Dict[tuple, Callable[[torch.Tensor], torch.Tensor]] = {}

    def get(self, cfg: FPQuantConfig) -> Callable[[torch.Tensor], torch.Tensor]:
        fn = self._cache.get(cfg.key)
        if fn is None:
            fn = _elem_quantizer(cfg.ebit, cfg.mbit, cfg.allow_subnormal, cfg.detailed_output, cfg.use_ceil,
                                 cfg.emax, cfg.emin, compiled=True)
            self._cache[cfg.key] = fn
        return fn


GLOBAL_FP_QUANT_CACHE = FPQuantCompilerCache()


def fp_quant(x: torch.Tensor, ebit: int, mbit: int, allow_subnormal: bool = True, detailed_output: bool = False,
             use_ceil: bool = False, emax: int = None, emin: int = None):
    """Scale quantizer (src/quantizer.py:259-328) on the GPU: round to E(ebit)M(mbit),
    half-up or ceil, optional subnormals."""
    if detailed_output or emax is not None or emin is not None:
        raise NotImplementedError("fp_quant: detailed_output/emax/emin are not implemented on the GPU path")
    return _scale_quant(x, ebit, mbit, allow_subnormal, use_ceil, clip=False)


def _scale_quant(x, ebit, mbit, allow_subnormal, use_ceil, clip):
    _lib.require_gpu(x, "fp_quant")
    if x.dtype not in _lib.DTYPE_CODE:
        raise NotImplementedError(f"Non-supported data type: {x.dtype}")
    xc = x.contiguous()
    y = torch.empty_like(xc)
    _lib.check(_lib.lib().hbq_scale_quant(_lib.ptr(xc), _lib.ptr(y), xc.numel(), _lib.DTYPE_CODE[x.dtype], ebit,
                                          mbit, int(allow_subnormal), int(use_ceil), int(clip),
                                          _lib.stream_of(xc)), NotImplementedError)
    return y


# ---------------------------------------------------------------------------
# quantizer modules
# ---------------------------------------------------------------------------
class _QBase(nn.Module):
    """Base quantizer: q() is the identity (src/quantizer.py:330-345)."""

    def __init__(self):
        super().__init__()

    def q(self, x: torch.Tensor):
        return x

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.q(x)


class _NotOnGPUPath(_QBase):
    def __init__(self, *args, **kwargs):
        raise NotImplementedError(f"{type(self).__name__} is not part of the MI355X HBQ GPU path")


class MXINTQuantizer(_NotOnGPUPath):
    """MXINT block quantizer (src/quantizer.py:347-428); not implemented here."""


class MXExQuantizer(_NotOnGPUPath):
    """Micro-exponent quantizer (src/quantizer.py:541-636); not implemented here."""


class VSQQuantizer(_NotOnGPUPath):
    """VSQ quantizer (src/quantizer.py:638-702); not implemented here."""


class MXFPQuantizer(_QBase):
    """MX/NV block floating point quantizer (src/quantizer.py:430-539).

    sc_mbit == 0 gives the power-of-two shared scale (MXFP4/MXFP8), otherwise
    an E(sc_ebit)M(sc_mbit) scale (NVFP4).  fp16 and fp32 inputs only, as in
    the reference (bf16 raises NotImplementedError)."""

    def __init__(self, block_size: int = 32, ebit: int = 2, mbit: int = 3, sc_ebit: int = 0, sc_mbit: int = 8,
                 per_tensor_scale: bool = False, scale_allow_subnormal: bool = False, use_round: bool = False,
                 use_ceil: bool = False, activate_dynamo: bool = False):
        super().__init__()
        self.ebit = ebit
        self.mbit = mbit
        self.sc_ebit = sc_ebit
        self.sc_mbit = sc_mbit
        self.block_size = block_size
        self.per_tensor_scale = per_tensor_scale
        self.scale_allow_subnormal = scale_allow_subnormal
        self.use_round = use_round
        self.use_ceil = use_ceil
        lp_config = FPQuantConfig(ebit=self.ebit, mbit=self.mbit, allow_subnormal=True, detailed_output=False)
        self._lp_config = lp_config
        # the element rounding follows the flag as in the reference (src/quantizer.py:464-469):
        # the compiled function of GLOBAL_FP_QUANT_CACHE, or the eager make_fp_quant
        self._fused = bool(activate_dynamo)

    @property
    def lpfp_quant(self):
        if self._fused:
            return GLOBAL_FP_QUANT_CACHE.get(self._lp_config)
        c = self._lp_config
        return make_fp_quant(c.ebit, c.mbit, c.allow_subnormal, c.detailed_output, c.use_ceil, c.emax, c.emin)

    def reshape(self, x: torch.Tensor):
        return _reshape_to_blocks(x, [-1], block_size=self.block_size)

    def _check_dtype(self, x):
        if x.dtype not in (torch.float32, torch.float16):
            raise NotImplementedError(f"Non-supported data type: {x.dtype}")

    def _tensor_scale(self, x):
        ele_max = get_max_norm(ebit=self.ebit, mbit=self.mbit)
        sc_max = get_max_norm(ebit=self.sc_ebit, mbit=self.sc_mbit)
        x_max = x.abs().max().item()
        return 1.0 if x_max == 0 else x_max / (ele_max * sc_max)

    def _run(self, x, block_size, want_codes, want_scales):
        self._check_dtype(x)
        _lib.require_gpu(x, type(self).__name__)
        xc, rows, cols = _as_rows(x)
        y = torch.empty_like(xc)
        nblk = -(-cols // block_size) if cols else 0
        scales = torch.empty(x.shape[:-1] + (nblk,), dtype=x.dtype, device=x.device) if want_scales else None
        codes = None
        if want_codes:
            per_row = (cols + 1) // 2 if self.mbit == 1 else cols
            codes = torch.empty(x.shape[:-1] + (per_row,), dtype=torch.uint8, device=x.device)
        per = bool(self.per_tensor_scale)
        ts = self._tensor_scale(xc) if per and xc.numel() else 1.0
        if xc.numel():
            _lib.check(_lib.lib().hbq_mxfp_qdq(
                _lib.ptr(xc), _lib.ptr(y), _lib.ptr(scales), _lib.ptr(codes), rows, cols, _lib.DTYPE_CODE[x.dtype],
                block_size, self.ebit, self.mbit, self.sc_ebit, self.sc_mbit, int(self.scale_allow_subnormal),
                int(self.use_round), int(self.use_ceil), int(per), float(ts), int(self._fused), _lib.stream_of(xc)),
                NotImplementedError)
        return y.view(x.shape), codes, scales

    def get_shared_scale(self, x: torch.Tensor) -> torch.Tensor:
        """Shared scale of each block of the blocked view x [..., n_blocks, block] -> [..., n_blocks, 1]."""
        self._check_dtype(x)
        _, _, s = self._run(x, x.shape[-1], want_codes=False, want_scales=True)
        return s.view(x.shape[:-1] + (1,))

    def q(self, x: torch.Tensor):
        y, _, _ = self._run(x, self.block_size, want_codes=False, want_scales=False)
        return y

    def quantize(self, x: torch.Tensor) -> QuantOutput:
        """q(x) plus the element codes and per-block scales."""
        y, codes, scales = self._run(x, self.block_size, want_codes=True, want_scales=True)
        return QuantOutput(y, codes, scales, None, None)


class HBQQuantizer(MXFPQuantizer):
    """Hierarchical (two-level) block quantizer (src/quantizer.py:704-859).

    Per block: an E5M3 L1 scale per scheme; per L2 sub-block the L2 factor
    with the least squared error; per block the scheme with the least error.
    fp16, bf16 and fp32 inputs."""

    L2_SCHEME = ["PoT", "INT", "SIG-1", "FP-1", "FP1", "FP-10", "FP-100", "Mix"]

    def __init__(self, block_size: int = 128, ebit: int = 2, mbit: int = 3, sc_ebit: int = 5, sc_mbit: int = 3,
                 l2_block_size: int = 4, l2_sc_bit: int = 1, l2_scheme: str = "PoT", keep_l2_scale: bool = False,
                 per_tensor_scale: bool = False, scale_allow_subnormal: bool = False, use_round: bool = False,
                 use_ceil: bool = False, use_quant_kernel: bool = True):
        super().__init__(block_size, ebit, mbit, sc_ebit, sc_mbit, per_tensor_scale, scale_allow_subnormal,
                         use_round, use_ceil, use_quant_kernel)
        assert block_size % l2_block_size == 0, "block_size must be divisible by l2_block_size"
        assert l2_scheme in self.L2_SCHEME, f"Invalid L2 scheme: {l2_scheme}"
        self.keep_l2_scale = keep_l2_scale
        self.l2_block_size = l2_block_size
        self.l2_sc_bit = l2_sc_bit
        self.l2_scheme = l2_scheme
        self.win_rate = []

    def _check_dtype(self, x):
        if x.dtype not in _lib.DTYPE_CODE:
            raise NotImplementedError(f"Non-supported data type: {x.dtype}")

    def quant_scale(self, scale: torch.Tensor):
        """L1 scale quantizer: clip to the E(sc_ebit)M(sc_mbit) range, then fp_quant (src/quantizer.py:735-739)."""
        return _scale_quant(scale, self.sc_ebit, self.sc_mbit, self.scale_allow_subnormal, self.use_ceil, clip=True)

    def l2_table(self, dtype=torch.float32, device=None):
        """L2 candidates [2^l2_sc_bit, n_schemes] (src/quantizer.py:745-770)."""
        r = torch.arange(2 ** self.l2_sc_bit, dtype=dtype, device=device)
        n = 2 ** self.l2_sc_bit
        fp = 1 + r / n
        tabs = {"PoT": torch.pow(2, r), "INT": r + 1, "SIG-1": 1 + r / 2, "FP-1": fp, "FP1": 1 + (r + 1) / n,
                "FP-10": 1 + r / (2 * n), "FP-100": 1 + r / (4 * n)}
        if self.l2_scheme == "Mix":
            return torch.stack([fp, tabs["FP-10"]], dim=-1)
        return tabs[self.l2_scheme][..., None]

    def _run_hbq(self, x, want_codes, want_stats):
        self._check_dtype(x)
        _lib.require_gpu(x, "HBQQuantizer")
        xc, rows, cols = _as_rows(x)
        B = self.block_size
        nblk = -(-cols // B) if cols else 0
        nsub = B // self.l2_block_size
        lead = x.shape[:-1]
        y = torch.empty_like(xc)
        l1 = l2i = sch = codes = None
        if want_stats:
            l1 = torch.empty(lead + (nblk,), dtype=x.dtype, device=x.device)
            l2i = torch.empty(lead + (nblk, nsub), dtype=torch.uint8, device=x.device)
            sch = torch.empty(lead + (nblk,), dtype=torch.uint8, device=x.device)
        if want_codes:
            per_row = (cols + 1) // 2 if self.mbit == 1 else cols
            codes = torch.empty(lead + (per_row,), dtype=torch.uint8, device=x.device)
        if xc.numel():
            _lib.check(_lib.lib().hbq_hbq_qdq(
                _lib.ptr(xc), _lib.ptr(y), _lib.ptr(l1), _lib.ptr(l2i), _lib.ptr(sch), _lib.ptr(codes), rows, cols,
                _lib.DTYPE_CODE[x.dtype], *self.abi_args(), _lib.stream_of(xc)), NotImplementedError)
        return y.view(x.shape), codes, l1, l2i, sch

    def abi_args(self):
        """The quantizer's arguments of the C ABI, block_size .. compiled (include/hbq_amd.h)."""
        return (self.block_size, self.ebit, self.mbit, self.sc_ebit, self.sc_mbit, self.l2_block_size,
                self.l2_sc_bit, self.L2_SCHEME.index(self.l2_scheme), int(self.scale_allow_subnormal),
                int(self.use_ceil), int(self._fused))

    def q(self, x: torch.Tensor):
        y, _, l1, l2i, sch = self._run_hbq(x, want_codes=False, want_stats=self.keep_l2_scale)
        if self.keep_l2_scale:
            self.blk_l2_scheme = sch.long()
            self.shared_scale = l1
            self.l2_scale = l2i.long()
            tab = self.l2_table(dtype=x.dtype, device=x.device)
            self.real_l2_scale = tab[self.l2_scale, self.blk_l2_scheme[..., None]]
        else:
            for name in ("l2_scale", "blk_l2_scheme", "shared_scale", "real_l2_scale"):
                self.__dict__.pop(name, None)
        return y

    def quantize(self, x: torch.Tensor) -> QuantOutput:
        """q(x) plus element codes, L1 scales, L2 indices and scheme bits."""
        y, codes, l1, l2i, sch = self._run_hbq(x, want_codes=True, want_stats=True)
        return QuantOutput(y, codes, l1, l2i, sch)
