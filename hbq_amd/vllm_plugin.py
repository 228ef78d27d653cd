"""vLLM quantization plugin over the HIP quantizers: the `hbq_nvfp4` method.

A second caller of the quantizers, beside the PTQ path: vLLM builds one
`HBQNVFP4LinearMethod` per linear layer (lm_head excluded). The method
fake-quantizes the loaded weight once, in row chunks, and quantizes each
activation before the layer's matmul. Helpers quantize post-RoPE Q and the K/V
cache the way the Transformers path does. Mirrors vllm/src/hbq_vllm_quant.py
(the reference plugin): the config keys and their defaults (`default_nvfp4_config`,
:608-657), the quantizer construction (`_build_quantizer`, :47-81), the chunked
weight quantization (:263-282), the K/V helpers (:284-338), the AWQ scale and clip
handling (:120-208), `HBQNVFP4LinearMethod` (:493-555) and `HBQNVFP4Config`
(:558-605).

vLLM is optional. When it imports, the classes derive from its linear-method and
quantization-config bases, and the config is registered as "hbq_nvfp4". Without
it they work on plain `torch.nn.Linear` layers, which is how the tests run them.
The attention-forward patch that calls the K/V helpers inside vLLM's
LlamaAttention (reference :399-490) depends on vLLM's module internals. It is not
part of this module.

One difference from the reference: AWQ metadata files are read with
`torch.load(..., weights_only=True)`, which executes nothing from the file.
"""
from __future__ import annotations

import json
import os
from typing import Any

import torch

from .quantizer import HBQQuantizer, MXFPQuantizer

try:
    from vllm.model_executor.layers.linear import LinearBase, UnquantizedLinearMethod
    from vllm.model_executor.layers.quantization import register_quantization_config
    from vllm.model_executor.layers.quantization.base_config import QuantizationConfig, QuantizeMethodBase
    HAVE_VLLM = True
except ImportError:   # the plugin still works on plain torch layers
    HAVE_VLLM = False
    LinearBase = None
    UnquantizedLinearMethod = object
    QuantizationConfig = object
    QuantizeMethodBase = object

CONFIG_ENV = "HBQ_VLLM_QUANT_CONFIG_JSON"
SUPPORTED_QTYPES = ("mxfp", "hbq")

_active: dict[str, Any] | None = None
_awq_cache: dict[str, dict[str, Any]] = {}


def default_nvfp4_config() -> dict[str, Any]:
    """The plugin's default: NVFP4 (E2M1, block 16, E5M3 scale) weights and activations,
    no K/V or attention-weight quantization (vllm/src/hbq_vllm_quant.py:608-657)."""
    blk = {}
    for p in ("act", "wgt"):
        blk.update({f"{p}_ebit": 2, f"{p}_mbit": 1, f"{p}_block_size": 16, f"{p}_sc_ebit": 5, f"{p}_sc_mbit": 3,
                    f"{p}_per_tensor_scale": False, f"{p}_scale_use_ceil": False, f"{p}_l2_sc_bit": 2,
                    f"{p}_l2_block_size": 8})
    blk["scale_allow_subnormal"] = False
    blk["act_l2_scheme"] = "SIG-1"
    blk["wgt_l2_scheme"] = "Mix"
    flags = ("quant_before_hadamard", "quant_before_silu", "quant_before_rms_norm", "quant_output_layer",
             "quant_post_rope_q", "quant_4b_kv", "quant_k_cache", "quant_v_cache", "quant_attn_wgt")
    quantization = {"xqtype": "mxfp", "wqtype": "mxfp"}
    quantization.update({f: False for f in flags})
    return {"quantization": quantization, "block_quant": blk}


def set_active_quant_config(quant_config: dict[str, Any]) -> None:
    """Make `quant_config` the one the plugin uses. It is also stored, as JSON, in the
    environment, so that vLLM worker processes started later see it
    (vllm/src/hbq_vllm_quant.py:84-91)."""
    global _active
    _active = quant_config
    os.environ[CONFIG_ENV] = json.dumps(quant_config)


def active_quant_config() -> dict[str, Any]:
    """The active config: the one set in this process, else the environment's, else
    the NVFP4 default."""
    if _active is not None:
        return _active
    raw = os.environ.get(CONFIG_ENV)
    return json.loads(raw) if raw else default_nvfp4_config()


def _check_qtype(kind: str, qtype: str) -> None:
    if qtype not in SUPPORTED_QTYPES:
        raise ValueError(f"HBQ vLLM prototype only supports {kind}=mxfp or hbq, got {qtype!r}")


def build_quantizer(quant_config: dict[str, Any], prefix: str, qtype: str | None = None,
                    force_4bit: bool = False):
    """The quantizer of `prefix` ("act" or "wgt") in `quant_config`.

    As in the reference plugin, `use_ceil` reaches both quantizer kinds, the HBQ
    quantizer uses the eager element rounding (use_quant_kernel=False), and
    `force_4bit` (the 4-bit K/V option) replaces the element format by E2M1
    (vllm/src/hbq_vllm_quant.py:47-81)."""
    blk = quant_config.get("block_quant", {})
    if qtype is None:
        qtype = quant_config.get("quantization", {}).get("xqtype" if prefix == "act" else "wqtype", "mxfp")
    _check_qtype(prefix, qtype)
    kw = dict(block_size=blk[f"{prefix}_block_size"],
              ebit=2 if force_4bit else blk[f"{prefix}_ebit"],
              mbit=1 if force_4bit else blk[f"{prefix}_mbit"],
              sc_ebit=blk[f"{prefix}_sc_ebit"], sc_mbit=blk[f"{prefix}_sc_mbit"],
              per_tensor_scale=blk.get(f"{prefix}_per_tensor_scale", False),
              scale_allow_subnormal=blk.get("scale_allow_subnormal", False),
              use_ceil=blk.get(f"{prefix}_scale_use_ceil", False))
    if qtype == "mxfp":
        return MXFPQuantizer(**kw, activate_dynamo=False)
    return HBQQuantizer(**kw, l2_block_size=blk[f"{prefix}_l2_block_size"], l2_sc_bit=blk[f"{prefix}_l2_sc_bit"],
                        l2_scheme=blk[f"{prefix}_l2_scheme"], use_quant_kernel=False)


def weight_quant_chunk_rows(quant_config: dict[str, Any]) -> int:
    """Rows quantized at a time: `block_quant.wgt_quant_chunk_rows`, else the
    HBQ_WGT_QUANT_CHUNK_ROWS environment variable, else 1024."""
    return int(quant_config.get("block_quant", {}).get("wgt_quant_chunk_rows",
                                                        os.environ.get("HBQ_WGT_QUANT_CHUNK_ROWS", 1024)))


def quantize_weight_in_chunks(weight: torch.Tensor, quantizer, chunk_rows: int) -> torch.Tensor:
    """quantizer.q(weight), a slice of output rows at a time. Blocks run along the last
    dimension, so row slices keep every block whole and only bound the temporaries
    (vllm/src/hbq_vllm_quant.py:263-282)."""
    if weight.dim() < 2 or chunk_rows <= 0 or weight.shape[0] <= chunk_rows:
        return quantizer.q(weight).to(weight.dtype)
    out = torch.empty_like(weight)
    for r0 in range(0, weight.shape[0], chunk_rows):
        r1 = min(r0 + chunk_rows, weight.shape[0])
        out[r0:r1] = quantizer.q(weight[r0:r1]).to(weight.dtype)
    return out


def act_quantizer(quant_config: dict[str, Any] | None = None):
    cfg = quant_config or active_quant_config()
    return build_quantizer(cfg, "act", qtype=cfg.get("quantization", {}).get("xqtype", "mxfp"))


def kv_quantizer(quant_config: dict[str, Any] | None = None):
    """The activation quantizer, in E2M1 when `quant_4b_kv` is set (reference :251-260)."""
    cfg = quant_config or active_quant_config()
    q = cfg.get("quantization", {})
    return build_quantizer(cfg, "act", qtype=q.get("xqtype", "mxfp"), force_4bit=q.get("quant_4b_kv", False))


def quantize_post_rope_q(q: torch.Tensor, num_heads: int, head_dim: int, quant_config=None) -> torch.Tensor:
    """Post-RoPE Q, [tokens, heads * head_dim], through the activation quantizer along
    head_dim (reference :284-289)."""
    return act_quantizer(quant_config).q(q.reshape(-1, num_heads, head_dim)).reshape(q.shape).to(q.dtype)


def quantize_k_cache(k: torch.Tensor, num_kv_heads: int, head_dim: int, quant_config=None) -> torch.Tensor:
    """Post-RoPE K, [tokens, kv_heads * head_dim], along head_dim (reference :292-298)."""
    return kv_quantizer(quant_config).q(k.reshape(-1, num_kv_heads, head_dim)).reshape(k.shape).to(k.dtype)


def sequence_spans(positions: torch.Tensor | None, n_tokens: int) -> list[tuple[int, int]]:
    """[start, end) token ranges of the sequences vLLM packed into one batch: a new one
    starts wherever a position does not follow the previous one (reference :301-311)."""
    if positions is None or positions.numel() != n_tokens:
        return [(0, n_tokens)]
    pos = positions.detach().flatten().to("cpu", torch.long)
    cuts = (torch.nonzero(pos[1:] != pos[:-1] + 1).flatten() + 1).tolist()
    bounds = [0] + cuts + [n_tokens]
    return list(zip(bounds[:-1], bounds[1:]))


def quantize_v_cache(v: torch.Tensor, num_kv_heads: int, head_dim: int, positions: torch.Tensor | None = None,
                     quant_config=None) -> torch.Tensor:
    """V, [tokens, kv_heads * head_dim], quantized along the token axis of each sequence
    separately: the Transformers path's [batch, kv_heads, head_dim, tokens] layout
    (reference :314-336)."""
    vv = v.reshape(-1, num_kv_heads, head_dim)
    qz = kv_quantizer(quant_config)
    out = torch.empty_like(vv)
    for t0, t1 in sequence_spans(positions, vv.shape[0]):
        if t1 > t0:
            seq = qz.q(vv[t0:t1].permute(1, 2, 0).contiguous())
            out[t0:t1] = seq.permute(2, 0, 1).to(v.dtype)
    return out.reshape(v.shape)


# ---- AWQ scales and clips (reference :120-208) -------------------------------------

def awq_target(name: str) -> str:
    """vLLM's fused layer for a Hugging Face projection name: q/k/v_proj -> qkv_proj,
    gate/up_proj -> gate_up_proj; other names unchanged."""
    head, _, leaf = name.rpartition(".")
    if head.endswith(".self_attn") and leaf in ("q_proj", "k_proj", "v_proj"):
        return head + ".qkv_proj"
    if head.endswith(".mlp") and leaf in ("gate_proj", "up_proj"):
        return head + ".gate_up_proj"
    return name


def awq_metadata(quant_config: dict[str, Any] | None = None) -> dict[str, Any] | None:
    """{"scale": {vLLM layer: input-channel scale}, "clip": {HF layer: clip}} from the AWQ
    file of `awq.load_path` (or `awq.dump_path`), or None when `awq.enable` is off."""
    cfg = quant_config or active_quant_config()
    awq = cfg.get("awq", {})
    if not awq.get("enable", False):
        return None
    path = awq.get("load_path") or awq.get("dump_path")
    if not path:
        raise ValueError("awq.enable is true but neither awq.load_path nor awq.dump_path is set")
    path = str(path)
    if path not in _awq_cache:
        raw = torch.load(path, map_location="cpu", weights_only=True)
        scales = {awq_target(n): s.detach().cpu() for _, names, s in raw.get("scale", []) for n in names}
        clips = {n: c.detach().cpu() for n, c in raw.get("clip", [])}
        _awq_cache[path] = {"scale": scales, "clip": clips}
    return _awq_cache[path]


def _clip_rows(w: torch.Tensor, max_val: torch.Tensor) -> None:
    if w.shape[0] != max_val.shape[0]:
        raise ValueError(f"AWQ clip row mismatch for weight shape {tuple(w.shape)} and clip shape "
                         f"{tuple(max_val.shape)}")
    m = max_val.to(w.device, w.dtype)
    view = w.reshape(*m.shape[:2], -1)
    view.copy_(torch.clamp(view, -m, m))


def apply_awq_clip(layer: torch.nn.Module, prefix: str, quant_config=None) -> None:
    """Clip the weight rows of `prefix` to the AWQ maxima; a fused qkv or gate_up layer
    takes the clips of its parts, in row order (v only for qkv, as the reference)."""
    meta = awq_metadata(quant_config)
    w = getattr(layer, "weight", None)
    if meta is None or w is None:
        return
    clips = meta["clip"]
    if prefix.endswith(".self_attn.qkv_proj"):
        c = clips.get(prefix[: -len(".qkv_proj")] + ".v_proj")
        if c is not None:
            _clip_rows(w.data[-c.shape[0]:], c)
        return
    if prefix.endswith(".mlp.gate_up_proj"):
        base, row = prefix[: -len(".gate_up_proj")], 0
        for part in ("gate_proj", "up_proj"):
            c = clips.get(f"{base}.{part}")
            if c is not None:
                _clip_rows(w.data[row:row + c.shape[0]], c)
                row += c.shape[0]
        return
    c = clips.get(prefix)
    if c is not None:
        _clip_rows(w.data, c)


# ---- the linear method and the config -----------------------------------------------

class HBQNVFP4LinearMethod(UnquantizedLinearMethod):
    """Fake-quantized weights and activations for one linear layer
    (vllm/src/hbq_vllm_quant.py:493-555)."""

    def __init__(self, quant_config: dict[str, Any], prefix: str) -> None:
        super().__init__()
        self.quant_config = quant_config
        self.prefix = prefix
        q = quant_config.get("quantization", {})
        self.act_q = build_quantizer(quant_config, "act", qtype=q.get("xqtype", "mxfp"))
        self.wgt_q = build_quantizer(quant_config, "wgt", qtype=q.get("wqtype", "mxfp"))

    def _awq_scale(self):
        meta = awq_metadata(self.quant_config)
        return None if meta is None else meta["scale"].get(self.prefix)

    @torch.inference_mode()
    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """Once per layer: AWQ scale and clip, then the weight quantizer in row chunks.
        HBQ_DEBUG_SKIP_WGT_QUANT=1 leaves the weight as loaded."""
        if HAVE_VLLM:
            base = getattr(super(), "process_weights_after_loading", None)
            if base is not None:
                base(layer)
        w = getattr(layer, "weight", None)
        if w is None or getattr(layer, "hbq_weight_quantized", False):
            return
        if os.environ.get("HBQ_DEBUG_SKIP_WGT_QUANT") == "1":
            return
        s = self._awq_scale()
        if s is not None:
            if s.numel() != w.shape[1]:
                raise ValueError(f"AWQ scale width mismatch for {self.prefix}: scale={tuple(s.shape)}, "
                                 f"weight={tuple(w.shape)}")
            w.data.mul_(s.to(w.device, w.dtype).view(1, -1))
        apply_awq_clip(layer, self.prefix, self.quant_config)
        w.data = quantize_weight_in_chunks(w.data, self.wgt_q, weight_quant_chunk_rows(self.quant_config))
        layer.hbq_weight_quantized = True

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: torch.Tensor | None = None) -> torch.Tensor:
        """layer(x) on the quantized activation (divided by the AWQ scale first, unless
        `awq.apply_act_scale` is false)."""
        s = self._awq_scale()
        if s is not None and self.quant_config.get("awq", {}).get("apply_act_scale", True):
            x = x / s.to(x.device, x.dtype).view(*([1] * (x.dim() - 1)), -1)
        xq = self.act_q.q(x)
        if HAVE_VLLM:
            return super().apply(layer, xq, bias)
        return torch.nn.functional.linear(xq, layer.weight, bias)


class HBQNVFP4Config(QuantizationConfig):
    """The `hbq_nvfp4` quantization config (vllm/src/hbq_vllm_quant.py:558-605)."""

    UNSUPPORTED = ("quant_attn_wgt", "quant_output_layer")

    def __init__(self, quant_config: dict[str, Any] | None = None) -> None:
        if HAVE_VLLM:
            super().__init__()
        self.quant_config = quant_config or active_quant_config()
        q = self.quant_config.get("quantization", {})
        _check_qtype("xqtype", q.get("xqtype", "mxfp"))
        _check_qtype("wqtype", q.get("wqtype", "mxfp"))
        on = [f for f in self.UNSUPPORTED if q.get(f, False)]
        if on:
            raise NotImplementedError("HBQ-vllm direct PTQ currently supports linear W/A quantization and optional "
                                      f"K/V cache fake quantization. Unsupported enabled flags: {on}")

    def get_name(self) -> str:
        return "hbq_nvfp4"

    def get_supported_act_dtypes(self) -> list[torch.dtype]:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return -1

    @staticmethod
    def get_config_filenames() -> list[str]:
        return []

    @classmethod
    def from_config(cls, config: dict[str, Any]) -> "HBQNVFP4Config":
        return cls(config or active_quant_config())

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        """The linear method for every linear layer but the LM head; None otherwise."""
        if "lm_head" in prefix:
            return None
        linear = isinstance(layer, LinearBase) if HAVE_VLLM else isinstance(layer, torch.nn.Linear)
        return HBQNVFP4LinearMethod(self.quant_config, prefix) if linear else None

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg, user_quant) -> str | None:
        return "hbq_nvfp4" if user_quant == "hbq_nvfp4" else None

    def get_scaled_act_names(self) -> list[str]:
        return []


if HAVE_VLLM:
    HBQNVFP4Config = register_quantization_config("hbq_nvfp4")(HBQNVFP4Config)
