"""Quantization-config driver: config keys -> quantizers, static weight
quantization, accumulation-kernel replacement.

Mirrors the parts of `PTQ` (src/ptq.py:24-404) that build and apply the hot
path; the model-loading and evaluation parts of the reference stay out.
The class keeps the reference's attribute names and defaults
(src/ptq.py:30-105) and its mapping of config keys onto quantizer constructors
(src/ptq.py:107-257).  Models are walked by duck typing instead of by Hugging
Face layer classes: a decoder layer is any module with `self_attn` (holding
`q_proj`, `k_proj`, `v_proj`, `o_proj`) and `mlp` (holding `gate_proj`,
`up_proj`, `down_proj`), whose projections are `_QBaseLinear`.
"""
import logging
import os

import torch

from .module import _QBaseLinear
from .ops import FP16AccumMatMul
from .quantizer import HBQQuantizer, MXExQuantizer, MXFPQuantizer, MXINTQuantizer, VSQQuantizer, _QBase


def load_config(path):
    """A quantization YAML (the reference's config/*.yaml layout) as a dict."""
    import yaml
    with open(path) as f:
        return yaml.safe_load(f)


class PTQ:
    """Block-quantization driver (src/ptq.py:24)."""

    def __init__(self, quant_config, model=None, tokenizer=None, logger=None):
        self.quant_config = quant_config
        self.model = model
        self.tokenizer = tokenizer
        self.logger = logger or logging.getLogger("hbq_amd.ptq")

        q = quant_config.get("quantization", {})
        b = quant_config.get("block_quant", {})
        acc = quant_config.get("accumulation", {})
        # KeyError when a type is missing, as in the reference (src/ptq.py:40-41)
        self.xqtype = q["xqtype"]
        self.wqtype = q["wqtype"]

        # element / scale formats (defaults: src/ptq.py:44-57)
        self.a_ebit = b.get("act_ebit", 0)
        self.a_mbit = b.get("act_mbit", 0)
        self.a_sc_ebit = b.get("act_sc_ebit", 0)
        self.a_sc_mbit = b.get("act_sc_mbit", 8)
        self.a_block_size = b.get("act_block_size", 32)
        self.kv_block_size = b.get("kv_block_size", self.a_block_size)
        self.a_per_tensor_scale = b.get("act_per_tensor_scale", False)
        self.w_ebit = b.get("wgt_ebit", 0)
        self.w_mbit = b.get("wgt_mbit", 0)
        self.w_sc_ebit = b.get("wgt_sc_ebit", 0)
        self.w_sc_mbit = b.get("wgt_sc_mbit", 8)
        self.w_block_size = b.get("wgt_block_size", 32)
        self.w_per_tensor_scale = b.get("wgt_per_tensor_scale", False)
        self.scale_allow_subnormal = b.get("scale_allow_subnormal", True)
        self.a_sc_bit = b.get("act_sc_bit", 8)
        self.w_sc_bit = b.get("wgt_sc_bit", 8)
        self.qk_mx_round = b.get("qk_mx_round", False)
        self.act_scale_use_ceil = b.get("act_scale_use_ceil", False)
        self.wgt_scale_use_ceil = b.get("wgt_scale_use_ceil", False)
        # HBQ L2 (src/ptq.py:71-77)
        self.wgt_l2_sc_bit = b.get("wgt_l2_sc_bit", 1)
        self.wgt_l2_block_size = b.get("wgt_l2_block_size", 4)
        self.wgt_l2_scheme = b.get("wgt_l2_scheme", "PoT")
        self.act_l2_sc_bit = b.get("act_l2_sc_bit", 1)
        self.act_l2_block_size = b.get("act_l2_block_size", 4)
        self.act_l2_scheme = b.get("act_l2_scheme", "PoT")

        # quantization points (src/ptq.py:80-91)
        self.quant_before_hadamard = q.get("quant_before_hadamard", False)
        self.quant_before_silu = q.get("quant_before_silu", False)
        self.quant_before_rms_norm = q.get("quant_before_rms_norm", False)
        self.quant_embedding_layer = q.get("quant_embedding_layer", False)
        self.quant_output_layer = q.get("quant_output_layer", False)
        self.quant_attn_wgt = q.get("quant_attn_wgt", False)
        self.quant_post_rope_qk = q.get("quant_post_rope_qk", False)
        self.quant_post_rope_q = q.get("quant_post_rope_q", False)
        self.quant_4b_kv = q.get("quant_4b_kv", False)
        self.quant_k_cache = q.get("quant_k_cache", False)
        self.quant_v_cache = q.get("quant_v_cache", False)
        self.quant_attn_wgt_use_quant_kernel = q.get("quant_attn_wgt_use_quant_kernel", True)

        # row-chunked weight quantization only for the models the reference names (src/ptq.py:93-100)
        cfg = getattr(model, "config", None)
        model_type = str(getattr(cfg, "model_type", "")).lower()
        model_name = str(getattr(cfg, "_name_or_path", "")).lower()
        self.large_model_memory_mode = model_type == "mixtral" or "llama-3.1-70b" in model_name
        self.chunk_static_wgt = self.large_model_memory_mode

        # low-precision accumulation (src/ptq.py:102-105)
        self.accumulation_type = acc.get("type", "fp32")
        self.accumulation_group_size = acc.get("group_size", 128)
        self.accumulation_quant_block_size = acc.get("quant_block_size", 16)

    # ---- config keys -> quantizers (src/ptq.py:107-257) ----
    def _build(self, qtype, side, use_round, kv=False):
        a = side == "act"
        ebit, mbit = (2, 1) if kv else ((self.a_ebit, self.a_mbit) if a else (self.w_ebit, self.w_mbit))
        sc_ebit = self.a_sc_ebit if a else self.w_sc_ebit
        sc_mbit = self.a_sc_mbit if a else self.w_sc_mbit
        block = self.kv_block_size if kv else (self.a_block_size if a else self.w_block_size)
        if qtype == "mxfp":
            return MXFPQuantizer(ebit=ebit, mbit=mbit, sc_ebit=sc_ebit, sc_mbit=sc_mbit, block_size=block,
                                 per_tensor_scale=self.a_per_tensor_scale if a else self.w_per_tensor_scale,
                                 scale_allow_subnormal=self.scale_allow_subnormal, use_round=use_round,
                                 use_ceil=self.act_scale_use_ceil if a else self.wgt_scale_use_ceil)
        if qtype == "mxint":
            return MXINTQuantizer(nbit=4 if kv else mbit, sc_ebit=sc_ebit, sc_mbit=sc_mbit, block_size=block,
                                  scale_allow_subnormal=self.scale_allow_subnormal)
        if qtype == "mxex" and not kv:
            return MXExQuantizer(sc_bit=self.a_sc_bit if a else self.w_sc_bit,
                                 l2_sc_bit=self.act_l2_sc_bit if a else self.wgt_l2_sc_bit, mbit=mbit,
                                 block_size=block,
                                 l2_block_size=self.act_l2_block_size if a else self.wgt_l2_block_size)
        if qtype == "vsq" and not kv:
            return VSQQuantizer(nbit=mbit, block_size=block, sc_mbit=sc_mbit)
        if qtype == "hbq":
            # the KV quantizer uses the activation L2 settings (src/ptq.py:242-253);
            # HBQ never receives use_round / use_ceil / per_tensor_scale
            return HBQQuantizer(ebit=ebit, mbit=mbit, sc_ebit=sc_ebit, sc_mbit=sc_mbit, block_size=block,
                                scale_allow_subnormal=self.scale_allow_subnormal,
                                l2_block_size=self.act_l2_block_size if a else self.wgt_l2_block_size,
                                l2_sc_bit=self.act_l2_sc_bit if a else self.wgt_l2_sc_bit,
                                l2_scheme=self.act_l2_scheme if a else self.wgt_l2_scheme,
                                # map_4b_kv_quantizer leaves the constructor default (src/ptq.py:242-253)
                                use_quant_kernel=True if kv else not self.large_model_memory_mode)
        if qtype == "none":
            return _QBase()
        what = "weight" if side == "wgt" else "activation"
        raise AssertionError(f"Invalid {what} quantizer type: {qtype}")

    def map_wgt_quantizer(self, use_round=False):
        return self._build(self.wqtype, "wgt", use_round)

    def map_act_quantizer(self, use_round=False, use_quant_kernel=True):
        # use_quant_kernel is accepted and not used, as in the reference (src/ptq.py:162,209)
        return self._build(self.xqtype, "act", use_round)

    def map_4b_kv_quantizer(self, use_round=False):
        """4-bit (E2M1) KV-cache quantizer with the activation quantizer's scales (src/ptq.py:216-257)."""
        return self._build(self.xqtype, "act", use_round, kv=True)

    # ---- injection into a model (src/ptq.py:259-336) ----
    def q_attn(self, module):
        module.quant_attn_wgt = self.quant_attn_wgt
        module.quant_post_rope_q = self.quant_post_rope_q
        module.quant_k_cache = self.quant_k_cache
        module.quant_v_cache = self.quant_v_cache
        r = self.qk_mx_round
        module.kv_quantizer = self.map_4b_kv_quantizer(use_round=r) if self.quant_4b_kv \
            else self.map_act_quantizer(use_round=r)
        module.attn_wgt_quantizer = self.map_act_quantizer(
            use_round=r, use_quant_kernel=self.quant_attn_wgt_use_quant_kernel) if self.quant_attn_wgt else None
        # q and k take the rounding MX scale when qk_mx_round is set; v and o do not
        for proj, rr in ((module.q_proj, r), (module.k_proj, r), (module.v_proj, False), (module.o_proj, False)):
            proj.wq = self.map_wgt_quantizer(use_round=rr)
            proj.aq = self.map_act_quantizer(use_round=rr)
        if self.quant_before_rms_norm:
            module.o_proj.yq = self.map_act_quantizer()

    def q_mlp(self, module, name=None, scales=None):
        for proj in (module.up_proj, module.gate_proj, module.down_proj):
            proj.wq = self.map_wgt_quantizer()
            proj.aq = self.map_act_quantizer()
        if self.quant_before_hadamard:
            module.up_proj.yq = self.map_act_quantizer()
            module.quantizer_after_act_fn = self.map_act_quantizer(None)
        if self.quant_before_silu:
            module.gate_proj.yq = self.map_act_quantizer()
        if self.quant_before_rms_norm:
            module.down_proj.yq = self.map_act_quantizer()

    def _decoder_layers(self):
        if self.model is None:
            return []
        return [m for _, m in self.model.named_modules() if hasattr(m, "self_attn") and hasattr(m, "mlp")]

    @torch.no_grad()
    def inject_quantizers(self, act_scales=None):
        for layer in self._decoder_layers():
            self.q_attn(layer.self_attn)
            self.q_mlp(layer.mlp)

    @torch.no_grad()
    def static_quant_linear_weight(self, linear, chunk_rows=None):
        """Quantize `linear.weight` in place with `linear.wq` (src/ptq.py:338-358): whole
        matrix, or row chunks of HBQ_WGT_CHUNK_ROWS rows in large-model mode."""
        weight = linear.weight
        if chunk_rows is None:
            chunk_rows = int(os.environ.get("HBQ_WGT_CHUNK_ROWS", "512"))
        if not self.chunk_static_wgt or weight.device.type != "cuda" or weight.ndim != 2 \
                or weight.shape[0] <= chunk_rows:
            weight.data = linear.wq(weight)
            return
        # blocks run along rows, so row chunks quantize exactly as the whole matrix
        for start in range(0, weight.shape[0], chunk_rows):
            end = min(start + chunk_rows, weight.shape[0])
            weight[start:end].copy_(linear.wq(weight[start:end].contiguous()))

    @torch.no_grad()
    def static_quant_wgt(self):
        for layer in self._decoder_layers():
            a, m = layer.self_attn, layer.mlp
            for lin in (a.q_proj, a.k_proj, a.v_proj, a.o_proj, m.gate_proj, m.up_proj, m.down_proj):
                self.static_quant_linear_weight(lin)
        if self.quant_output_layer and self.model is not None and hasattr(self.model, "lm_head"):
            head = self.model.lm_head
            self.static_quant_linear_weight(getattr(head, "proj", head))

    @torch.inference_mode()
    def replace_accum_kernel(self):
        """Install the low-precision-accumulation GEMM on every _QBaseLinear of the decoder
        layers (src/ptq.py:385-404)."""
        t = self.accumulation_type
        if t == "fp32":
            self.logger.info("Original accumulation kernel is used")
            return
        if t == "fp16":
            self.logger.info(f"FP16 accumulation kernel with group size {self.accumulation_group_size} is used")
            make = lambda: FP16AccumMatMul(group_size=self.accumulation_group_size)
        elif t == "fp16_quant":
            self.logger.info(f"FP16 accumulation kernel with MXINT8 psum quantization, group size "
                             f"{self.accumulation_group_size}, quant block size "
                             f"{self.accumulation_quant_block_size} is used")
            make = lambda: FP16AccumMatMul(group_size=self.accumulation_group_size,
                                           quant_block_size=self.accumulation_quant_block_size)
        else:
            raise ValueError(f"Invalid accumulation type: {t}")
        for layer in self._decoder_layers():
            for _, mod in layer.named_modules():
                if isinstance(mod, _QBaseLinear):
                    mod.ops = make()
