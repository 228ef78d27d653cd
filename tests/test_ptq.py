"""Config-key -> quantizer mapping, accumulation-kernel replacement and the
quantized linear layer (the callers of the hot path: src/ptq.py:107-404,
src/module.py:20-67).  The config dicts below hold the values of the
reference's config/*.yaml files for the formats in use."""
import logging

import pytest
import torch
import torch.nn as nn

from hbq_amd.module import _QBaseLinear
from hbq_amd.ops import FP16AccumMatMul
from hbq_amd.ptq import PTQ
from hbq_amd.quantizer import HBQQuantizer, MXFPQuantizer, _QBase

HBQ_BLOCK = dict(act_ebit=2, act_mbit=2, act_block_size=128, act_sc_ebit=5, act_sc_mbit=3,
                 wgt_ebit=2, wgt_mbit=1, wgt_block_size=128, wgt_sc_ebit=5, wgt_sc_mbit=3,
                 wgt_l2_sc_bit=2, wgt_l2_block_size=8, wgt_l2_scheme="Mix",
                 act_l2_sc_bit=2, act_l2_block_size=8, act_l2_scheme="SIG-1",
                 wgt_per_tensor_scale=False, act_per_tensor_scale=False,
                 scale_allow_subnormal=False, qk_mx_round=False)


def hbq_cfg(l2b=8, acc=None, kv=False):
    b = dict(HBQ_BLOCK, wgt_l2_block_size=l2b, act_l2_block_size=l2b)
    q = dict(xqtype="hbq", wqtype="hbq")
    if kv:
        q.update(quant_post_rope_q=True, quant_k_cache=True, quant_v_cache=True, quant_4b_kv=True,
                 quant_attn_wgt=True)
    return {"quantization": q, "block_quant": b, "accumulation": acc or {"type": "fp32"}}


def mx_cfg(mbit, block, sc_mbit, qk_round):
    b = dict(act_ebit=2, act_mbit=mbit, act_block_size=block, act_sc_ebit=5, act_sc_mbit=sc_mbit,
             wgt_ebit=2, wgt_mbit=mbit, wgt_block_size=block, wgt_sc_ebit=5, wgt_sc_mbit=sc_mbit,
             scale_allow_subnormal=False, qk_mx_round=qk_round)
    return {"quantization": {"xqtype": "mxfp", "wqtype": "mxfp"}, "block_quant": b,
            "accumulation": {"type": "fp16_quant", "group_size": 128, "quant_block_size": 32}}


class Attn(nn.Module):
    def __init__(self, d, kv):
        super().__init__()
        self.q_proj, self.k_proj = _QBaseLinear(d, d, bias=False), _QBaseLinear(d, kv, bias=False)
        self.v_proj, self.o_proj = _QBaseLinear(d, kv, bias=False), _QBaseLinear(d, d, bias=False)


class Mlp(nn.Module):
    def __init__(self, d, f):
        super().__init__()
        self.gate_proj, self.up_proj = _QBaseLinear(d, f, bias=False), _QBaseLinear(d, f, bias=False)
        self.down_proj = _QBaseLinear(f, d, bias=False)


class Layer(nn.Module):
    def __init__(self, d=256, kv=128, f=512):
        super().__init__()
        self.self_attn, self.mlp = Attn(d, kv), Mlp(d, f)


class Model(nn.Module):
    def __init__(self, n=2):
        super().__init__()
        self.layers = nn.ModuleList([Layer() for _ in range(n)])


def test_hbq_a_mapping():
    p = PTQ(hbq_cfg(), Model(), None, logging.getLogger("t"))
    a, w = p.map_act_quantizer(), p.map_wgt_quantizer()
    assert isinstance(a, HBQQuantizer) and isinstance(w, HBQQuantizer)
    assert (a.block_size, a.ebit, a.mbit, a.sc_ebit, a.sc_mbit) == (128, 2, 2, 5, 3)
    assert (a.l2_block_size, a.l2_sc_bit, a.l2_scheme) == (8, 2, "SIG-1")
    assert (w.mbit, w.l2_block_size, w.l2_sc_bit, w.l2_scheme) == (1, 8, 2, "Mix")
    assert a.scale_allow_subnormal is False and a.use_ceil is False and a.per_tensor_scale is False
    e = PTQ(hbq_cfg(l2b=32)).map_act_quantizer()
    assert e.l2_block_size == 32


def test_defaults_when_keys_absent():
    p = PTQ({"quantization": {"xqtype": "hbq", "wqtype": "none"}})
    a = p.map_act_quantizer()
    # src/ptq.py:44-77 defaults
    assert (a.ebit, a.mbit, a.sc_ebit, a.sc_mbit, a.block_size) == (0, 0, 0, 8, 32)
    assert (a.l2_sc_bit, a.l2_block_size, a.l2_scheme, a.scale_allow_subnormal) == (1, 4, "PoT", True)
    assert type(p.map_wgt_quantizer()) is _QBase
    assert (p.accumulation_type, p.accumulation_group_size, p.accumulation_quant_block_size) == ("fp32", 128, 16)
    with pytest.raises(KeyError):
        PTQ({"quantization": {"xqtype": "hbq"}})


def test_kv4_and_attention_points():
    m = Model(1)
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    att = m.layers[0].self_attn
    kvq = att.kv_quantizer
    assert isinstance(kvq, HBQQuantizer)
    assert (kvq.ebit, kvq.mbit, kvq.block_size, kvq.l2_block_size, kvq.l2_scheme) == (2, 1, 128, 8, "SIG-1")
    assert isinstance(att.attn_wgt_quantizer, HBQQuantizer) and att.attn_wgt_quantizer.mbit == 2
    assert att.quant_post_rope_q and att.quant_k_cache and att.quant_v_cache
    p2 = PTQ(hbq_cfg(), Model(1))
    p2.inject_quantizers()
    assert p2.model.layers[0].self_attn.attn_wgt_quantizer is None
    assert p2.model.layers[0].self_attn.kv_quantizer.mbit == 2     # act precision without quant_4b_kv


def test_mx_qk_round_and_nvfp():
    m = Model(1)
    p = PTQ(mx_cfg(1, 32, 0, True), m)
    p.inject_quantizers()
    a = m.layers[0].self_attn
    assert a.q_proj.aq.use_round and a.k_proj.wq.use_round
    assert not a.v_proj.aq.use_round and not a.o_proj.wq.use_round
    assert not m.layers[0].mlp.down_proj.aq.use_round
    nv = PTQ(mx_cfg(1, 16, 3, False)).map_wgt_quantizer()
    assert isinstance(nv, MXFPQuantizer) and (nv.block_size, nv.sc_ebit, nv.sc_mbit) == (16, 5, 3)


def test_replace_accum_kernel():
    m = Model(2)
    p = PTQ(mx_cfg(1, 32, 0, False), m)
    p.replace_accum_kernel()
    lins = [x for x in m.modules() if isinstance(x, _QBaseLinear)]
    assert len(lins) == 14
    assert all(isinstance(x.ops, FP16AccumMatMul) and x.ops.group_size == 128 and x.ops.quant_block_size == 32
               for x in lins)
    m2 = Model(1)
    PTQ(hbq_cfg(acc={"type": "fp16"}), m2).replace_accum_kernel()
    assert all(x.ops.group_size == 128 and x.ops.quant_block_size is None
               for x in m2.modules() if isinstance(x, _QBaseLinear))
    m3 = Model(1)
    PTQ(hbq_cfg(), m3).replace_accum_kernel()
    assert all(x.ops is None for x in m3.modules() if isinstance(x, _QBaseLinear))
    with pytest.raises(ValueError, match="Invalid accumulation type"):
        PTQ(hbq_cfg(acc={"type": "bf16"}), Model(1)).replace_accum_kernel()


def test_invalid_quantizer_type():
    with pytest.raises(AssertionError, match="Invalid weight quantizer type"):
        PTQ({"quantization": {"xqtype": "hbq", "wqtype": "int4"}}).map_wgt_quantizer()
    with pytest.raises(AssertionError, match="Invalid activation quantizer type"):
        PTQ({"quantization": {"xqtype": "int4", "wqtype": "hbq"}}).map_act_quantizer()


def test_identity_linear_cpu():
    torch.manual_seed(0)
    lin = _QBaseLinear(16, 8)
    x = torch.randn(3, 16)
    assert torch.equal(lin(x), torch.nn.functional.linear(x, lin.weight, lin.bias))
    with torch.no_grad():
        lin.weight[0, 0] = float("inf")
    x[0, 0] = 0.0
    with pytest.raises(RuntimeError, match="Non-finite output"):
        lin(torch.ones(2, 16))
