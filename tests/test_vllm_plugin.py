"""The vLLM plugin (hbq_amd/vllm_plugin.py, the reference's vllm/src/hbq_vllm_quant.py):
config handling and layer selection on the CPU; the linear method, the chunked weight
quantization, AWQ and the K/V helpers on the GPU, bit for bit against direct calls of
the quantizers (which the oracle tests pin)."""
import copy
import json

import pytest
import torch

from hbq_amd import vllm_plugin as vp
from hbq_amd.quantizer import HBQQuantizer, MXFPQuantizer


def _hbq_config():
    cfg = vp.default_nvfp4_config()
    cfg["quantization"].update(xqtype="hbq", wqtype="hbq")
    cfg["block_quant"].update(act_block_size=128, act_mbit=2, wgt_block_size=128, act_l2_block_size=8,
                              wgt_l2_block_size=8)
    return cfg


@pytest.fixture()
def clean_active(monkeypatch):
    monkeypatch.setattr(vp, "_active", None)
    monkeypatch.delenv(vp.CONFIG_ENV, raising=False)
    vp._awq_cache.clear()
    yield
    vp._awq_cache.clear()


def test_default_config_is_nvfp4(clean_active):
    cfg = vp.active_quant_config()
    assert cfg == vp.default_nvfp4_config()
    b = cfg["block_quant"]
    assert (b["act_ebit"], b["act_mbit"], b["act_block_size"], b["act_sc_ebit"], b["act_sc_mbit"]) == (2, 1, 16, 5, 3)
    assert cfg["quantization"]["xqtype"] == cfg["quantization"]["wqtype"] == "mxfp"
    assert not any(v for k, v in cfg["quantization"].items() if k.startswith("quant_"))


def test_active_config_travels_through_the_environment(clean_active, monkeypatch):
    cfg = _hbq_config()
    vp.set_active_quant_config(cfg)
    assert vp.active_quant_config() is cfg
    monkeypatch.setattr(vp, "_active", None)      # a worker process: only the environment
    assert vp.active_quant_config() == json.loads(json.dumps(cfg))


def test_build_quantizer_maps_the_keys():
    cfg = _hbq_config()
    cfg["block_quant"]["act_scale_use_ceil"] = True
    a = vp.build_quantizer(cfg, "act")
    assert isinstance(a, HBQQuantizer)
    assert (a.block_size, a.ebit, a.mbit, a.l2_block_size, a.l2_scheme) == (128, 2, 2, 8, "SIG-1")
    assert a.use_ceil and not a._fused                       # eager element rounding, as the plugin
    w = vp.build_quantizer(cfg, "wgt")
    assert isinstance(w, HBQQuantizer) and w.l2_scheme == "Mix" and w.mbit == 1
    m = vp.build_quantizer(vp.default_nvfp4_config(), "act")
    assert type(m) is MXFPQuantizer and (m.block_size, m.sc_ebit, m.sc_mbit) == (16, 5, 3)
    k = vp.build_quantizer(_hbq_config(), "act", force_4bit=True)
    assert (k.ebit, k.mbit) == (2, 1)
    with pytest.raises(ValueError):
        vp.build_quantizer(cfg, "act", qtype="int")


def test_config_selects_linear_layers(clean_active):
    c = vp.HBQNVFP4Config(_hbq_config())
    assert c.get_name() == "hbq_nvfp4" and c.get_min_capability() == -1
    assert c.get_supported_act_dtypes() == [torch.float16, torch.bfloat16]
    assert vp.HBQNVFP4Config.override_quantization_method(None, "hbq_nvfp4") == "hbq_nvfp4"
    assert vp.HBQNVFP4Config.override_quantization_method(None, "awq") is None
    lin = torch.nn.Linear(128, 64, bias=False)
    assert isinstance(c.get_quant_method(lin, "model.layers.0.mlp.down_proj"), vp.HBQNVFP4LinearMethod)
    assert c.get_quant_method(lin, "lm_head") is None
    assert c.get_quant_method(torch.nn.LayerNorm(8), "model.norm") is None
    assert vp.HBQNVFP4Config.from_config({}).quant_config == vp.default_nvfp4_config()


@pytest.mark.parametrize("flag", ["quant_attn_wgt", "quant_output_layer"])
def test_config_rejects_unsupported_flags(flag):
    cfg = vp.default_nvfp4_config()
    cfg["quantization"][flag] = True
    with pytest.raises(NotImplementedError):
        vp.HBQNVFP4Config(cfg)
    cfg = vp.default_nvfp4_config()
    cfg["quantization"]["wqtype"] = "vsq"
    with pytest.raises(ValueError):
        vp.HBQNVFP4Config(cfg)


def test_sequence_spans_and_awq_targets():
    pos = torch.tensor([0, 1, 2, 0, 1, 5, 6, 7])
    assert vp.sequence_spans(pos, 8) == [(0, 3), (3, 5), (5, 8)]
    assert vp.sequence_spans(pos, 9) == [(0, 9)]               # positions that do not match: one sequence
    assert vp.sequence_spans(None, 4) == [(0, 4)]
    assert vp.awq_target("model.layers.3.self_attn.k_proj") == "model.layers.3.self_attn.qkv_proj"
    assert vp.awq_target("model.layers.3.mlp.up_proj") == "model.layers.3.mlp.gate_up_proj"
    assert vp.awq_target("model.layers.3.mlp.down_proj") == "model.layers.3.mlp.down_proj"


def _awq_file(tmp_path, k, n_qkv, n_gate, n_up):
    g = torch.Generator().manual_seed(3)
    raw = {"scale": [("input_layernorm", ["m.l.self_attn.q_proj", "m.l.self_attn.k_proj", "m.l.self_attn.v_proj"],
                      torch.rand(k, generator=g) + 0.5)],
           "clip": [("m.l.self_attn.v_proj", torch.full((n_qkv // 2, 1, 1), 0.01)),
                    ("m.l.mlp.gate_proj", torch.full((n_gate, 1, 1), 0.02)),
                    ("m.l.mlp.up_proj", torch.full((n_up, 1, 1), 0.03))]}
    path = tmp_path / "awq.pt"
    torch.save(raw, path)
    return str(path), raw


def test_awq_metadata_and_clips(clean_active, tmp_path):
    path, raw = _awq_file(tmp_path, 64, 32, 16, 16)
    cfg = vp.default_nvfp4_config()
    cfg["awq"] = {"enable": True, "load_path": path}
    meta = vp.awq_metadata(cfg)
    assert torch.equal(meta["scale"]["m.l.self_attn.qkv_proj"], raw["scale"][0][2])
    lin = torch.nn.Linear(64, 32, bias=False)
    with torch.no_grad():
        lin.weight.fill_(1.0)
    vp.apply_awq_clip(lin, "m.l.self_attn.qkv_proj", cfg)   # only the v rows (the last 16) are clipped
    assert torch.all(lin.weight[:16] == 1.0) and torch.all(lin.weight[16:] == 0.01)
    gu = torch.nn.Linear(64, 32, bias=False)
    with torch.no_grad():
        gu.weight.fill_(-1.0)
    vp.apply_awq_clip(gu, "m.l.mlp.gate_up_proj", cfg)
    assert torch.all(gu.weight[:16] == -0.02) and torch.all(gu.weight[16:] == -0.03)
    cfg["awq"] = {"enable": True}
    vp._awq_cache.clear()
    with pytest.raises(ValueError):
        vp.awq_metadata(cfg)


@pytest.mark.gpu
@pytest.mark.parametrize("kind", ["nvfp4", "hbq"])
def test_linear_method_equals_direct_quantizers(gpu, clean_active, kind):
    """process_weights_after_loading gives wgt_q.q(W) (chunked or not) and apply gives
    linear(act_q.q(x), Wq, bias), bit for bit."""
    cfg = vp.default_nvfp4_config() if kind == "nvfp4" else _hbq_config()
    g = torch.Generator(device=gpu).manual_seed(11)
    lin = torch.nn.Linear(512, 384, bias=True).to(gpu).half()
    with torch.no_grad():
        lin.weight.copy_(torch.randn(384, 512, device=gpu, generator=g) * 0.05)
    w0 = lin.weight.detach().clone()
    cfg["block_quant"]["wgt_quant_chunk_rows"] = 100                 # ragged chunks of rows
    m = vp.HBQNVFP4Config(cfg).get_quant_method(lin, "model.layers.0.self_attn.o_proj")
    m.process_weights_after_loading(lin)
    wq = vp.build_quantizer(cfg, "wgt").q(w0)
    assert torch.equal(lin.weight.view(torch.int16), wq.view(torch.int16))
    assert lin.hbq_weight_quantized
    m.process_weights_after_loading(lin)                              # once only
    assert torch.equal(lin.weight.view(torch.int16), wq.view(torch.int16))
    x = torch.randn(7, 3, 512, device=gpu, generator=g).half()
    y = m.apply(lin, x, lin.bias)
    ref = torch.nn.functional.linear(vp.build_quantizer(cfg, "act").q(x), wq, lin.bias)
    assert torch.equal(y.view(torch.int16), ref.view(torch.int16))


@pytest.mark.gpu
def test_linear_method_with_awq(gpu, clean_active, tmp_path):
    path, raw = _awq_file(tmp_path, 512, 96, 16, 16)
    cfg = vp.default_nvfp4_config()
    cfg["awq"] = {"enable": True, "load_path": path}
    g = torch.Generator(device=gpu).manual_seed(12)
    lin = torch.nn.Linear(512, 96, bias=False).to(gpu).half()
    with torch.no_grad():
        lin.weight.copy_(torch.randn(96, 512, device=gpu, generator=g) * 0.05)
    w0 = lin.weight.detach().clone()
    m = vp.HBQNVFP4LinearMethod(cfg, "m.l.self_attn.qkv_proj")
    m.process_weights_after_loading(lin)
    s = raw["scale"][0][2].to(gpu).half()
    ws = w0 * s.view(1, -1)
    ws[-48:] = torch.clamp(ws[-48:], -0.01, 0.01)
    assert torch.equal(lin.weight.view(torch.int16), vp.build_quantizer(cfg, "wgt").q(ws).view(torch.int16))
    x = torch.randn(5, 512, device=gpu, generator=g).half()
    ref = torch.nn.functional.linear(vp.build_quantizer(cfg, "act").q(x / s.view(1, -1)), lin.weight)
    assert torch.equal(m.apply(lin, x).view(torch.int16), ref.view(torch.int16))
    cfg2 = copy.deepcopy(cfg)
    cfg2["awq"]["apply_act_scale"] = False
    ref2 = torch.nn.functional.linear(vp.build_quantizer(cfg, "act").q(x), lin.weight)
    assert torch.equal(vp.HBQNVFP4LinearMethod(cfg2, m.prefix).apply(lin, x).view(torch.int16),
                       ref2.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("four_bit", [False, True])
def test_kv_helpers_equal_direct_quantizers(gpu, clean_active, four_bit):
    cfg = _hbq_config()
    cfg["block_quant"].update(act_block_size=128, act_l2_block_size=16)
    cfg["quantization"]["quant_4b_kv"] = four_bit
    heads, kvh, d = 8, 2, 128
    g = torch.Generator(device=gpu).manual_seed(13)
    T = 300
    q = torch.randn(T, heads * d, device=gpu, generator=g).half()
    k = torch.randn(T, kvh * d, device=gpu, generator=g).half()
    v = torch.randn(T, kvh * d, device=gpu, generator=g).half()
    aq = vp.build_quantizer(cfg, "act")
    kq = vp.build_quantizer(cfg, "act", force_4bit=four_bit)
    assert torch.equal(vp.quantize_post_rope_q(q, heads, d, cfg).view(torch.int16),
                       aq.q(q.view(T, heads, d)).view(T, -1).view(torch.int16))
    assert torch.equal(vp.quantize_k_cache(k, kvh, d, cfg).view(torch.int16),
                       kq.q(k.view(T, kvh, d)).view(T, -1).view(torch.int16))
    # two packed sequences of 172 and 128 tokens: V is quantized along each one's tokens
    pos = torch.cat([torch.arange(172), torch.arange(128)]).to(gpu)
    got = vp.quantize_v_cache(v, kvh, d, pos, cfg)
    vv = v.view(T, kvh, d)
    ref = torch.cat([kq.q(vv[a:b].permute(1, 2, 0).contiguous()).permute(2, 0, 1)
                     for a, b in [(0, 172), (172, 300)]]).reshape(T, -1)
    assert torch.equal(got.view(torch.int16), ref.view(torch.int16))
