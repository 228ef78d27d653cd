"""GPU parity of the fused quantizer kernels against the reference goldens and the CPU oracle.

Every comparison is bit-exact (NaN positions compared as NaN)."""
import numpy as np
import pytest
import torch

from helpers import TDT, mismatches, synth, to_bits, to_torch

pytestmark = pytest.mark.gpu

MXCFG = {
    "mxfp4": dict(block_size=32, ebit=2, mbit=1, sc_ebit=5, sc_mbit=0),
    "mxfp4_round": dict(block_size=32, ebit=2, mbit=1, sc_ebit=5, sc_mbit=0, use_round=True),
    "mxfp8": dict(block_size=32, ebit=2, mbit=5, sc_ebit=5, sc_mbit=0),
    "mxfp8_round": dict(block_size=32, ebit=2, mbit=5, sc_ebit=5, sc_mbit=0, use_round=True),
    "nvfp4": dict(block_size=16, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3),
    "nvfp4_ceil": dict(block_size=16, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3, use_ceil=True),
}
HBQCFG = {
    "hbq_a_act": dict(ebit=2, mbit=2, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
    "hbq_a_wgt": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix"),
    "hbq_e_act": dict(ebit=2, mbit=2, l2_block_size=32, l2_sc_bit=2, l2_scheme="SIG-1"),
    "hbq_e_wgt": dict(ebit=2, mbit=1, l2_block_size=32, l2_sc_bit=2, l2_scheme="Mix"),
    "hbq_kv4": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
    "hbq_a_wgt_ceil": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix", use_ceil=True),
    "hbq_pot": dict(ebit=2, mbit=1, l2_block_size=4, l2_sc_bit=1, l2_scheme="PoT"),
    # no reference fixtures for these: checked against the oracle and the generic kernel
    "hbq_m3": dict(ebit=2, mbit=3, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
    "hbq_l16": dict(ebit=2, mbit=2, l2_block_size=16, l2_sc_bit=2, l2_scheme="FP-1"),
    # two-scheme (Mix) tables at 3 and 2 mantissa bits: the largest magnitude rows in LDS
    "hbq_m3_mix": dict(ebit=2, mbit=3, l2_block_size=16, l2_sc_bit=2, l2_scheme="Mix"),
    "hbq_m2_mix": dict(ebit=2, mbit=2, l2_block_size=32, l2_sc_bit=2, l2_scheme="Mix"),
}
NO_FIXTURES = ("hbq_m3", "hbq_l16", "hbq_m3_mix", "hbq_m2_mix")


def _table_and_generic(q, x):
    """q.quantize(x) on the table-driven kernel (a call that it declines fails instead of
    falling back) and on the generic kernel."""
    from hbq_amd import _lib
    old = _lib.lib().hbq_set_generic_only(2)
    try:
        fast = q.quantize(x)
        _lib.lib().hbq_set_generic_only(1)
        gen = q.quantize(x)
    finally:
        _lib.lib().hbq_set_generic_only(old)
    return fast, gen


def _mx(kw, **extra):
    from hbq_amd.quantizer import MXFPQuantizer
    return MXFPQuantizer(scale_allow_subnormal=False, **kw, **extra)


def _hbq(kw, **extra):
    from hbq_amd.quantizer import HBQQuantizer
    return HBQQuantizer(block_size=128, sc_ebit=5, sc_mbit=3, scale_allow_subnormal=False, **kw, **extra)


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("em", [(2, 1), (2, 2), (2, 5)])
def test_element_quantizer_exhaustive(gpu, golden_elem, golden_compiled, dt, em):
    """make_fp_quant (eager) and GLOBAL_FP_QUANT_CACHE's compiled quantizer over all 65,536
    bit patterns equal the reference's tables (src/quantizer.py:38-63,187-257)."""
    from hbq_amd.quantizer import FPQuantConfig, GLOBAL_FP_QUANT_CACHE, make_fp_quant
    print(f"elem dt={dt} E{em[0]}M{em[1]}", flush=True)
    allb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    x = to_torch(allb, dt).to(gpu)
    key = f"elem_{dt}_e{em[0]}m{em[1]}"
    assert mismatches(to_bits(make_fp_quant(*em)(x)), golden_elem[key], dt) == 0
    fused = GLOBAL_FP_QUANT_CACHE.get(FPQuantConfig(ebit=em[0], mbit=em[1]))
    assert mismatches(to_bits(fused(x)), golden_compiled[key], dt) == 0


@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("use_ceil", [False, True])
@pytest.mark.parametrize("clip", [False, True])
def test_scale_quantizer_vs_oracle(gpu, oracle, dt, use_ceil, clip):
    """fp_quant / quant_scale to E5M3 against the oracle: every 16-bit pattern, or a wide fp32 sample."""
    from hbq_amd.quantizer import HBQQuantizer, fp_quant
    print(f"scale dt={dt} ceil={use_ceil} clip={clip}", flush=True)
    if dt == "f32":
        g = torch.Generator().manual_seed(5)
        x = (torch.rand(1 << 20, generator=g) * 60 - 30).exp2() * torch.sign(torch.randn(1 << 20, generator=g))
        xb = x.numpy()
    else:
        xb = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    xt = to_torch(xb, dt).to(gpu)
    if clip:
        y = HBQQuantizer(use_ceil=use_ceil).quant_scale(xt)
        lo, hi = 2.0 ** -14, 61440.0
        xc = to_torch(xb, dt).float().clamp(lo, hi).to(TDT[dt])
        ref = oracle.fp_quant(to_bits(xc), dt, 5, 3, allow_subnormal=False, use_ceil=use_ceil)
    else:
        y = fp_quant(xt, 5, 3, allow_subnormal=False, use_ceil=use_ceil)
        ref = oracle.fp_quant(xb, dt, 5, 3, allow_subnormal=False, use_ceil=use_ceil)
    assert mismatches(to_bits(y), ref, dt) == 0


@pytest.mark.parametrize("name", list(MXCFG))
def test_mxfp_golden(gpu, golden_mxfp, name):
    print(f"mxfp golden {name}", flush=True)
    q = _mx(MXCFG[name])
    x = to_torch(golden_mxfp["x_f16"], "f16").to(gpu)
    assert mismatches(to_bits(q.q(x)), golden_mxfp[f"{name}_f16"], "f16") == 0
    blocks = q.reshape(x)[0]
    s = q.get_shared_scale(blocks).squeeze(-1)
    assert mismatches(to_bits(s), golden_mxfp[f"{name}_f16_scale"], "f16") == 0
    x32 = torch.from_numpy(golden_mxfp["x_f32"]).to(gpu)
    assert mismatches(to_bits(q.q(x32)), golden_mxfp[f"{name}_f32"], "f32") == 0


@pytest.mark.parametrize("name", ["mxfp4", "nvfp4"])
def test_mxfp_golden_ragged(gpu, golden_mxfp, name):
    print(f"mxfp ragged {name}", flush=True)
    x = to_torch(golden_mxfp["x_ragged_f16"], "f16").to(gpu)
    assert mismatches(to_bits(_mx(MXCFG[name]).q(x)), golden_mxfp[f"{name}_ragged_f16"], "f16") == 0


def test_mxfp_bf16_raises(gpu):
    """The reference's get_shared_scale rejects bf16 (src/quantizer.py:482-487)."""
    with pytest.raises(NotImplementedError):
        _mx(MXCFG["mxfp4"]).q(torch.zeros(4, 32, dtype=torch.bfloat16, device=gpu))


@pytest.mark.parametrize("name", [n for n in HBQCFG if n not in NO_FIXTURES])
@pytest.mark.parametrize("inp", ["f16", "f16w", "bf16"])
@pytest.mark.parametrize("uqk", [False, True])
def test_hbq_golden(gpu, golden_hbq, golden_extra, golden_compiled, name, inp, uqk):
    """HBQQuantizer.q against the reference's outputs: use_quant_kernel=False (the eager element
    quantizer) and True (the compiled one, the default PTQ builds)."""
    key = f"{name}_{inp}"
    fx = golden_compiled if uqk else (golden_hbq if key in golden_hbq.files else golden_extra)
    print(f"hbq golden {key} use_quant_kernel={uqk}", flush=True)
    dt = "bf16" if inp == "bf16" else "f16"
    q = _hbq(HBQCFG[name], keep_l2_scale=True, use_quant_kernel=uqk)
    x = to_torch(golden_hbq[f"x_{inp}"], dt).to(gpu)
    y = q.q(x)
    assert mismatches(to_bits(y), fx[key], dt) == 0
    assert mismatches(to_bits(q.shared_scale), fx[key + "_l1"], dt) == 0
    assert np.array_equal(q.l2_scale.cpu().numpy(), fx[key + "_l2idx"].astype(np.int64))
    assert np.array_equal(q.blk_l2_scheme.cpu().numpy(), fx[key + "_scheme"].astype(np.int64))
    if not uqk:
        assert mismatches(to_bits(q.real_l2_scale), fx[key + "_l2val"], dt) == 0


@pytest.mark.parametrize("name", ["mxfp4", "mxfp8", "nvfp4"])
def test_mxfp_compiled_golden(gpu, golden_mxfp, golden_compiled, name):
    """MXFPQuantizer(activate_dynamo=True): the compiled element quantizer inside MXFP q."""
    q = _mx(MXCFG[name], activate_dynamo=True)
    x = to_torch(golden_mxfp["x_f16"], "f16").to(gpu)
    assert mismatches(to_bits(q.q(x)), golden_compiled[f"{name}_f16"], "f16") == 0
    x32 = torch.from_numpy(golden_mxfp["x_f32"]).to(gpu)
    assert mismatches(to_bits(q.q(x32)), golden_compiled[f"{name}_f32"], "f32") == 0


@pytest.mark.parametrize("name", ["nvfp4", "mxfp4"])
def test_mxfp_per_tensor_scale_golden(gpu, golden_extra, name):
    """per_tensor_scale=True (src/quantizer.py:516-524,535-536) against the reference's outputs,
    an all-zero tensor (tensor scale 1) included."""
    q = _mx(MXCFG[name], per_tensor_scale=True)
    for key, ref in (("x_f16", f"{name}_pts_f16"), ("x_f32", f"{name}_pts_f32"),
                     ("x_zero_f16", f"{name}_pts_zero_f16")):
        dt = "f32" if key == "x_f32" else "f16"
        x = (torch.from_numpy(golden_extra[key]) if dt == "f32" else to_torch(golden_extra[key], dt)).to(gpu)
        assert mismatches(to_bits(q.q(x)), golden_extra[ref], dt) == 0, key


def test_hbq_golden_ragged(gpu, golden_hbq):
    x = to_torch(golden_hbq["x_ragged_f16"], "f16").to(gpu)
    y = _hbq(HBQCFG["hbq_a_act"], use_quant_kernel=False).q(x)
    assert mismatches(to_bits(y), golden_hbq["hbq_a_act_ragged_f16"], "f16") == 0


def _edge_rows(x):
    """Overwrite a few rows with zeros, +-inf, NaN, huge and subnormal values, negative zeros,
    and blocks whose small elements give u = R(t / l2) = 0 (the output is +0 whatever the sign)."""
    x = x.clone()
    x[0] = 0
    x[1, ::7] = float("inf")
    x[2, 5] = float("nan")
    x[3, 3::11] = -float("inf")
    x[4] = x[4] * 1e-6
    x[5] = x[5].sign() * 60000
    x[6, ::2] = -0.0
    tiny, big = (6e-8, 6e4) if x.dtype == torch.float16 else (1e-38, 1e5)
    x[7] = x[7].sign() * tiny
    x[7, ::128] = big
    return x


@pytest.mark.parametrize("name", list(HBQCFG))
@pytest.mark.parametrize("dt", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("uqk", [True, False])
def test_hbq_vs_oracle(gpu, oracle, name, dt, uqk):
    """HBQ on a 256 x 4096 mixture with edge rows, all dtypes, both element roundings, against the oracle."""
    print(f"hbq oracle {name} {dt} use_quant_kernel={uqk}", flush=True)
    x = _edge_rows(synth(256, 4096, 11, dt))
    q = _hbq(HBQCFG[name], keep_l2_scale=True, use_quant_kernel=uqk)
    y = q.q(x.to(gpu))
    ref = oracle.hbq_qdq(to_bits(x), dt, block_size=128, use_quant_kernel=uqk, **HBQCFG[name])
    assert mismatches(to_bits(y), ref["y"], dt) == 0
    assert mismatches(to_bits(q.shared_scale), ref["l1"], dt) == 0
    assert np.array_equal(q.l2_scale.cpu().numpy(), ref["l2idx"].astype(np.int64))
    assert np.array_equal(q.blk_l2_scheme.cpu().numpy(), ref["scheme"].astype(np.int64))


@pytest.mark.parametrize("name", list(MXCFG))
@pytest.mark.parametrize("dt", ["f16", "f32"])
@pytest.mark.parametrize("dyn", [False, True])
def test_mxfp_vs_oracle(gpu, oracle, name, dt, dyn):
    print(f"mxfp oracle {name} {dt} activate_dynamo={dyn}", flush=True)
    x = _edge_rows(synth(256, 4096, 12, dt))
    q = _mx(MXCFG[name], activate_dynamo=dyn)
    out = q.quantize(x.to(gpu))
    y, s = oracle.mxfp_qdq(to_bits(x), dt, compiled=dyn, **MXCFG[name])
    assert mismatches(to_bits(out.y), y, dt) == 0
    assert mismatches(to_bits(out.scales), s, dt) == 0


@pytest.mark.parametrize("block,l2b", [(16, 4), (32, 8), (64, 16), (256, 32), (1024, 32)])
@pytest.mark.parametrize("scheme", ["Mix", "SIG-1", "INT"])
def test_hbq_block_shapes_vs_oracle(gpu, oracle, block, l2b, scheme):
    """Other block / L2 block sizes and schemes, with a ragged last dimension."""
    print(f"hbq shapes B={block} l2b={l2b} {scheme}", flush=True)
    x = synth(64, 3 * block + 48, 13, "f16")
    kw = dict(ebit=2, mbit=1, l2_block_size=l2b, l2_sc_bit=2, l2_scheme=scheme)
    from hbq_amd.quantizer import HBQQuantizer
    y = HBQQuantizer(block_size=block, sc_ebit=5, sc_mbit=3, **kw).q(x.to(gpu))
    ref = oracle.hbq_qdq(to_bits(x), "f16", block_size=block, **kw)
    assert mismatches(to_bits(y), ref["y"], "f16") == 0


def test_hbq_config1_full(gpu, oracle):
    """Config 1 tensor: bf16 4096 x 4096 ~ N(0,1) with a 0.5% Laplace(20) tail, HBQ-A/E act and wgt."""
    x = synth(4096, 4096, 1001, "bf16", outliers=0)
    xg = x.to(gpu)
    for name in ("hbq_a_act", "hbq_a_wgt", "hbq_e_act", "hbq_e_wgt"):
        print(f"config1 {name}", flush=True)
        y = _hbq(HBQCFG[name]).q(xg)
        ref = oracle.hbq_qdq(to_bits(x), "bf16", block_size=128, **HBQCFG[name])
        assert mismatches(to_bits(y), ref["y"], "bf16") == 0, name


def _decode(codes, mbit, n):
    """Element values of E2Mm codes (sign | exp field | mantissa)."""
    c = codes.astype(np.int64)
    if mbit == 1:
        c = np.stack([c & 0xF, c >> 4], axis=-1).reshape(c.shape[:-1] + (-1,))[..., :n]
    sign = np.where((c >> (mbit + 2)) & 1, -1.0, 1.0)
    ef = (c >> mbit) & 3
    mf = c & ((1 << mbit) - 1)
    mag = np.where(ef == 0, mf / 2.0 ** mbit, (1 + mf / 2.0 ** mbit) * 2.0 ** (ef - 1))
    return sign * mag


@pytest.mark.parametrize("name", ["hbq_a_act", "hbq_a_wgt", "hbq_e_wgt"])
def test_hbq_codes_decode(gpu, name):
    """Codes x L2 factor x L1 scale reproduce the dequantized output exactly."""
    x = synth(128, 1024, 14, "f16")
    q = _hbq(HBQCFG[name])
    out = q.quantize(x.to(gpu))
    mbit = HBQCFG[name]["mbit"]
    vals = _decode(out.codes.cpu().numpy(), mbit, 1024)
    tab = q.l2_table(dtype=torch.float32).numpy()
    l2b = HBQCFG[name]["l2_block_size"]
    l2 = tab[out.l2_index.cpu().numpy().astype(np.int64), out.scheme.cpu().numpy().astype(np.int64)[..., None]]
    l2e = np.repeat(l2.reshape(128, -1), l2b, axis=1)
    l1e = np.repeat(out.scales.float().cpu().numpy(), 128, axis=1)
    dq = torch.from_numpy(vals * l2e).half().float().mul(torch.from_numpy(l1e)).half()
    assert mismatches(to_bits(dq), to_bits(out.y), "f16") == 0


@pytest.mark.parametrize("name", ["mxfp4", "mxfp8", "nvfp4"])
def test_mxfp_codes_decode(gpu, name):
    x = synth(128, 1024, 15, "f16")
    q = _mx(MXCFG[name])
    out = q.quantize(x.to(gpu))
    B = MXCFG[name]["block_size"]
    vals = _decode(out.codes.cpu().numpy(), MXCFG[name]["mbit"], 1024)
    s = np.repeat(out.scales.float().cpu().numpy(), B, axis=1)
    dq = torch.from_numpy(vals * s).half()
    assert mismatches(to_bits(dq), to_bits(out.y), "f16") == 0


def test_hbq_3d_input(gpu, oracle):
    """Blocks run along the last dim of any-rank input; attributes keep the leading dims."""
    x = synth(6 * 32, 256, 16, "f16").view(6, 32, 256)
    q = _hbq(HBQCFG["hbq_kv4"], keep_l2_scale=True)
    y = q.q(x.to(gpu))
    assert y.shape == x.shape and q.shared_scale.shape == (6, 32, 2) and q.l2_scale.shape == (6, 32, 2, 16)
    ref = oracle.hbq_qdq(to_bits(x.view(-1, 256)), "f16", block_size=128, **HBQCFG["hbq_kv4"])
    assert mismatches(to_bits(y.view(-1, 256)), ref["y"], "f16") == 0


@pytest.mark.parametrize("name", ["hbq_a_act", "hbq_a_wgt", "hbq_e_act", "hbq_e_wgt", "hbq_kv4", "hbq_a_wgt_ceil",
                                  "hbq_m3", "hbq_l16", "hbq_m3_mix", "hbq_m2_mix"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("uqk", [True, False])
def test_hbq_table_kernel_equals_generic(gpu, name, dt, uqk):
    """The table-driven kernel and the generic kernel agree bit for bit, codes and scales included."""
    print(f"fast vs generic {name} {dt} use_quant_kernel={uqk}", flush=True)
    x = _edge_rows(synth(512, 4096, 17, dt)).to(gpu)
    q = _hbq(HBQCFG[name], use_quant_kernel=uqk)
    fast, gen = _table_and_generic(q, x)
    assert mismatches(to_bits(fast.y), to_bits(gen.y), dt) == 0
    ok = ~torch.isnan(fast.y)          # codes of NaN outputs are unspecified
    per_byte = ok if q.mbit != 1 else ok.view(ok.shape[0], -1, 2).all(-1)
    assert torch.equal(fast.codes[per_byte], gen.codes[per_byte])
    assert mismatches(to_bits(fast.scales), to_bits(gen.scales), dt) == 0
    assert torch.equal(fast.l2_index, gen.l2_index) and torch.equal(fast.scheme, gen.scheme)


MXFAST = dict(MXCFG, e2m2_pot=dict(block_size=32, ebit=2, mbit=2, sc_ebit=8, sc_mbit=0),
              e2m3_fp=dict(block_size=16, ebit=2, mbit=3, sc_ebit=5, sc_mbit=3),
              e2m5_fp=dict(block_size=32, ebit=2, mbit=5, sc_ebit=4, sc_mbit=3))


@pytest.mark.parametrize("name", list(MXFAST))
@pytest.mark.parametrize("dyn", [False, True])
def test_mxfp_table_kernel_equals_generic(gpu, name, dyn):
    """The table-driven MXFP / NVFP kernel (fp16, whole blocks) and the generic kernel agree
    bit for bit on outputs, codes and scales, edge rows (zeros, +-inf, NaN, huge, subnormal,
    quotients in the fp16 subnormal range) included."""
    print(f"mx fast vs generic {name} activate_dynamo={dyn}", flush=True)
    x = _edge_rows(synth(512, 4096, 18, "f16"))
    x[6] = x[6] * 1e-3            # blocks whose quotients reach the fp16 subnormal range
    x[7, ::3] = 0.0
    xg = x.to(gpu)
    q = _mx(MXFAST[name], activate_dynamo=dyn)
    fast, gen = _table_and_generic(q, xg)
    assert mismatches(to_bits(fast.y), to_bits(gen.y), "f16") == 0
    assert torch.equal(fast.codes, gen.codes)
    assert mismatches(to_bits(fast.scales), to_bits(gen.scales), "f16") == 0


@pytest.mark.parametrize("name", ["mxfp4", "mxfp8", "nvfp4"])
@pytest.mark.parametrize("shape", [(1, 32), (3, 96), (7, 208), (5, 1056), (33, 4064)])
def test_mxfp_table_kernel_partial_tiles(gpu, oracle, name, shape):
    """Shapes whose element count is not a multiple of a wave's 1024-element tile: the table
    kernel's partial last tile against the oracle."""
    rows, cols = shape
    if cols % MXCFG[name]["block_size"]:
        pytest.skip("ragged rows take the generic kernel")
    x = synth(rows, cols, 19, "f16", outliers=min(8, cols))
    out = _mx(MXCFG[name]).quantize(x.to(gpu))
    y, s = oracle.mxfp_qdq(to_bits(x), "f16", **MXCFG[name])
    assert mismatches(to_bits(out.y), y, "f16") == 0
    assert mismatches(to_bits(out.scales), s, "f16") == 0


@pytest.mark.parametrize("name", ["hbq_a_wgt", "hbq_e_wgt", "hbq_a_act"])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("rows", [1, 37, 129])
def test_hbq_table_kernel_partial_tiles(gpu, oracle, name, dt, rows):
    """Block counts that leave the last workgroup tile partial (32 blocks a tile for bf16,
    64 for fp16 one-scheme, 128 for the fp16 two-scheme kernel), on the table kernel only,
    against the oracle: outputs, L1 scales, L2 indices and schemes."""
    print(f"hbq partial tiles {name} {dt} rows={rows}", flush=True)
    x = synth(rows, 4096, 24 + rows, dt)
    q = _hbq(HBQCFG[name], keep_l2_scale=True)
    from hbq_amd import _lib
    old = _lib.lib().hbq_set_generic_only(2)
    try:
        y = q.q(x.to(gpu))
    finally:
        _lib.lib().hbq_set_generic_only(old)
    ref = oracle.hbq_qdq(to_bits(x), dt, block_size=128, **HBQCFG[name])
    assert mismatches(to_bits(y), ref["y"], dt) == 0
    assert mismatches(to_bits(q.shared_scale), ref["l1"], dt) == 0
    assert np.array_equal(q.l2_scale.cpu().numpy(), ref["l2idx"].astype(np.int64))
    assert np.array_equal(q.blk_l2_scheme.cpu().numpy(), ref["scheme"].astype(np.int64))


@pytest.mark.parametrize("name", ["hbq_a_act", "hbq_a_wgt", "hbq_kv4"])
def test_hbq_causal_zero_blocks(gpu, oracle, name):
    """Attention-weight-like input (row i zero past column i): waves whose eight blocks are all
    zero take the table kernel's zero path; everything equals the oracle and the generic kernel."""
    print(f"hbq causal zeros {name}", flush=True)
    T = 2048
    g = torch.Generator().manual_seed(23)
    x = torch.softmax(torch.randn(64, T, generator=g) * 3, dim=-1)
    rows = torch.arange(64)[:, None] * 32 + 7
    x = torch.where(torch.arange(T)[None, :] > rows, torch.zeros(()), x).half()
    q = _hbq(HBQCFG[name], keep_l2_scale=True)
    y = q.q(x.to(gpu))
    ref = oracle.hbq_qdq(to_bits(x), "f16", block_size=128, **HBQCFG[name])
    assert mismatches(to_bits(y), ref["y"], "f16") == 0
    assert mismatches(to_bits(q.shared_scale), ref["l1"], "f16") == 0
    assert np.array_equal(q.l2_scale.cpu().numpy(), ref["l2idx"].astype(np.int64))
    assert np.array_equal(q.blk_l2_scheme.cpu().numpy(), ref["scheme"].astype(np.int64))
    fast, gen = _table_and_generic(q, x.to(gpu))
    assert torch.equal(fast.codes, gen.codes)


def test_quantizers_beyond_int32_offsets(gpu):
    """Element offsets past 2^31 (the largest tensors a 288 GB device holds): rows at the
    start, across the 2^31-element boundary and at the end quantize exactly as the same
    rows alone, on the table kernels and the generic kernel (blocks are independent)."""
    from hbq_amd import _lib
    from hbq_amd.quantizer import HBQQuantizer, MXFPQuantizer
    cols = 4096
    b = (1 << 31) // cols
    rows = b + 64
    print(f"int64 offsets: {rows}x{cols} bf16", flush=True)
    g = torch.Generator(device=gpu).manual_seed(31)
    x = torch.randn(rows, cols, device=gpu, dtype=torch.bfloat16, generator=g)
    spans = [(0, 8), (b - 8, b + 8), (rows - 8, rows)]

    def same_rows(qz, x, y):
        for r0, r1 in spans:
            alone = qz.q(x[r0:r1].clone())
            assert torch.equal(y[r0:r1].view(torch.int16), alone.view(torch.int16)), (r0, r1)

    hbq = HBQQuantizer(block_size=128, **HBQCFG["hbq_a_act"])
    y = hbq.q(x)
    same_rows(hbq, x, y)
    old = _lib.lib().hbq_set_generic_only(1)
    try:
        y2 = hbq.q(x)
    finally:
        _lib.lib().hbq_set_generic_only(old)
    assert torch.equal(y.view(torch.int16), y2.view(torch.int16))
    del y, y2
    xh = x.half()
    del x
    mx = MXFPQuantizer(scale_allow_subnormal=False, **MXCFG["mxfp4"])
    same_rows(mx, xh, mx.q(xh))
