"""Packed HBQ wire format: code/scale decoding pinned by the reference's RTL MAC
vectors, the oracle's pack/unpack pinned by the oracle quantizer, and the HIP
pack/unpack kernels against both (bit for bit)."""
import os

import numpy as np
import pytest
import torch

from helpers import mismatches, synth, to_bits

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")

# (mbit, l2_block_size, l2_sc_bit, scheme): HBQ-A act / wgt, HBQ-E act / wgt, and others
CONFIGS = [(2, 8, 2, "SIG-1"), (1, 8, 2, "Mix"), (2, 32, 2, "SIG-1"), (1, 32, 2, "Mix"), (3, 16, 1, "PoT"),
           (1, 8, 0, "PoT"), (2, 4, 3, "FP-10"), (1, 16, 1, "FP-100")]


@pytest.fixture(scope="module")
def kat():
    return np.load(os.path.join(GOLDEN, "rtl_mac_kat.npz"))


@pytest.fixture(scope="module")
def PK():
    from oracle import packed
    return packed


def kat_cases(kat):
    return sorted(k[: -len("_scaled_psum")] for k in kat.files if k.endswith("_scaled_psum"))


def test_rtl_kat_code_decode(kat, PK):
    """Every block's fixed-point dot product of the MAC vectors equals the sum of the decoded
    codes (sign | exponent | mantissa, subnormal exponent field 0): E2M1 weights against
    E2M1..E2M5 activations, 30 vector sets, 4,160 blocks."""
    n = 0
    for case in kat_cases(kat):
        kind, a, b = case.split("_")
        Y, B = int(a[1:]), int(b[1:])
        act = PK.code_int(kat[case + "_act"], Y - 3).reshape(-1, B)
        wgt = PK.code_int(kat[case + "_wgt"], 1).reshape(-1, B)
        np.testing.assert_array_equal((act * wgt).sum(1), kat[case + "_psum"], err_msg=case)
        n += act.shape[0]
    assert n == 4160


def _scaled_ulps(kat, PK, case, scale_fn):
    kind, a, b = case.split("_")
    Y = int(a[1:])
    exact = kat[case + "_psum"] * 2.0 ** -((4 - 3) + (Y - 3)) * scale_fn(kat[case + "_scale_act"]) * \
        scale_fn(kat[case + "_scale_wgt"])
    h = exact.astype(np.float16)
    h[np.abs(h) < 2.0 ** -14] = 0            # the MAC's fp16 output flushes subnormals
    key = lambda u: np.where(u & 0x8000, -(u & 0x7FFF).astype(np.int64), (u & 0x7FFF).astype(np.int64))
    return np.abs(key(h.view(np.uint16)) - key(kat[case + "_scaled_psum"]))


def test_rtl_kat_scale_decode(kat, PK):
    """The E5M3 scale byte (nv, bias 15) and the 5-bit power-of-two scale (mx) decode so that
    psum * 2^-(fixed scale) * s_act * s_wgt rounds to the testbench's fp16 scaled psum: within
    1 ulp for > 99% of the blocks and 8 ulp for all (the testbench itself allows its golden
    model's differently rounded scale product, tb_WXAY.sv:263-273).  A bias off by one fails."""
    pot = lambda b: np.exp2(b.astype(np.float64) - 15)
    for bias_shift, expect_ok in ((0, True), (1, False)):
        d = []
        for case in kat_cases(kat):
            if case.startswith("nv"):
                fn = lambda b: PK.e5m3_value(b) * 2.0 ** -bias_shift
            else:
                fn = lambda b: pot(b) * 2.0 ** -bias_shift
            d.append(_scaled_ulps(kat, PK, case, fn))
        d = np.concatenate(d)
        ok = (d <= 1).mean() > 0.99 and d.max() <= 8
        assert ok == expect_ok, (bias_shift, (d <= 1).mean(), d.max())


def test_e5m3_byte_is_fp16_bits(PK):
    """Every E5M3 value's byte equals bits [14:7] of its fp16 pattern (low 7 bits zero)."""
    for b in range(0xF8):
        v = PK.e5m3_value(np.array([b]))[0]
        h = int(np.array([v], np.float16).view(np.uint16)[0])
        assert h & 0x7F == 0 and h >> 7 == b, b
        assert PK.e5m3_byte(np.array([v]))[0] == b
    assert PK.e5m3_byte(np.array([np.nan, np.inf, -1.0, -0.0, 1.0 + 2 ** -4, 70000.0])).tolist() == [0xFF] * 6


def test_bitstring_closed_form(PK):
    """LSB-first fields: two 5-bit codes 0b10101, 0b00011 -> bytes 0b01110101, 0b00000000."""
    out = PK._bitstring(np.array([[0b10101, 0b00011]]), 5, 2)
    assert out.tolist() == [[0b01110101, 0]]
    np.testing.assert_array_equal(PK._fields(out, 5, 2), [[0b10101, 0b00011]])


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cfg", CONFIGS)
def test_oracle_pack_unpack_roundtrip(oracle, PK, dt, cfg):
    """unpack(pack(codes, scales)) reproduces the oracle quantizer's output bit for bit,
    edge blocks included (all-zero, tiny negatives, an outlier channel)."""
    mbit, l2b, l2s, sch = cfg
    x = synth(6, 512, 91, dt)
    x[0, :128] = 0
    x[1, 130] = -1e-6
    xb = to_bits(x)
    res = oracle.hbq_qdq(xb, dt, 128, 2, mbit, 5, 3, l2b, l2s, sch)
    codes = PK.hbq_codes(xb, dt, res, 128, mbit, l2b, l2s, sch)
    p = PK.pack(codes, res["l1"], res["l2idx"], res["scheme"], dt, 128, mbit, l2b, l2s, sch)
    y = PK.unpack(p, 6, 512, dt, 128, mbit, l2b, l2s, sch)
    assert mismatches(y, res["y"], dt) == 0
    # a planted decode mistake (the l2 factor of candidate j+1) is caught
    if l2s:
        bad = dict(p)
        bad["l2"] = PK._bitstring((PK._fields(p["l2"], l2s, 512 // l2b) + 1) % (1 << l2s), l2s, p["l2"].shape[1])
        assert mismatches(PK.unpack(bad, 6, 512, dt, 128, mbit, l2b, l2s, sch), res["y"], dt) > 0


@pytest.mark.parametrize("cfg", CONFIGS)
def test_packed_strides_abi(PK, cfg):
    """hbq_hbq_packed_strides (host-only) agrees with the oracle's layout."""
    from hbq_amd.packed import packed_strides
    mbit, l2b, l2s, sch = cfg
    for cols in (128, 512, 4096, 14336):
        assert packed_strides(cols, 128, mbit, l2b, l2s, sch) == PK.strides(cols, 128, mbit, l2b, l2s, sch)
    with pytest.raises(ValueError):
        packed_strides(100, 128, mbit, l2b, l2s, sch)


# ---------------------------------------------------------------------------- GPU


def _gpu_codes_per_element(codes, mbit, cols):
    c = to_bits_u8(codes)
    if mbit == 1:
        c = np.stack([c & 0xF, c >> 4], axis=-1).reshape(c.shape[0], -1)[:, :cols]
    return c


def to_bits_u8(t):
    return t.detach().cpu().numpy().astype(np.uint8)


@pytest.mark.gpu
@pytest.mark.parametrize("generic", [False, True])
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("cfg", CONFIGS)
def test_gpu_pack_unpack(gpu, oracle, PK, cfg, dt, generic):
    """HIP pack of the HIP quantizer's outputs equals the oracle's packing of the same outputs;
    HIP unpack returns the quantizer's y bit for bit (NaN blocks as NaN), and decodes the
    oracle's bytes to the oracle's values."""
    from hbq_amd import _lib
    from hbq_amd.packed import pack, unpack
    from hbq_amd.quantizer import HBQQuantizer
    mbit, l2b, l2s, sch = cfg
    print(f"packed {cfg} {dt} generic={generic}", flush=True)
    x = synth(64, 1024, 92, dt)
    x[0, :128] = 0
    x[1, 130] = -1e-6
    x[2, 300] = float("inf")
    x[3, 700] = float("nan")
    x = x.to(gpu)
    q = HBQQuantizer(128, 2, mbit, 5, 3, l2b, l2s, sch)
    old = _lib.lib().hbq_set_generic_only(int(generic))
    try:
        ref = q.quantize(x)
        p = pack(q, x)
        y = unpack(p)
    finally:
        _lib.lib().hbq_set_generic_only(old)
    torch.cuda.synchronize()
    assert mismatches(to_bits(y), to_bits(ref.y), dt) == 0
    codes = _gpu_codes_per_element(ref.codes, mbit, 1024)
    po = PK.pack(codes, to_bits(ref.scales), to_bits_u8(ref.l2_index), to_bits_u8(ref.scheme), dt, 128, mbit, l2b,
                 l2s, sch)
    np.testing.assert_array_equal(to_bits_u8(p.codes), po["codes"])
    np.testing.assert_array_equal(to_bits_u8(p.l1), po["l1"])
    if l2s:
        np.testing.assert_array_equal(to_bits_u8(p.l2), po["l2"])
    if sch == "Mix":
        np.testing.assert_array_equal(to_bits_u8(p.scheme), po["scheme"])
    assert to_bits_u8(p.l1)[3, 5] == 0xFF                     # the NaN block
    yo = PK.unpack(po, 64, 1024, dt, 128, mbit, l2b, l2s, sch)
    assert mismatches(yo, to_bits(y), dt) == 0


@pytest.mark.gpu
def test_gpu_packed_full_size_roundtrip(gpu):
    """At the gate/up weight shape (14336 x 4096, HBQ-A wgt) unpack(pack(W)) == q(W); the
    packed form takes 0.540 B per element."""
    from hbq_amd.packed import pack
    from hbq_amd.quantizer import HBQQuantizer
    print("packed full size", flush=True)
    g = torch.Generator(device=gpu).manual_seed(5)
    W = (torch.randn(14336, 4096, device=gpu, generator=g) * 0.02).half()
    q = HBQQuantizer(128, 2, 1, 5, 3, 8, 2, "Mix")
    p = pack(q, W)
    y = q.q(W)
    assert torch.equal(p.unpack().view(torch.int16), y.view(torch.int16))
    assert abs(p.nbytes / W.numel() - (0.5 + 1 / 128 + 2 / 64 + 1 / 1024)) < 1e-6


@pytest.mark.gpu
@pytest.mark.parametrize("ops", ["fp32", "mxint8"])
def test_gpu_packed_weights_prefill(gpu, ops):
    """A prefill with packed weights (decoded before each GEMM) gives the same logits bit for
    bit as one with PTQ's in-place fake-quantized weights."""
    from hbq_amd.llama import LlamaConfig, LlamaForCausalLM
    from hbq_amd.module import _QBaseLinear
    from hbq_amd.ops import FP16AccumMatMul, FP32AccumMatMul
    from hbq_amd.packed import pack_linear_weights
    from hbq_amd.ptq import PTQ
    from test_ptq import hbq_cfg
    print(f"packed prefill {ops}", flush=True)
    tiny = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, vocab_size=1000)
    ids = torch.randint(0, 1000, (1, 64), device=gpu, generator=torch.Generator(device=gpu).manual_seed(3))
    outs = []
    for packed in (False, True):
        m = LlamaForCausalLM(tiny).random_init_(seed=9).half().to(gpu)
        p = PTQ(hbq_cfg(kv=True), m)
        p.inject_quantizers()
        for mod in m.modules():
            if isinstance(mod, _QBaseLinear) and mod is not m.lm_head:
                mod.ops = FP32AccumMatMul() if ops == "fp32" else FP16AccumMatMul(128, 32)
        if packed:
            assert pack_linear_weights(m) == 2 * 7
            assert m.layers[0].mlp.up_proj.weight.numel() == 0
        else:
            p.static_quant_wgt()
        with torch.no_grad():
            outs.append(m(ids))
            if packed:      # q/k/v decoded into one stacked scratch and run as one GEMM
                for layer in m.layers:
                    layer.self_attn.stack_qkv = True
                outs.append(m(ids))
    for o in outs[1:]:
        assert torch.equal(outs[0].view(torch.int16), o.view(torch.int16))


PACKED_GEMM_CASES = [("fp32", 0, 0), ("grouped", 128, 0), ("grouped", 32, 0), ("grouped", 16, 0),
                     ("mxint8", 128, 32), ("mxint8", 64, 16), ("mxint8", 256, 4), ("mxfp8", 128, 32),
                     ("mxfp8", 64, 8)]


@pytest.mark.gpu
@pytest.mark.parametrize("wcfg", [(8, 2, "Mix"), (32, 2, "Mix"), (16, 1, "FP-1"), (8, 0, "PoT")])
@pytest.mark.parametrize("case", PACKED_GEMM_CASES)
def test_gpu_packed_gemm_bit_identical(gpu, case, wcfg):
    """The GEMM that decodes the packed weight in registers gives the bits of the blockquant_ext
    GEMM on the unpacked weight, for 1..32 rows, every accumulation mode and HBQ-A / HBQ-E weights."""
    from hbq_amd import blockquant_ext as ext
    from hbq_amd.packed import pack, packed_gemm
    from hbq_amd.quantizer import HBQQuantizer
    mode, gk, gn = case
    l2b, l2s, sch = wcfg
    print(f"packed gemm {case} {wcfg}", flush=True)
    K, N = 1024, 416
    W = synth(N, K, 61, "f16", std=0.02).to(gpu)
    p = pack(HBQQuantizer(128, 2, 1, 5, 3, l2b, l2s, sch), W)
    Wq = p.unpack()
    for M in (1, 5, 16, 32):
        A = synth(M, K, 62 + M, "f16").to(gpu)
        ref = {"fp32": lambda: ext.gemm_fp32_accum_nk(A, Wq),
               "grouped": lambda: ext.gemm_fp16_grouped_accum_nk(A, Wq, gk),
               "mxint8": lambda: ext.gemm_blockquant_mxint8_nk(A, Wq, gk, gn),
               "mxfp8": lambda: ext.gemm_blockquant_mxfp8_nk(A, Wq, gk, gn)}[mode]()
        got = packed_gemm(A, p, mode, gk, gn)
        assert torch.isfinite(ref.float()).all()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), (M, case, wcfg)


@pytest.mark.gpu
def test_gpu_packed_gemm_decode_step(gpu):
    """A decode step (4 tokens) through a model with packed weights: the linears take the in-register
    decode path and the logits equal those of the fake-quantized weights."""
    from hbq_amd.llama import LlamaConfig, LlamaForCausalLM
    from hbq_amd.module import _QBaseLinear
    from hbq_amd.ops import FP16AccumMatMul
    from hbq_amd import packed as PKD
    from hbq_amd.packed import pack_linear_weights
    from hbq_amd.ptq import PTQ
    from test_ptq import hbq_cfg
    print("packed decode step", flush=True)
    tiny = LlamaConfig(hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
                       num_key_value_heads=2, vocab_size=1000)
    ids = torch.randint(0, 1000, (1, 4), device=gpu, generator=torch.Generator(device=gpu).manual_seed(5))
    outs = []
    calls = []
    orig = PKD.packed_gemm
    for packed in (False, True):
        m = LlamaForCausalLM(tiny).random_init_(seed=10).half().to(gpu)
        p = PTQ(hbq_cfg(kv=True), m)
        p.inject_quantizers()
        for mod in m.modules():
            if isinstance(mod, _QBaseLinear) and mod is not m.lm_head:
                mod.ops = FP16AccumMatMul(128, 32)
        if packed:
            pack_linear_weights(m)
            PKD.packed_gemm = lambda *a, **k: (calls.append(1), orig(*a, **k))[1]
        else:
            p.static_quant_wgt()
        try:
            with torch.no_grad():
                outs.append(m(ids))
        finally:
            PKD.packed_gemm = orig
    assert len(calls) == 2 * 7
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
