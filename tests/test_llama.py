"""The Llama decoder with the reference's quantization points (src/module.py:93-199,
547-569) driven by PTQ: structure on the CPU, kernels and quantization points on
the GPU against the oracle."""
import numpy as np
import pytest
import torch

from hbq_amd import quantizer as Q
from hbq_amd.llama import LlamaConfig, LlamaForCausalLM
from hbq_amd.module import _QBaseLinear
from hbq_amd.ptq import PTQ
from helpers import mismatches, to_bits
from test_ptq import hbq_cfg

TINY = LlamaConfig(hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
                   num_key_value_heads=2, vocab_size=1000)


def test_structure_and_injection_cpu():
    m = LlamaForCausalLM(TINY).random_init_()
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    a = m.layers[0].self_attn
    assert a.quant_post_rope_q and a.quant_k_cache and a.quant_v_cache and a.quant_attn_wgt
    assert isinstance(a.kv_quantizer, Q.HBQQuantizer) and a.kv_quantizer.mbit == 1
    assert sum(isinstance(x, _QBaseLinear) for x in m.modules()) == 2 * 7 + 1
    # unquantized forward (identity quantizers) on the CPU
    m2 = LlamaForCausalLM(TINY).random_init_()
    y = m2(torch.randint(0, 1000, (1, 16)))
    assert y.shape == (1, 16, 1000) and torch.isfinite(y).all()


@pytest.mark.gpu
def test_quantization_points_match_oracle(gpu, oracle):
    """Every quantizer call of a prefill (X of each linear, post-RoPE Q, K and V caches, the
    attention weights) returns the oracle's result on the same input."""
    print("llama quantization points", flush=True)
    torch.manual_seed(0)
    m = LlamaForCausalLM(TINY).random_init_().half().to(gpu)
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    p.static_quant_wgt()
    calls = []
    for mod in m.modules():
        for attr in ("aq", "kv_quantizer", "attn_wgt_quantizer"):
            qz = getattr(mod, attr, None)
            if isinstance(qz, Q.HBQQuantizer) and not hasattr(qz, "_wrapped"):
                orig = qz.q

                def rec(x, _orig=orig, _qz=qz):
                    y = _orig(x)
                    calls.append((_qz, x.detach().clone(), y.detach().clone()))
                    return y
                qz.q = rec
                qz._wrapped = True
    # the attention weights go through the in-place causal quantizer, not qz.q
    import hbq_amd.llama as L
    orig_causal = L.quantize_causal_

    def rec_causal(qz, p):
        x = p.detach().clone()
        y = orig_causal(qz, p)
        calls.append((qz, x, y.detach().clone()))
        return y
    L.quantize_causal_ = rec_causal
    ids = torch.randint(0, TINY.vocab_size, (1, 128), device=gpu)
    try:
        with torch.no_grad():
            out = m(ids)
    finally:
        L.quantize_causal_ = orig_causal
    assert torch.isfinite(out).all()
    kinds = set()
    for qz, x, y in calls:
        xs = to_bits(x.reshape(-1, x.shape[-1]))
        ref = oracle.hbq_qdq(xs, "f16", block_size=qz.block_size, ebit=qz.ebit, mbit=qz.mbit, sc_ebit=qz.sc_ebit,
                             sc_mbit=qz.sc_mbit, l2_block_size=qz.l2_block_size, l2_sc_bit=qz.l2_sc_bit,
                             l2_scheme=qz.l2_scheme, use_quant_kernel=qz._fused)["y"]
        assert mismatches(to_bits(y.reshape(-1, y.shape[-1])), ref, "f16") == 0
        kinds.add((qz.mbit, tuple(x.shape[-2:]) if x.dim() == 4 else "x"))
    # X of the projections (q/k/v and gate/up share one quantized copy), Q (E2M2), K and V
    # (E2M1, V transposed: tokens last), P
    assert len(calls) == TINY.num_hidden_layers * (4 + 4)
    assert (1, (128, TINY.head_dim)) in kinds and (1, (TINY.head_dim, 128)) in kinds and (2, (128, 128)) in kinds


@pytest.mark.gpu
def test_prefill_fast_kernels_equal_generic(gpu):
    """The same prefill with every quantizer forced onto the generic kernel: identical logits."""
    from hbq_amd import _lib
    print("llama prefill fast vs generic", flush=True)
    m = LlamaForCausalLM(TINY).random_init_(seed=3).half().to(gpu)
    p = PTQ(hbq_cfg(kv=True, acc={"type": "fp16_quant", "group_size": 128, "quant_block_size": 32}), m)
    p.inject_quantizers()
    p.static_quant_wgt()
    p.replace_accum_kernel()
    ids = torch.randint(0, TINY.vocab_size, (1, 256), device=gpu)
    with torch.no_grad():
        a = m(ids)
        old = _lib.lib().hbq_set_generic_only(1)
        try:
            b = m(ids)
        finally:
            _lib.lib().hbq_set_generic_only(old)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_nonfinite_raises_after_forward_cpu():
    m = LlamaForCausalLM(TINY).random_init_()
    with torch.no_grad():
        m.layers[1].mlp.down_proj.weight.fill_(float("inf"))
    with pytest.raises(RuntimeError, match="Non-finite output"):
        m(torch.randint(0, 1000, (1, 8)))


@pytest.mark.gpu
def test_dedupe_equal_to_separate_quantization(gpu):
    """Quantizing the shared input once gives the same projections as quantizing per projection."""
    m = LlamaForCausalLM(TINY).random_init_(seed=5).half().to(gpu)
    p = PTQ(hbq_cfg(), m)
    p.inject_quantizers()
    a = m.layers[0].self_attn
    x = torch.randn(1, 64, TINY.hidden_size, device=gpu).half()
    with torch.no_grad():
        sep = [a.q_proj(x), a.k_proj(x), a.v_proj(x)]
        xq = a.q_proj.aq(x)
        shared = [a.q_proj.forward_quantized(xq), a.k_proj.forward_quantized(xq), a.v_proj.forward_quantized(xq)]
    for u, w in zip(sep, shared):
        assert torch.equal(u.view(torch.int16), w.view(torch.int16))


@pytest.mark.gpu
def test_hip_fp32_gemm_linears(gpu):
    """The prefill with the linears on the HIP fp32-accumulation GEMM stays close to F.linear
    (same quantized operands; only the fp32 summation order differs)."""
    from hbq_amd.ops import use_hip_fp32_gemm
    m = LlamaForCausalLM(TINY).random_init_(seed=6).half().to(gpu)
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    p.static_quant_wgt()
    ids = torch.randint(0, TINY.vocab_size, (1, 128), device=gpu)
    with torch.no_grad():
        a = m(ids).float()
        assert use_hip_fp32_gemm(m) == TINY.num_hidden_layers * 7
        b = m(ids).float()
    rel = ((a - b).norm() / a.norm()).item()
    print(f"hip fp32 gemm vs F.linear: normwise rel {rel:.2e}", flush=True)
    assert rel < 2e-2


def test_stacked_weight_views_cpu():
    """The stack holds the weights as consecutive row ranges; parameters view it (in-place
    updates reach it); a replaced weight makes the next call build it again."""
    from hbq_amd.module import _stacked_weight
    torch.manual_seed(1)
    mods = [_QBaseLinear(32, n, bias=False) for n in (48, 16, 16)]
    ref = [m.weight.detach().clone() for m in mods]
    W = _stacked_weight(mods)
    assert W.shape == (80, 32) and torch.equal(W, torch.cat(ref))
    assert all(m.weight.data_ptr() == W[o:].data_ptr() for m, o in zip(mods, (0, 48, 64)))
    assert _stacked_weight(mods) is W
    with torch.no_grad():
        mods[1].weight[3].fill_(7.0)            # in place: lands in the stack
    assert torch.equal(W[51], torch.full((32,), 7.0)) and _stacked_weight(mods) is W
    new = torch.randn(16, 32)
    mods[2].weight.data = new.clone()           # replaced: built again with the new rows
    W2 = _stacked_weight(mods)
    assert W2 is not W and torch.equal(W2[64:], new) and torch.equal(W2[48:64], mods[1].weight)
    assert mods[2].weight.data_ptr() == W2[64:].data_ptr()


def test_fusable_rules_cpu():
    """Stacking needs one HIP operator type and settings, no bias and psum blocks that do not
    straddle two linears; a CPU weight is never stacked."""
    from hbq_amd.module import _fusable
    from hbq_amd.ops import FP16AccumMatMul
    mods = [_QBaseLinear(32, n, bias=False, ops=FP16AccumMatMul(64, 32)) for n in (64, 32)]
    for m in mods:
        m.half()
    assert not _fusable(mods)                   # CPU weights
    assert not _fusable([_QBaseLinear(32, 64, bias=False), _QBaseLinear(32, 64, bias=False)])   # F.linear


@pytest.mark.gpu
@pytest.mark.parametrize("ops", ["fp32", "fp16", "grouped", "mxint8"])
def test_stacked_qkv_bit_identical(gpu, ops):
    """A prefill with q, k and v as one GEMM over the stacked weights gives the same bits as
    three GEMMs, for every HIP accumulation mode; after a weight is replaced the stack follows."""
    from hbq_amd.module import _fusable
    from hbq_amd.ops import FP16AccumMatMul, FP32AccumMatMul, stack_qkv_gemms
    print(f"stacked qkv {ops}", flush=True)
    make = {"fp32": FP32AccumMatMul, "fp16": FP16AccumMatMul, "grouped": lambda: FP16AccumMatMul(64),
            "mxint8": lambda: FP16AccumMatMul(64, 16)}[ops]
    m = LlamaForCausalLM(TINY).random_init_(seed=8).half().to(gpu)
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    for mod in m.modules():
        if isinstance(mod, _QBaseLinear) and mod is not m.lm_head:
            mod.ops = make()
    p.static_quant_wgt()
    ids = torch.randint(0, TINY.vocab_size, (1, 96), device=gpu, generator=torch.Generator(device=gpu).manual_seed(8))
    a = m.layers[0].self_attn
    with torch.no_grad():
        sep = m(ids)
        assert stack_qkv_gemms(m) == TINY.num_hidden_layers
        assert _fusable((a.q_proj, a.k_proj, a.v_proj))
        st = m(ids)
        assert a.q_proj.weight.data_ptr() == a.q_proj.__dict__["_hbq_stack"].data_ptr()
        assert torch.equal(sep.view(torch.int16), st.view(torch.int16))
        a.v_proj.weight.data = a.v_proj.weight.detach().flip(0).contiguous()
        st2 = m(ids)
        for layer in m.layers:
            layer.self_attn.stack_qkv = False
        sep2 = m(ids)
    assert torch.equal(sep2.view(torch.int16), st2.view(torch.int16))
    assert not torch.equal(st.view(torch.int16), st2.view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_scale_causal_mask_matches_torch(gpu, dt):
    """The fused scale + causal bias pass equals torch's `s * scale` then `s + bias`
    (src/module.py:96-112) bit for bit, with -0, infinities and large values in the scores."""
    from hbq_amd.llama import scale_causal_mask_
    g = torch.Generator(device=gpu).manual_seed(12)
    for T in (8, 64, 136):
        s = (torch.randn(3, T, T, device=gpu, generator=g) * 40).to(dt)
        s[0, 0, :4] = torch.tensor([-0.0, float("inf"), -float("inf"), 3e4], dtype=dt)
        s[1, 5, 2] = -0.0
        s[2, T - 1, T - 1] = torch.finfo(dt).max
        scale = 1.0 / (128 ** 0.5)
        ref = s * scale
        ref = ref + torch.full((T, T), float("-inf"), device=gpu, dtype=dt).triu(1)
        got = scale_causal_mask_(s.clone(), scale)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), T


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rope_matches_torch(gpu, dt):
    """The fused rotary pass equals torch's q * cos + rotate_half(q) * sin bit for bit, read from
    a strided [b, t, h, d] view (a column slice of the stacked q/k/v output) and written
    contiguous [b, h, t, d]."""
    from hbq_amd.llama import LlamaConfig, apply_rope, rope, rotary
    g = torch.Generator(device=gpu).manual_seed(13)
    b, T, H, d = 2, 96, 4, 64
    full = (torch.randn(b, T, 3 * H * d, device=gpu, generator=g) * 8).to(dt)
    full[0, 0, :8] = torch.tensor([-0.0, float("inf"), -float("inf"), float("nan"), 6e4, -6e4, 1e-7, -1e-7],
                                  dtype=torch.float32).to(dt)
    x = full[..., H * d: 2 * H * d].view(b, T, H, d)          # strided like the k slice
    cos, sin = rotary(LlamaConfig(hidden_size=H * d, num_attention_heads=H, num_key_value_heads=H), T, gpu)
    ref, _ = apply_rope(x.transpose(1, 2), x.transpose(1, 2), cos, sin)
    got = rope(x, cos.to(dt).contiguous(), sin.to(dt).contiguous())
    assert got.is_contiguous() and got.shape == ref.shape
    assert torch.equal(got.view(torch.int16), ref.contiguous().view(torch.int16))


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_causal_softmax_matches_torch(gpu, dt):
    """The fused scale + causal bias + softmax pass equals torch's `s * scale`, `s + bias` and
    `torch.softmax` bit for bit, rows with infinities and NaN included."""
    from hbq_amd.llama import causal_softmax_
    g = torch.Generator(device=gpu).manual_seed(14)
    scale = 1.0 / (128 ** 0.5)
    for T in (64, 128, 256, 2048):
        mats = 3 if T < 2048 else 2
        s = (torch.randn(mats, T, T, device=gpu, generator=g) * 30).to(dt)
        s[0, 5, 2] = float("inf")            # unmasked +inf: NaN row in torch
        s[0, 6, 9] = float("inf")            # masked +inf: inf - inf = NaN as well
        s[0, 7, 3] = -float("inf")
        s[1, 8, 1] = float("nan")
        s[1, 3, 40] = float("nan")          # masked NaN: the whole row is NaN
        s[1, 4, 50] = -float("inf")         # masked -inf: an ordinary masked row
        s[1, T - 1, :] = -6e4 if dt == torch.float16 else -3e38
        ref = s * scale
        ref = ref + torch.full((T, T), float("-inf"), device=gpu, dtype=dt).triu(1)
        ref = torch.softmax(ref, dim=-1)
        got = causal_softmax_(s.clone(), scale)
        same = got.view(torch.int16) == ref.view(torch.int16)
        assert bool(same.all()), (T, int((~same).sum()))


def test_grouped_query_attention_equals_repeated_kv_cpu():
    """The attention that multiplies each kv head by its query heads as one operand equals
    the one on repeat_interleave'd k and v (repeat_kv), up to the fp32 summation order."""
    torch.manual_seed(3)
    a = LlamaForCausalLM(TINY).layers[0].self_attn
    H, KVH, T, d = TINY.num_attention_heads, TINY.num_key_value_heads, 32, TINY.head_dim
    q = torch.randn(2, H, T, d)
    k = torch.randn(2, KVH, T, d)
    v = torch.randn(2, KVH, T, d)
    out, p = a.manual_sdpa(q, k, v)
    out_t, _ = a.manual_sdpa(q, k, None, vT=v.transpose(-1, -2).contiguous())   # the V^T entry
    torch.testing.assert_close(out_t, out, rtol=1e-6, atol=1e-6)
    kr, vr = k.repeat_interleave(H // KVH, dim=1), v.repeat_interleave(H // KVH, dim=1)
    s = q @ kr.transpose(-2, -1) / d ** 0.5 + torch.full((T, T), float("-inf")).triu(1)
    pr = torch.softmax(s, dim=-1)
    assert p.shape == (2, H, T, T)
    torch.testing.assert_close(p, pr, rtol=1e-5, atol=1e-6)
    torch.testing.assert_close(out, pr @ vr, rtol=1e-5, atol=1e-5)


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_add_rmsnorm_matches_torch(gpu, dt):
    """The fused residual add + RMSNorm equals x + res and the torch RMSNorm bit for bit,
    infinities and NaN included; without res, the norm alone."""
    from hbq_amd.llama import RMSNorm
    g = torch.Generator(device=gpu).manual_seed(21)
    norm = RMSNorm(1024, 1e-5).to(gpu).to(dt)
    with torch.no_grad():
        norm.weight.copy_(torch.randn(1024, device=gpu, generator=g) * 0.5 + 1)
    x = (torch.randn(64, 1024, device=gpu, generator=g) * 3).to(dt)
    res = (torch.randn(64, 1024, device=gpu, generator=g) * 2).to(dt)
    x[0, :] = x[0, :] * 1e-3                 # tiny rows
    x[1, :] = 60000.0 if dt == torch.float16 else 1e30
    res[2, 5] = float("inf")
    res[3, 7] = float("nan")
    with torch.no_grad():
        s, y = norm.add_norm(x, res)
        s_ref = x + res
        y_ref = norm(s_ref)
        y0, y0_ref = norm.add_norm(x)[1], norm(x)
    for name, got, ref in (("sum", s, s_ref), ("norm", y, y_ref), ("norm alone", y0, y0_ref)):
        same = got.view(torch.int16) == ref.view(torch.int16)
        bad = (~same).nonzero()[:4].tolist()
        assert bool(same.all()), (name, int((~same).sum()), [(i, float(got[i[0], i[1]]), float(ref[i[0], i[1]]))
                                                            for i in bad])


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_silu_mul_matches_torch(gpu, dt):
    """silu(gate) * up in one HIP pass equals torch's two ops bit for bit, over every 16-bit
    pattern of the gate."""
    from hbq_amd.llama import silu_mul
    gate = torch.arange(-32768, 32768, dtype=torch.int32, device=gpu).to(torch.int16).view(dt)
    up = torch.randn(gate.shape, device=gpu, generator=torch.Generator(device=gpu).manual_seed(4)).to(dt) * 4
    got = silu_mul(gate, up)
    ref = torch.nn.functional.silu(gate) * up
    same = got.view(torch.int16) == ref.view(torch.int16)
    assert bool(same.all()), int((~same).sum())


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_causal_quantizer_equals_full(gpu, dt):
    """The in-place attention-weight quantizer that never touches the blocks above the
    diagonal gives qz.q(p) bit for bit on causal softmax outputs (HBQ-A act, HBQ-E act and
    a Mix weight configuration)."""
    from hbq_amd.llama import causal_softmax_, quantize_causal_
    g = torch.Generator(device=gpu).manual_seed(8)
    qzs = [Q.HBQQuantizer(block_size=128, ebit=2, mbit=2, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
           Q.HBQQuantizer(block_size=128, ebit=2, mbit=2, l2_block_size=32, l2_sc_bit=2, l2_scheme="SIG-1"),
           Q.HBQQuantizer(block_size=128, ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix")]
    for T, mats in ((128, 5), (256, 3), (2048, 2)):
        s = (torch.randn(mats, T, T, device=gpu, generator=g) * 8).to(dt)
        p = causal_softmax_(s, 0.088)
        for qz in qzs:
            ref = qz.q(p)
            pin = p.clone()
            got = quantize_causal_(qz, pin)
            assert got is pin                   # the in-place kernel ran
            same = got.view(torch.int16) == ref.view(torch.int16)
            assert bool(same.all()), (T, qz.l2_scheme, qz.l2_block_size, int((~same).sum()))


# activation quantizers that the fused producer passes take (E2M2, one L2 scheme, block 128)
FUSED_QZ = [dict(l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),                        # HBQ-A act
            dict(l2_block_size=32, l2_sc_bit=2, l2_scheme="SIG-1"),                       # HBQ-E act
            dict(l2_block_size=16, l2_sc_bit=1, l2_scheme="FP-1", use_quant_kernel=False),
            dict(l2_block_size=8, l2_sc_bit=2, l2_scheme="PoT", use_ceil=True)]


def _fused_qz(kw):
    return Q.HBQQuantizer(block_size=128, ebit=2, mbit=2, sc_ebit=5, sc_mbit=3, **kw)


def _same16(got, ref, what):
    same = got.view(torch.int16) == ref.view(torch.int16)
    assert bool(same.all()), (what, int((~same).sum()), (~same).nonzero()[:4].tolist())


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_rms_apply_quant_equals_two_passes(gpu, dt):
    """The RMSNorm apply step with the input quantizer in the same pass gives aq.q(norm(x +
    res)) bit for bit, the sum too; rows of tiny, huge, infinite and NaN values included."""
    from hbq_amd.llama import RMSNorm
    g = torch.Generator(device=gpu).manual_seed(31)
    for cols in (1024, 4096):
        norm = RMSNorm(cols, 1e-5).to(gpu).to(dt)
        with torch.no_grad():
            norm.weight.copy_(torch.randn(cols, device=gpu, generator=g) * 0.5 + 1)
        x = (torch.randn(37, cols, device=gpu, generator=g) * 3).to(dt)
        res = (torch.randn(37, cols, device=gpu, generator=g) * 2).to(dt)
        x[0, :] = x[0, :] * 1e-3
        x[1, :] = 60000.0 if dt == torch.float16 else 1e30
        x[4, ::7] *= 80.0                                   # outlier channels
        res[2, 5] = float("inf")
        res[3, 7] = float("nan")
        # a huge value per block and tiny ones whose quotients underflow (u = 0: +0 whatever
        # the sign), and a row of negative zeros
        big, tiny = (6e4, 6e-8) if dt == torch.float16 else (1e30, 1e-30)
        x[5, :] = tiny * torch.sign(x[5, :])
        x[5, ::128] = big
        res[5, :] = 0.0
        x[6, :] = -0.0
        res[6, :] = -0.0
        for kw in FUSED_QZ:
            qz = _fused_qz(kw)
            with torch.no_grad():
                s, yq, done = norm.add_norm_quant(x, res, qz)
                s_ref, y_ref = norm.add_norm(x, res)
                ref = qz.q(y_ref)
                y0, done0 = norm.add_norm_quant(x, None, qz)[1:]
                ref0 = qz.q(norm.add_norm(x)[1])
            assert done and done0, kw
            _same16(s, s_ref, ("sum", cols, kw))
            _same16(yq, ref, ("norm + quantizer", cols, kw))
            _same16(y0, ref0, ("norm alone + quantizer", cols, kw))


@pytest.mark.gpu
@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_silu_mul_quant_equals_two_passes(gpu, dt):
    """silu(gate) * up with the input quantizer in the same pass gives aq.q(silu_mul(gate,
    up)) bit for bit: every 16-bit pattern of the gate, a [37, 14336] MLP-shaped input, and
    blocks whose tiny products quantize to u = 0 next to a huge one."""
    from hbq_amd.llama import silu_mul, silu_mul_quant
    g = torch.Generator(device=gpu).manual_seed(32)
    gate_all = torch.arange(-32768, 32768, dtype=torch.int32, device=gpu).to(torch.int16).view(dt).view(512, 128)
    # blocks of one huge product and tiny ones of either sign, whose quotients underflow
    big, tiny = (6e4, 6e-8) if dt == torch.float16 else (1e30, 1e-30)
    mix = torch.full((64, 1024), -tiny, device=gpu).to(dt)
    mix[:, 1::3] = tiny
    mix[:, ::128] = big
    cases = [(gate_all, (torch.randn(512, 128, device=gpu, generator=g) * 4).to(dt)),
             ((torch.randn(37, 14336, device=gpu, generator=g) * 2).to(dt),
              (torch.randn(37, 14336, device=gpu, generator=g)).to(dt)),
             (mix, torch.ones(64, 1024, device=gpu).to(dt))]
    for gate, up in cases:
        for kw in FUSED_QZ:
            qz = _fused_qz(kw)
            got = silu_mul_quant(gate, up, qz)
            assert got is not None, kw
            _same16(got, qz.q(silu_mul(gate, up)), (tuple(gate.shape), kw))


@pytest.mark.gpu
def test_attention_output_into_o_proj_layout(gpu):
    """The P V product written straight into [b, T, H, d] (per query head, W shared by the
    kv head's group) equals the kv-head-batched product transposed, bit for bit."""
    m = LlamaForCausalLM(TINY).random_init_(seed=7).half().to(gpu)
    a = m.layers[0].self_attn
    g = torch.Generator(device=gpu).manual_seed(7)
    b, T, d = 1, 256, TINY.head_dim
    q = torch.randn(b, TINY.num_attention_heads, T, d, device=gpu, generator=g).half()
    k = torch.randn(b, TINY.num_key_value_heads, T, d, device=gpu, generator=g).half()
    vT = torch.randn(b, TINY.num_key_value_heads, d, T, device=gpu, generator=g).half()
    with torch.no_grad():
        ref, _ = a.manual_sdpa(q, k, None, vT=vT)
        got, _ = a.manual_sdpa(q, k, None, vT=vT, out_bthd=True)
    assert got.shape == (b, T, TINY.num_attention_heads, d) and got.is_contiguous()
    assert torch.equal(got.view(torch.int16), ref.transpose(1, 2).contiguous().view(torch.int16))


@pytest.mark.gpu
def test_fused_input_quantizers_same_logits(gpu):
    """A prefill with the linears' input quantizers computed inside the norms and the SiLU
    product gives the logits of the separate passes bit for bit, with three fewer quantizer
    passes per layer (q/k/v, gate/up and down inputs)."""
    from hbq_amd.ops import fuse_input_quantizers, stack_qkv_gemms, use_hip_fp32_gemm
    m = LlamaForCausalLM(TINY).random_init_(seed=6).half().to(gpu)
    p = PTQ(hbq_cfg(kv=True), m)
    p.inject_quantizers()
    p.static_quant_wgt()
    use_hip_fp32_gemm(m)
    stack_qkv_gemms(m)
    ids = torch.randint(0, TINY.vocab_size, (1, 256), device=gpu, generator=torch.Generator(device=gpu).manual_seed(6))
    calls = []
    orig = Q.HBQQuantizer.q

    def counting(self, x):
        calls.append(1)
        return orig(self, x)
    Q.HBQQuantizer.q = counting
    try:
        with torch.no_grad():
            ref = m(ids)
            n_sep = len(calls)
            assert fuse_input_quantizers(m) == TINY.num_hidden_layers
            calls.clear()
            out = m(ids)
            n_fused = len(calls)
    finally:
        Q.HBQQuantizer.q = orig
        fuse_input_quantizers(m, on=False)
    assert n_sep - n_fused == 3 * TINY.num_hidden_layers, (n_sep, n_fused)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
