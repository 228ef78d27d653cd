"""configs[2], configs[3] and configs[4] at their full shapes on the GPU, against the oracle.

The GEMM rows are independent: output row m depends on A's row m and all of B.  So a
sample of rows computed by the oracle from the full-length rows and the whole B *is* the
reference at that shape.  For each configuration:

* the full GEMM runs on the GPU in both operand layouts, W[N, K] and B[K, N] (the
  latter through the transpose), which must give the same bits;
* on 32 sampled rows (tile edges, the middle, the end) the fused epilogue must equal
  the oracle's epilogue on the kernel's own fp32 group partials, bit for bit
  (gemm.cu:354-377, 1198-1277: the fp16 adds and the psum quantization);
* and the oracle's whole GEMM on those rows (sequential fmaf partials) must agree
  within a normwise relative error of 1e-3.

one full-size decoder layer at T = 2048 with every quantizer call (X of the
linears, Q, the K and V caches, the attention weights, and the static weight
quantization) checked on sampled rows against the oracle, and the full 32-layer prefill
with packed decoder weights giving the same logits bit for bit as the fake-quantized
fp16 weights.
"""
import numpy as np
import pytest
import torch

from helpers import mismatches, to_bits

pytestmark = pytest.mark.gpu

HBQ_E_ACT = dict(block_size=128, ebit=2, mbit=2, sc_ebit=5, sc_mbit=3, l2_block_size=32, l2_sc_bit=2,
                 l2_scheme="SIG-1")
HBQ_E_WGT = dict(block_size=128, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3, l2_block_size=32, l2_sc_bit=2,
                 l2_scheme="Mix")
NVFP4 = dict(block_size=16, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3)

# (name, M, K, N, op, group_n, operand format)
CASES = [
    ("cfg2_gateup_grouped", 4096, 4096, 14336, "grouped", 0, "hbq_e"),
    ("cfg2_gateup_mxint8", 4096, 4096, 14336, "mxint8", 32, "hbq_e"),
    ("cfg2_down_grouped", 4096, 14336, 4096, "grouped", 0, "hbq_e"),
    ("cfg3_mxint8_hbq_e", 8192, 4096, 4096, "mxint8", 32, "hbq_e"),
    ("cfg3_mxint8_nvfp4", 8192, 4096, 4096, "mxint8", 32, "nvfp4"),
]


def _operands(M, K, N, fmt, dev, seed):
    """fp16 activations N(0, 1) with 8 outlier channels x50 and weights N(0, 0.02), both
    fake-quantized as the configuration prescribes (use_quant_kernel=True, PTQ's choice)."""
    from hbq_amd.quantizer import HBQQuantizer, MXFPQuantizer
    g = torch.Generator(device=dev).manual_seed(seed)
    X = torch.randn(M, K, device=dev, generator=g)
    oc = torch.randperm(K, device=dev, generator=g)[:8]
    X[:, oc] *= 50.0
    X = X.half()
    W = (torch.randn(N, K, device=dev, generator=g) * 0.02).half()
    if fmt == "hbq_e":
        return HBQQuantizer(**HBQ_E_ACT).q(X), HBQQuantizer(**HBQ_E_WGT).q(W)
    q = MXFPQuantizer(scale_allow_subnormal=False, **NVFP4)
    return q.q(X), q.q(W)


def _sample_rows(M):
    mid = M // 2
    rows = list(range(0, 6)) + [127, 128, 255, 256, 257, 511] + list(range(mid - 3, mid + 3))
    rows += [1000, 2047, 2048, 3333] + list(range(M - 6, M))
    rows = sorted(set(r for r in rows if r < M))
    return rows[:32]


def _gemm(ext, op, A, B, gn, nk):
    if op == "grouped":
        return ext.gemm_fp16_grouped_accum(A, B, 128, b_is_nk=nk)
    return ext.gemm_blockquant_mxint8(A, B, 128, gn, b_is_nk=nk)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_config_gemm_full_shape(gpu, oracle, case):
    from hbq_amd import blockquant_ext as ext
    name, M, K, N, op, gn, fmt = case
    print(f"{name}: M={M} K={K} N={N} {op} gn={gn} {fmt}", flush=True)
    Xq, Wq = _operands(M, K, N, fmt, gpu, seed=M + K + N)
    C = _gemm(ext, op, Xq, Wq, gn, nk=True)
    Bkn = Wq.t().contiguous()
    C_kn = _gemm(ext, op, Xq, Bkn, gn, nk=False)
    assert torch.equal(C.view(torch.int16), C_kn.view(torch.int16)), "W[N,K] and B[K,N] layouts differ"
    assert torch.isfinite(C).all()

    rows = _sample_rows(M)
    Xr = Xq[rows].contiguous()
    C_rows = to_bits(C[rows])
    # the epilogue on the kernel's own group partials of those rows: bit for bit
    P = ext.group_partials(Xr, Wq, 128, b_is_nk=True).cpu().numpy()
    assert P.shape == (K // 128, len(rows), N)
    ref_ep = oracle.epilogue(P, op, gn)
    assert mismatches(C_rows, ref_ep, "f16") == 0, "epilogue on the kernel's partials"
    # the whole oracle GEMM on those rows (sequential fmaf partials): normwise 1e-3
    Xb, Bb = to_bits(Xr), to_bits(Bkn)
    ref = oracle.gemm_fp16_grouped_accum(Xb, Bb, 128) if op == "grouped" else \
        oracle.gemm_blockquant_mxint8(Xb, Bb, 128, gn)
    g = torch.from_numpy(C_rows.view(np.float16).astype(np.float64))
    r = torch.from_numpy(ref.view(np.float16).astype(np.float64))
    rel = ((g - r).norm() / r.norm()).item()
    frac = float((C_rows != ref).mean())
    print(f"{name}: normwise rel err {rel:.2e}, differing elements {frac:.4%}", flush=True)
    assert rel <= 1e-3


def _layer_model(dev, layers):
    from hbq_amd.llama import LlamaConfig, LlamaForCausalLM
    from hbq_amd.ops import stack_qkv_gemms, use_hip_fp32_gemm
    from hbq_amd.ptq import PTQ
    from test_ptq import hbq_cfg
    with torch.device(dev):
        m = LlamaForCausalLM(LlamaConfig(num_hidden_layers=layers)).half()
    m.random_init_(seed=4)
    p = PTQ(hbq_cfg(kv=True), m)     # config/hbq_a_kv.yaml
    p.inject_quantizers()
    use_hip_fp32_gemm(m)
    stack_qkv_gemms(m)
    return m, p


def _row_index(n, k=16):
    idx = sorted(set([0, 1, 2, 3, n - 4, n - 3, n - 2, n - 1] + list(np.linspace(0, n - 1, k - 8).astype(int))))
    return torch.tensor(idx)


def _oracle_rows(oracle, qz, x_rows, dt="f16"):
    return oracle.hbq_qdq(to_bits(x_rows), dt, block_size=qz.block_size, ebit=qz.ebit, mbit=qz.mbit,
                          sc_ebit=qz.sc_ebit, sc_mbit=qz.sc_mbit, l2_block_size=qz.l2_block_size,
                          l2_sc_bit=qz.l2_sc_bit, l2_scheme=qz.l2_scheme, use_ceil=qz.use_ceil,
                          use_quant_kernel=qz._fused)["y"]


def test_config4_full_layer_quantization_points(gpu, oracle):
    """One Llama-3-8B decoder layer at T = 2048 (hidden 4096, 32 heads / 8 KV heads, MLP
    14336): every quantizer call of the prefill, and the static weight quantization, equal
    the oracle on sampled rows of the same full-size inputs (src/module.py:42-67,93-199,
    547-569; src/ptq.py:338-358)."""
    import hbq_amd.llama as L
    from hbq_amd import quantizer as Q
    from hbq_amd.module import _QBaseLinear
    print("config4: one full-size layer, T = 2048", flush=True)
    T = 2048
    m, p = _layer_model(gpu, layers=1)
    # static weight quantization: sampled rows of every linear's weight before and after
    wsamples = []
    for name, mod in m.named_modules():
        if isinstance(mod, _QBaseLinear) and isinstance(getattr(mod, "wq", None), Q.HBQQuantizer):
            idx = _row_index(mod.weight.shape[0])
            wsamples.append((name, mod, idx, mod.weight.detach()[idx.to(gpu)].clone()))
    p.static_quant_wgt()
    for name, mod, idx, before in wsamples:
        got = to_bits(mod.weight.detach()[idx.to(gpu)])
        assert mismatches(got, _oracle_rows(oracle, mod.wq, before), "f16") == 0, name

    checks = []

    def record(qz, x, y):
        x2, y2 = x.reshape(-1, x.shape[-1]), y.reshape(-1, y.shape[-1])
        idx = _row_index(x2.shape[0]).to(x.device)
        checks.append((qz, tuple(x.shape), x2[idx].clone(), y2[idx].clone()))

    for mod in m.modules():
        for attr in ("aq", "kv_quantizer", "attn_wgt_quantizer"):
            qz = getattr(mod, attr, None)
            if isinstance(qz, Q.HBQQuantizer) and "q" not in qz.__dict__:
                orig = qz.q

                def rec(x, _orig=orig, _qz=qz):
                    y = _orig(x)
                    record(_qz, x, y)
                    return y
                qz.q = rec
    orig_causal = L.quantize_causal_

    def rec_causal(qz, pm):
        p2 = pm.reshape(-1, pm.shape[-1])
        idx = _row_index(p2.shape[0]).to(pm.device)
        before = p2[idx].clone()
        y = orig_causal(qz, pm)
        checks.append((qz, tuple(pm.shape), before, y.reshape(-1, y.shape[-1])[idx].clone()))
        return y
    L.quantize_causal_ = rec_causal
    ids = torch.randint(0, 128256, (1, T), device=gpu, generator=torch.Generator(device=gpu).manual_seed(5))
    try:
        with torch.no_grad():
            out = m(ids)
    finally:
        L.quantize_causal_ = orig_causal
    assert torch.isfinite(out).all()
    shapes = set()
    for qz, shape, xr, yr in checks:
        assert mismatches(to_bits(yr), _oracle_rows(oracle, qz, xr), "f16") == 0, shape
        shapes.add(shape)
    print("config4 quantization points:", sorted(shapes), flush=True)
    # X of q/k/v (shared), o, gate/up (shared), down; Q, K, V^T; the attention weights
    assert (1, T, 4096) in shapes and (1, T, 14336) in shapes
    assert (1, 32, T, T) in shapes and (1, 32, T, 128) in shapes
    assert (1, 8, T, 128) in shapes and (1, 8, 128, T) in shapes
    assert len(checks) == 8


def test_config4_packed_weights_same_logits(gpu):
    """The full 32-layer Llama-3-8B prefill at T = 2048: decoder weights packed (3.8 GB
    instead of 14 GB, decoded before each GEMM) give the same logits, bit for bit, as the
    fake-quantized fp16 weights."""
    from hbq_amd.packed import pack_linear_weights
    print("config4: 32 layers, fake-quantized weights", flush=True)
    T = 2048
    ids = torch.randint(0, 128256, (1, T), device=gpu, generator=torch.Generator(device=gpu).manual_seed(4))
    m, p = _layer_model(gpu, layers=32)
    p.static_quant_wgt()
    with torch.no_grad():
        ref = m(ids)
    assert torch.isfinite(ref).all()
    del m, p
    torch.cuda.empty_cache()
    print("config4: 32 layers, packed weights", flush=True)
    m, p = _layer_model(gpu, layers=32)
    pack_linear_weights(m)
    with torch.no_grad():
        out = m(ids)
    assert torch.equal(out.view(torch.int16), ref.view(torch.int16))
