"""one Llama-3-8B q_proj-shaped linear, HBQ-A W4/A5 (config/hbq_a.yaml) then a
matmul with fp32 accumulation.  Codes, scales and dequantized tensors against the oracle
(bit-exact), the product against float64 (normwise tolerance 1e-3: the fp32 sum order of
the reference's F.linear is not pinned, the fp16 output rounding is 2^-11)."""
import numpy as np
import pytest
import torch

from helpers import mismatches, to_bits, to_torch
from hbq_amd.quantizer import HBQQuantizer

pytestmark = pytest.mark.gpu


def config0_inputs(seed=1000):
    g = torch.Generator().manual_seed(seed)
    W = (torch.randn(4096, 4096, generator=g) * 0.02).half()
    X = torch.randn(2048, 4096, generator=g)
    X[:, torch.randperm(4096, generator=g)[:8]] *= 50.0
    return W, X.half()


def test_config0_linear(gpu, oracle):
    print("configs[0] q_proj linear", flush=True)
    W, X = config0_inputs()
    wq = HBQQuantizer(block_size=128, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3, l2_block_size=8, l2_sc_bit=2,
                      l2_scheme="Mix", keep_l2_scale=True)
    aq = HBQQuantizer(block_size=128, ebit=2, mbit=2, sc_ebit=5, sc_mbit=3, l2_block_size=8, l2_sc_bit=2,
                      l2_scheme="SIG-1", keep_l2_scale=True)
    Wq = wq.q(W.to(gpu))
    w_attrs = (wq.shared_scale, wq.l2_scale, wq.blk_l2_scheme)
    Xq = aq.q(X.to(gpu))
    x_attrs = (aq.shared_scale, aq.l2_scale, aq.blk_l2_scheme)
    for q, (src, kw), attrs in ((Wq, (W, dict(mbit=1, l2_scheme="Mix")), w_attrs),
                                (Xq, (X, dict(mbit=2, l2_scheme="SIG-1")), x_attrs)):
        ref = oracle.hbq_qdq(to_bits(src), "f16", block_size=128, ebit=2, sc_ebit=5, sc_mbit=3, l2_block_size=8,
                             l2_sc_bit=2, **kw)
        assert mismatches(to_bits(q), ref["y"], "f16") == 0
        assert mismatches(to_bits(attrs[0].reshape(ref["l1"].shape)), ref["l1"], "f16") == 0
        assert np.array_equal(attrs[1].cpu().numpy().reshape(ref["l2idx"].shape), ref["l2idx"])
        assert np.array_equal(attrs[2].cpu().numpy().reshape(ref["scheme"].shape), ref["scheme"])
    from hbq_amd import blockquant_ext as ext
    Y = ext.gemm_fp32_accum_nk(Xq, Wq)
    ref = Xq.double().cpu() @ Wq.double().cpu().t()
    rel = ((Y.double().cpu() - ref).norm() / ref.norm()).item()
    print(f"configs[0] product: normwise rel err {rel:.2e}", flush=True)
    assert Y.shape == (2048, 4096) and rel <= 1e-3
