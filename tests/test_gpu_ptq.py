"""The callers of the hot path on the GPU: static weight quantization and the
quantized linear layer with each accumulation kernel (src/ptq.py:338-404,
src/module.py:42-67), checked against the oracle."""
import numpy as np
import pytest
import torch

from helpers import mismatches, synth, to_bits, to_torch
from hbq_amd import blockquant_ext as ext
from hbq_amd.module import _QBaseLinear
from hbq_amd.ptq import PTQ
from test_ptq import Model, hbq_cfg

pytestmark = pytest.mark.gpu


def oracle_hbq(oracle, t, **kw):
    return oracle.hbq_qdq(to_bits(t), "f16", **kw)["y"]


WGT = dict(block_size=128, ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix")
ACT = dict(block_size=128, ebit=2, mbit=2, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1")


def test_static_weight_quant_matches_oracle(gpu, oracle):
    print("static weight quant 384x1024", flush=True)
    w = synth(384, 1024, 21, "f16", std=0.02, outliers=0)
    lin = _QBaseLinear(1024, 384, bias=False).half().to(gpu)
    with torch.no_grad():
        lin.weight.copy_(w.to(gpu))
    p = PTQ(hbq_cfg())
    lin.wq = p.map_wgt_quantizer()
    p.static_quant_linear_weight(lin)
    assert mismatches(to_bits(lin.weight), oracle_hbq(oracle, w, **WGT), "f16") == 0


def test_chunked_weight_quant_equals_whole(gpu):
    print("chunked weight quant", flush=True)
    w = synth(640, 512, 22, "f16", std=0.02, outliers=0).to(gpu)
    p = PTQ(hbq_cfg())
    a, b = _QBaseLinear(512, 640, bias=False).half().to(gpu), _QBaseLinear(512, 640, bias=False).half().to(gpu)
    with torch.no_grad():
        a.weight.copy_(w)
        b.weight.copy_(w)
    a.wq = b.wq = p.map_wgt_quantizer()
    p.static_quant_linear_weight(a)
    p.chunk_static_wgt = True          # the large-model path: row chunks of 128
    p.static_quant_linear_weight(b, chunk_rows=128)
    assert torch.equal(a.weight.view(torch.int16), b.weight.view(torch.int16))


@pytest.mark.parametrize("acc", [{"type": "fp32"}, {"type": "fp16", "group_size": 128},
                                 {"type": "fp16_quant", "group_size": 128, "quant_block_size": 32}])
def test_linear_forward(gpu, oracle, acc):
    print(f"linear forward acc={acc}", flush=True)
    m = Model(1).half().to(gpu)
    p = PTQ(hbq_cfg(acc=acc), m)
    p.inject_quantizers()
    with torch.no_grad():
        for lin in m.modules():
            if isinstance(lin, _QBaseLinear):
                lin.weight.copy_(torch.randn_like(lin.weight) * 0.02)
    p.static_quant_wgt()
    p.replace_accum_kernel()
    lin = m.layers[0].mlp.gate_proj
    x = synth(64, 256, 23, "f16").view(2, 32, 256)
    y = lin(x.to(gpu))
    xq = to_torch(oracle_hbq(oracle, x.view(64, 256), **ACT), "f16").to(gpu)
    # the input quantizer's output is the oracle's
    assert mismatches(to_bits(lin.aq(x.to(gpu))).reshape(64, 256), to_bits(xq), "f16") == 0
    W = lin.weight
    if acc["type"] == "fp32":
        ref = torch.nn.functional.linear(xq, W)
    elif acc["type"] == "fp16":
        ref = ext.gemm_fp16_grouped_accum(xq, W.t().contiguous(), 128)
    else:
        ref = ext.gemm_blockquant_mxint8(xq, W.t().contiguous(), 128, 32)
    assert y.shape == (2, 32, 512)
    assert torch.equal(y.view(64, 512).view(torch.int16), ref.view(torch.int16))


def test_linear_nonfinite_raises(gpu):
    lin = _QBaseLinear(128, 32, bias=False).half().to(gpu)
    with torch.no_grad():
        lin.weight.fill_(60000.0)
    with pytest.raises(RuntimeError, match="Non-finite output"):
        lin(torch.full((4, 128), 100.0, dtype=torch.float16, device=gpu))


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16, torch.float32])
def test_flag_nonfinite(gpu, dt):
    """hbq_flag_nonfinite: set for a NaN / +inf / -inf anywhere (the 16-byte body or the
    tail), left alone for finite extremes (max normal, subnormals, -0)."""
    from hbq_amd import _lib
    L = _lib.lib()
    big = torch.finfo(dt).max
    for n in (1, 7, 8, 9, 1000, 3 * 4096 + 5):
        base = torch.randn(n, device=gpu).to(dt)
        base[0] = big
        base[-1] = -big
        if n > 2:
            base[1] = torch.finfo(dt).tiny / 4   # subnormal
            base[2] = -0.0
        flag = torch.zeros(1, dtype=torch.int32, device=gpu)
        _lib.check(L.hbq_flag_nonfinite(_lib.ptr(base), 1, n, n, _lib.DTYPE_CODE[dt], _lib.ptr(flag),
                                        _lib.stream_of(base)))
        assert int(flag.item()) == 0, n
        for pos in sorted({0, n // 2, n - 1}):
            for bad in (float("nan"), float("inf"), -float("inf")):
                x = base.clone()
                x[pos] = bad
                flag.zero_()
                _lib.check(L.hbq_flag_nonfinite(_lib.ptr(x), 1, n, n, _lib.DTYPE_CODE[dt], _lib.ptr(flag),
                                                _lib.stream_of(x)))
                assert int(flag.item()) == 1, (n, pos, bad)


@pytest.mark.parametrize("dt", [torch.float16, torch.float32])
def test_flag_nonfinite_column_slice(gpu, dt):
    """A column slice of a wider output (row stride > cols): only its own columns count."""
    from hbq_amd import _lib
    L = _lib.lib()
    y = torch.randn(64, 96, device=gpu).to(dt)
    y[5, 90] = float("nan")                      # outside the slice [:, 8:72]
    flag = torch.zeros(1, dtype=torch.int32, device=gpu)
    for lo, hi, expect in ((8, 72, 0), (8, 91, 1), (3, 8, 0), (3, 9, 0)):
        sl = y[:, lo:hi]
        flag.zero_()
        _lib.check(L.hbq_flag_nonfinite(_lib.ptr(sl), sl.shape[0], sl.shape[1], sl.stride(0),
                                        _lib.DTYPE_CODE[dt], _lib.ptr(flag), _lib.stream_of(sl)))
        assert int(flag.item()) == expect, (lo, hi)
    y[63, 8] = -float("inf")
    flag.zero_()
    sl = y[:, 8:72]
    _lib.check(L.hbq_flag_nonfinite(_lib.ptr(sl), 64, 64, 96, _lib.DTYPE_CODE[dt], _lib.ptr(flag), _lib.stream_of(sl)))
    assert int(flag.item()) == 1
