"""Write the golden fixtures that pin the CPU oracle to the reference quantizer.

This script is the only place that executes reference code.  It runs in the
build container (never on the GPU box), loads ``src/quantizer.py`` from the
read-only reference checkout by file path, and stores inputs/outputs as small
``.npz`` fixtures next to this file.  Only functions that no closed form or
library routine pins are executed:

* ``make_fp_quant`` (element rounding with the 0.5004 threshold and the
  cast back to the tensor dtype, ``src/quantizer.py:187-257``): exhaustive over
  all 65,536 fp16 and bf16 bit patterns for E2M1, E2M2 and E2M5.
* ``MXFPQuantizer.q`` (``src/quantizer.py:513-539``), which rounds elements
  through ``make_fp_quant``: MXFP4, MXFP8 and NVFP4 on seeded tensors.
* ``HBQQuantizer.q`` (``src/quantizer.py:741-859``), whose candidate search
  depends on torch's fp32 accumulation order inside ``sum``: HBQ-A/HBQ-E
  activation and weight variants and the 4-bit KV variant, fp16 and bf16,
  with ``keep_l2_scale=True`` so the L1/L2/scheme choices are recorded.
* The ``torch.compile``d element quantizer that ``GLOBAL_FP_QUANT_CACHE``
  serves (``src/quantizer.py:38-63``) and that ``HBQQuantizer`` uses by default
  (``use_quant_kernel=True``, ``src/quantizer.py:468-469,724``), which is what
  ``PTQ`` builds for every HBQ quantizer: exhaustive element tables and the
  HBQ fixtures again with ``use_quant_kernel=True`` (``compiled_quant.npz``).
  Inductor compiles it for the CPU here (g++); the generator records whether
  the compile fell back to eager (``src/quantizer.py:57-60``).
* ``MXFPQuantizer.q`` with ``per_tensor_scale=True`` (``src/quantizer.py:516-524,
  535-536``), and the PoT HBQ variant on the weight and bf16 inputs
  (``extra_quant.npz``).

Usage:  python tests/golden/gen_golden.py [/root/reference]
"""
import contextlib
import importlib.util
import io
import os
import sys

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))


def load_reference(ref_root):
    path = os.path.join(ref_root, "src", "quantizer.py")
    spec = importlib.util.spec_from_file_location("hbq_reference_quantizer", path)
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def u16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def synth_rows(rows, cols, seed, dtype, wgt=False):
    """Seeded mixture with the value classes the quantizers branch on."""
    g = torch.Generator().manual_seed(seed)
    std = 0.02 if wgt else 1.0
    x = torch.randn(rows, cols, generator=g, dtype=torch.float32) * std
    # outlier channels x50
    oc = torch.randperm(cols, generator=g)[:8]
    x[:, oc] *= 50.0
    # Laplace tail (scale 20*std) on 0.5% of entries
    n = rows * cols
    idx = torch.randperm(n, generator=g)[: n // 200]
    u = torch.rand(idx.numel(), generator=g) - 0.5
    lap = -20.0 * std * torch.sign(u) * torch.log1p(-2.0 * u.abs())
    x.view(-1)[idx] = lap
    # edge rows
    x[0] = 0.0                                   # all-zero blocks
    x[1] = torch.randn(cols, generator=g) * 1e-6  # fp16 subnormal range
    x[2] = torch.randn(cols, generator=g) * 2e4   # near fp16 max
    x[3, ::2] = 0.0
    x[3, 1::4] = -0.0
    x[4] = torch.randint(-8, 9, (cols,), generator=g).float() * 0.25  # exact grid values
    pot = 2.0 ** torch.randint(-12, 12, (cols,), generator=g).float()
    x[5] = pot * torch.sign(torch.randn(cols, generator=g))            # powers of two
    # values a few ulps below powers of two (floor(log2) quirk)
    base = 2.0 ** torch.randint(-10, 14, (cols,), generator=g).float()
    x[6] = base * (1.0 - torch.randint(1, 6, (cols,), generator=g).float() * 2.0 ** -11)
    x[7] = torch.randn(cols, generator=g) * 3e-3
    return x.to(dtype)


def main():
    ref_root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    ref = load_reference(ref_root)
    torch.manual_seed(0)
    out = {"torch_version": np.array(torch.__version__)}

    # 1. element quantizer, exhaustive over every 16-bit pattern
    allbits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    for dt, dname in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
        xs = allbits.view(dt)
        for (e, m) in ((2, 1), (2, 2), (2, 5)):
            f = ref.make_fp_quant(e, m, True, False, False, None, None)
            out[f"elem_{dname}_e{e}m{m}"] = u16(f(xs.clone()))
    np.savez_compressed(os.path.join(HERE, "elem_quant.npz"), **out)

    # 2. MXFP / NVFP quantize-dequantize on seeded tensors
    mx = {"torch_version": np.array(torch.__version__)}
    x16 = synth_rows(32, 1024, 1001, torch.float16)
    x32 = synth_rows(16, 512, 1002, torch.float32)
    mx["x_f16"] = u16(x16)
    mx["x_f32"] = x32.numpy()
    mxcfgs = {
        "mxfp4": dict(block_size=32, ebit=2, mbit=1, sc_ebit=5, sc_mbit=0),
        "mxfp4_round": dict(block_size=32, ebit=2, mbit=1, sc_ebit=5, sc_mbit=0, use_round=True),
        "mxfp8": dict(block_size=32, ebit=2, mbit=5, sc_ebit=5, sc_mbit=0),
        "mxfp8_round": dict(block_size=32, ebit=2, mbit=5, sc_ebit=5, sc_mbit=0, use_round=True),
        "nvfp4": dict(block_size=16, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3),
        "nvfp4_ceil": dict(block_size=16, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3, use_ceil=True),
    }
    for name, kw in mxcfgs.items():
        q = ref.MXFPQuantizer(scale_allow_subnormal=False, **kw)
        mx[f"{name}_f16"] = u16(q.q(x16.clone()))
        mx[f"{name}_f16_scale"] = u16(q.get_shared_scale(q.reshape(x16.clone())[0]).squeeze(-1))
        mx[f"{name}_f32"] = q.q(x32.clone()).numpy()
    # ragged last dim (zero padding to the block) and a 3-D input
    xr = synth_rows(8, 200, 1003, torch.float16)
    mx["x_ragged_f16"] = u16(xr)
    for name in ("mxfp4", "nvfp4"):
        q = ref.MXFPQuantizer(scale_allow_subnormal=False, **mxcfgs[name])
        mx[f"{name}_ragged_f16"] = u16(q.q(xr.clone()))
    np.savez_compressed(os.path.join(HERE, "mxfp_quant.npz"), **mx)

    # 3. HBQ quantize-dequantize with recorded L1/L2/scheme choices
    hb = {"torch_version": np.array(torch.__version__)}
    hbcfgs = {
        "hbq_a_act": dict(ebit=2, mbit=2, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
        "hbq_a_wgt": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix"),
        "hbq_e_act": dict(ebit=2, mbit=2, l2_block_size=32, l2_sc_bit=2, l2_scheme="SIG-1"),
        "hbq_e_wgt": dict(ebit=2, mbit=1, l2_block_size=32, l2_sc_bit=2, l2_scheme="Mix"),
        "hbq_kv4": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="SIG-1"),
        "hbq_a_wgt_ceil": dict(ebit=2, mbit=1, l2_block_size=8, l2_sc_bit=2, l2_scheme="Mix", use_ceil=True),
        "hbq_pot": dict(ebit=2, mbit=1, l2_block_size=4, l2_sc_bit=1, l2_scheme="PoT"),
    }
    inputs = {
        "f16": synth_rows(32, 1024, 2001, torch.float16),
        "f16w": synth_rows(32, 1024, 2002, torch.float16, wgt=True),
        "bf16": synth_rows(32, 1024, 2003, torch.bfloat16),
    }
    for k, v in inputs.items():
        hb[f"x_{k}"] = u16(v)
    for name, kw in hbcfgs.items():
        for k, v in inputs.items():
            if name == "hbq_pot" and k != "f16":
                continue
            q = ref.HBQQuantizer(block_size=128, sc_ebit=5, sc_mbit=3, keep_l2_scale=True,
                                 scale_allow_subnormal=False, use_quant_kernel=False, **kw)
            y = q.q(v.clone())
            hb[f"{name}_{k}"] = u16(y)
            hb[f"{name}_{k}_l1"] = u16(q.shared_scale)
            hb[f"{name}_{k}_l2idx"] = q.l2_scale.numpy().astype(np.uint8)
            hb[f"{name}_{k}_scheme"] = q.blk_l2_scheme.numpy().astype(np.uint8)
            hb[f"{name}_{k}_l2val"] = u16(q.real_l2_scale)
    xr = synth_rows(8, 300, 2004, torch.float16)
    hb["x_ragged_f16"] = u16(xr)
    q = ref.HBQQuantizer(block_size=128, sc_ebit=5, sc_mbit=3, scale_allow_subnormal=False,
                         use_quant_kernel=False, **hbcfgs["hbq_a_act"])
    hb["hbq_a_act_ragged_f16"] = u16(q.q(xr.clone()))
    np.savez_compressed(os.path.join(HERE, "hbq_quant.npz"), **hb)

    write_compiled(ref, inputs, hbcfgs, mxcfgs, x16, x32)
    write_extra(ref, inputs, hbcfgs, mxcfgs)
    print("wrote", sorted(os.listdir(HERE)))


def write_compiled(ref, inputs, hbcfgs, mxcfgs, x16, x32):
    """The compiled element quantizer, alone and inside HBQQuantizer.q / MXFPQuantizer.q."""
    cq = {"torch_version": np.array(torch.__version__)}
    allbits = torch.arange(65536, dtype=torch.int32).to(torch.int16)
    fell_back = False
    for (e, m) in ((2, 1), (2, 2), (2, 5)):
        cfg = ref.FPQuantConfig(ebit=e, mbit=m, allow_subnormal=True, detailed_output=False)
        buf = io.StringIO()
        with contextlib.redirect_stdout(buf):   # the cache prints a message when it falls back
            f = ref.GLOBAL_FP_QUANT_CACHE.get(cfg)
        fell_back |= "compile failed" in buf.getvalue()
        for dt, dname in ((torch.float16, "f16"), (torch.bfloat16, "bf16")):
            cq[f"elem_{dname}_e{e}m{m}"] = u16(f(allbits.view(dt).clone()))
    cq["compile_fell_back"] = np.array(bool(fell_back))
    for name, kw in hbcfgs.items():
        for k, v in inputs.items():
            q = ref.HBQQuantizer(block_size=128, sc_ebit=5, sc_mbit=3, keep_l2_scale=True,
                                 scale_allow_subnormal=False, use_quant_kernel=True, **kw)
            y = q.q(v.clone())
            cq[f"{name}_{k}"] = u16(y)
            cq[f"{name}_{k}_l1"] = u16(q.shared_scale)
            cq[f"{name}_{k}_l2idx"] = q.l2_scale.numpy().astype(np.uint8)
            cq[f"{name}_{k}_scheme"] = q.blk_l2_scheme.numpy().astype(np.uint8)
    for name in ("mxfp4", "mxfp8", "nvfp4"):
        q = ref.MXFPQuantizer(scale_allow_subnormal=False, activate_dynamo=True, **mxcfgs[name])
        cq[f"{name}_f16"] = u16(q.q(x16.clone()))
        cq[f"{name}_f32"] = q.q(x32.clone()).numpy()
    np.savez_compressed(os.path.join(HERE, "compiled_quant.npz"), **cq)


def write_extra(ref, inputs, hbcfgs, mxcfgs):
    """Branches no configuration turns on: the NVFP per-tensor scale, PoT HBQ on more inputs."""
    ex = {"torch_version": np.array(torch.__version__)}
    xs16 = synth_rows(16, 512, 3001, torch.float16)
    xs32 = synth_rows(16, 512, 3002, torch.float32)
    ex["x_f16"] = u16(xs16)
    ex["x_f32"] = xs32.numpy()
    ex["x_zero_f16"] = u16(torch.zeros(4, 64, dtype=torch.float16))
    for name in ("nvfp4", "mxfp4"):
        q = ref.MXFPQuantizer(scale_allow_subnormal=False, per_tensor_scale=True, **mxcfgs[name])
        ex[f"{name}_pts_f16"] = u16(q.q(xs16.clone()))
        ex[f"{name}_pts_f32"] = q.q(xs32.clone()).numpy()
        ex[f"{name}_pts_zero_f16"] = u16(q.q(torch.zeros(4, 64, dtype=torch.float16)))
    for k in ("f16w", "bf16"):
        q = ref.HBQQuantizer(block_size=128, sc_ebit=5, sc_mbit=3, keep_l2_scale=True,
                             scale_allow_subnormal=False, use_quant_kernel=False, **hbcfgs["hbq_pot"])
        y = q.q(inputs[k].clone())
        ex[f"hbq_pot_{k}"] = u16(y)
        ex[f"hbq_pot_{k}_l1"] = u16(q.shared_scale)
        ex[f"hbq_pot_{k}_l2idx"] = q.l2_scale.numpy().astype(np.uint8)
        ex[f"hbq_pot_{k}_scheme"] = q.blk_l2_scheme.numpy().astype(np.uint8)
        ex[f"hbq_pot_{k}_l2val"] = u16(q.real_l2_scale)
    np.savez_compressed(os.path.join(HERE, "extra_quant.npz"), **ex)


if __name__ == "__main__":
    main()
