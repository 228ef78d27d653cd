"""CPU checks of the arithmetic identities the GPU kernels rely on.

The quantizer kernels replace every reference division R_T(x / s) by a scale
s (an E5M3 L1 scale, an L2 factor, the NVFP scale) with R_T(R32(x * R32(1/s)))
whenever the quotient is not in T's subnormal range.  That is exact only
because no quotient lies within the product's error of a rounding boundary of
T.  These tests check it for every fp16 / bf16 input and every scale value."""
import numpy as np
import pytest
import torch

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)


def _values(dt):
    t = torch.from_numpy(ALL16.view(np.int16)).view(dt).float()
    t = t[torch.isfinite(t)]
    return t.numpy().astype(np.float32)


def _scales():
    e5m3 = [(1 + m / 8) * 2.0 ** e for e in range(-14, 16) for m in range(8)]
    l2 = [1.0, 1.5, 2.0, 2.5, 1.25, 1.75, 1.125, 1.375, 3.0, 4.0, 1.0625, 1.1875, 8.0]
    elem_max = [6.0, 7.0, 7.875]
    return np.array(sorted(set(e5m3 + l2 + elem_max)), np.float64)


def _round_T(v32, dt):
    return torch.from_numpy(np.ascontiguousarray(v32, np.float32)).to(dt).float().numpy()


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_reciprocal_division_identity(dt):
    x = _values(dt)
    tiny = 2.0 ** -14 if dt == torch.float16 else 2.0 ** -126
    bad = 0
    for s in _scales():
        exact = _round_T((x.astype(np.float64) / s).astype(np.float32), dt)   # float64 -> f32 -> T: innocuous
        r32 = np.float32(1.0) / np.float32(s)
        prod = (x * r32).astype(np.float32)
        approx = _round_T(prod, dt)
        use = np.abs(prod) >= tiny                    # the kernel divides exactly below this
        bad += int((exact[use] != approx[use]).sum())
    assert bad == 0


def test_fp16_double_rounding_innocuous():
    """R16(R32(a op b)) == R16(a op b) for fp16 a, b (the oracle's and the kernels' 'compute in
    fp32, round to fp16' steps): checked for + - * / on a dense random sample."""
    rng = np.random.default_rng(0)
    a = rng.standard_normal(200000).astype(np.float16)
    b = (rng.standard_normal(200000) * 7).astype(np.float16)
    a64, b64 = a.astype(np.float64), b.astype(np.float64)
    for op in (np.add, np.subtract, np.multiply, np.divide):
        with np.errstate(divide="ignore", invalid="ignore"):
            once = op(a64, b64).astype(np.float16)
            twice = op(a.astype(np.float32), b.astype(np.float32)).astype(np.float16)
        same = (once == twice) | (np.isnan(once) & np.isnan(twice))
        assert same.all(), op


def _elem_max_divisors(dt):
    """em = R_T(ele_max * max_j l2_j) of every configuration the table-driven HBQ kernel takes:
    E2M1..E2M3 elements, l2_sc_bit 0..2, every L2 scheme (src/quantizer.py:745-770)."""
    out = set()
    for ele_max in (6.0, 7.0, 7.5):
        for sc_bit in (0, 1, 2):
            J = 1 << sc_bit
            r = J - 1
            for m in (2.0 ** r, r + 1, 1 + r / 2, 1 + r / J, 1 + (r + 1) / J, 1 + r / (2 * J), 1 + r / (4 * J)):
                out.add(float(_round_T(np.array([ele_max * m], np.float64).astype(np.float32), dt)[0]))
    return sorted(out)


@pytest.mark.parametrize("dt", [torch.float16, torch.bfloat16])
def test_elem_max_reciprocal(dt):
    """The table kernel's L1 scale input R_T(amax * R32(1/em)), clamped to [2^-14, 61440] as the
    kernel does, equals the reference's R_T(amax / em) clamped, for every non-negative T value amax
    and every element-max divisor em."""
    a = _values(dt)
    a = a[a >= 0]
    for em in _elem_max_divisors(dt):
        exact = _round_T((a.astype(np.float64) / em).astype(np.float32), dt)
        approx = _round_T((a * (np.float32(1.0) / np.float32(em))).astype(np.float32), dt)
        lo, hi = np.float32(2.0 ** -14), np.float32(61440.0)
        assert np.array_equal(np.clip(exact, lo, hi), np.clip(approx, lo, hi)), em


def test_fp16_single_rounding_reciprocal_product():
    """R16 of the exact product x * R32(1/s) (one rounding, as v_fma_mix computes it) equals
    R16(x / s) for every fp16 x and every E5M3 scale s, wherever the quotient is not in the
    fp16 subnormal range (the NVFP element path of the table-driven MXFP kernel)."""
    x = _values(torch.float16).astype(np.float64)
    bad = 0
    for s in [(1 + m / 8) * 2.0 ** e for e in range(-14, 16) for m in range(8)]:
        r = np.float64(np.float32(1.0) / np.float32(s))
        exact = _round_T((x / s).astype(np.float32), torch.float16)   # float64 quotient -> f32 -> f16: innocuous
        once = (x * r).astype(np.float16).astype(np.float32)   # exact float64 product, one rounding to fp16
        use = np.abs(x * r) >= 2.0 ** -14
        bad += int((exact[use] != once[use]).sum())
    assert bad == 0
