"""The CPU oracle, pinned: reference goldens, torch library behaviour, closed forms.

Runs without a GPU.  Each check is chosen so that a plausible slip in the
restatement (a dropped rounding step, the wrong rounding constant, a wrong
summation order, a wrong exponent rule) fails it."""
from fractions import Fraction

import numpy as np
import pytest
import torch

from helpers import as_float, mismatches, synth, to_bits, to_torch

ALL16 = np.arange(65536, dtype=np.uint32).astype(np.uint16)

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
}


# ---------------------------------------------------------------------------
# reference goldens (tests/golden/gen_golden.py ran src/quantizer.py)
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("em", [(2, 1), (2, 2), (2, 5)])
def test_elem_quant_golden_exhaustive(oracle, golden_elem, dt, em):
    y = oracle.elem_quant(ALL16, dt, *em)
    assert mismatches(y, golden_elem[f"elem_{dt}_e{em[0]}m{em[1]}"], dt) == 0


@pytest.mark.parametrize("name", list(MXCFG))
def test_mxfp_golden(oracle, golden_mxfp, name):
    y, s = oracle.mxfp_qdq(golden_mxfp["x_f16"], "f16", **MXCFG[name])
    assert mismatches(y, golden_mxfp[f"{name}_f16"], "f16") == 0
    assert mismatches(s, golden_mxfp[f"{name}_f16_scale"], "f16") == 0
    y, _ = oracle.mxfp_qdq(golden_mxfp["x_f32"], "f32", **MXCFG[name])
    assert mismatches(y, golden_mxfp[f"{name}_f32"], "f32") == 0
    if name in ("mxfp4", "nvfp4"):
        y, _ = oracle.mxfp_qdq(golden_mxfp["x_ragged_f16"], "f16", **MXCFG[name])
        assert mismatches(y, golden_mxfp[f"{name}_ragged_f16"], "f16") == 0


@pytest.mark.parametrize("name", list(HBQCFG))
@pytest.mark.parametrize("inp", ["f16", "f16w", "bf16"])
def test_hbq_golden(oracle, golden_hbq, name, inp):
    key = f"{name}_{inp}"
    if key not in golden_hbq:
        pytest.skip("no fixture")
    dt = "bf16" if inp == "bf16" else "f16"
    r = oracle.hbq_qdq(golden_hbq[f"x_{inp}"], dt, block_size=128, **HBQCFG[name])
    assert mismatches(r["y"], golden_hbq[key], dt) == 0
    assert mismatches(r["l1"], golden_hbq[key + "_l1"], dt) == 0
    assert np.array_equal(r["l2idx"], golden_hbq[key + "_l2idx"])
    assert np.array_equal(r["scheme"], golden_hbq[key + "_scheme"])
    assert mismatches(r["l2val"], golden_hbq[key + "_l2val"], dt) == 0


def test_hbq_golden_ragged(oracle, golden_hbq):
    r = oracle.hbq_qdq(golden_hbq["x_ragged_f16"], "f16", block_size=128, **HBQCFG["hbq_a_act"])
    assert mismatches(r["y"], golden_hbq["hbq_a_act_ragged_f16"], "f16") == 0


# ---------------------------------------------------------------------------
# torch library behaviour the reference relies on
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("dt", ["f16", "bf16"])
def test_floor_log2_matches_torch_exhaustive(oracle, dt):
    """floor(R_T(log2 |x|)) for every finite nonzero 16-bit value equals torch's."""
    xt = to_torch(ALL16, dt)
    fin = torch.isfinite(xt) & (xt != 0)
    ref = torch.floor(torch.log2(xt.abs())).float().numpy()
    got = oracle.floor_log2(ALL16, dt)
    assert np.array_equal(got[fin.numpy()], ref[fin.numpy()])


def test_floor_log2_quirk_count(oracle):
    """The R_T rounding makes the exponent one too large just below powers of two."""
    xt = to_torch(ALL16, "f16")
    pos = (torch.isfinite(xt) & (xt > 0)).numpy()
    true_e = np.floor(np.log2(xt.double().numpy()[pos]))
    got = oracle.floor_log2(ALL16, "f16")[pos]
    assert int((got != true_e).sum()) == 94


def _adversarial_column(rng, n):
    """Sums whose fp16 result depends on the fp32 association order: 1025 + (0.5 - 2^-12)
    + four 2^-14 terms is a tie at fp16 only if the small terms meet before the large one."""
    col = np.zeros(n, np.float32)
    pos = rng.permutation(n)[:6]
    col[pos[0]] = 1025.0
    col[pos[1]] = 0.5 - 2.0 ** -12
    col[pos[2:6]] = 2.0 ** -14
    return col


@pytest.mark.parametrize("l2b,S", [(8, 1), (8, 2), (32, 1), (32, 2)])
def test_subblock_sum_order_matches_torch(oracle, l2b, S):
    """sum(dim=-3) over the HBQ candidate error tensor [R, nblk, nsub, l2b, J, S] (src/quantizer.py:802)."""
    rng = np.random.default_rng(l2b * 10 + S)
    R, nblk, J, nsub = 4, 4, 4, 128 // l2b
    v = np.zeros((R, nblk, nsub, l2b, J, S), np.float32)
    for idx in np.ndindex(R, nblk, nsub, J, S):
        v[idx[0], idx[1], idx[2], :, idx[3], idx[4]] = _adversarial_column(rng, l2b)
    ref = torch.from_numpy(v).half().sum(dim=-3).float().numpy()
    bad = 0
    for idx in np.ndindex(R, nblk, nsub, J, S):
        col = v[idx[0], idx[1], idx[2], :, idx[3], idx[4]]
        bad += np.float16(oracle.cascade_sum(col)) != np.float16(ref[idx[0], idx[1], idx[2], idx[3], idx[4]])
    assert bad == 0


@pytest.mark.parametrize("l2b", [8, 32])
def test_scheme_sum_order_matches_torch(oracle, l2b):
    """sum(dim=(-2, -3)) over [R, nblk, nsub, l2b, 2] (src/quantizer.py:814), Mix scheme."""
    rng = np.random.default_rng(l2b)
    R, nblk, nsub = 8, 8, 128 // l2b
    v = np.zeros((R, nblk, nsub, l2b, 2), np.float32)
    for idx in np.ndindex(R, nblk, 2):
        v[idx[0], idx[1], :, :, idx[2]] = _adversarial_column(rng, 128).reshape(nsub, l2b)
    ref = torch.from_numpy(v).half().sum(dim=(-2, -3)).float().numpy()
    bad = 0
    for idx in np.ndindex(R, nblk, 2):
        col = v[idx[0], idx[1], :, :, idx[2]].reshape(-1)
        bad += np.float16(oracle.row_sum(col)) != np.float16(ref[idx])
    assert bad == 0


def test_argmin_first_index():
    """torch.min(dim) returns the first of equal minima (src/quantizer.py:803,815)."""
    _, i = torch.tensor([3.0, 1.0, 1.0, 2.0]).half().min(-1)
    assert int(i) == 1


# ---------------------------------------------------------------------------
# closed forms
# ---------------------------------------------------------------------------
def _e5m3_values():
    out = []
    for e in range(-14, 16):
        for m in range(8):
            out.append((1 + m / 8) * 2.0 ** e)
    return np.array(sorted(out))


@pytest.mark.parametrize("use_ceil", [False, True])
def test_scale_quant_closed_form(oracle, use_ceil):
    """E5M3 scale rounding of every positive normal fp16 value: nearest with ties up (or the
    smallest grid value >= x for ceil), except where floor(R16(log2 x)) exceeds the binade."""
    xt = to_torch(ALL16, "f16").float().numpy()
    sel = np.isfinite(xt) & (xt >= 2.0 ** -14) & (xt <= 61440.0)
    x = xt[sel]
    grid = _e5m3_values()
    hi = np.searchsorted(grid, x, side="left")
    up = grid[np.minimum(hi, len(grid) - 1)]
    lo = grid[np.maximum(hi - 1, 0)]
    exact = grid[np.minimum(hi, len(grid) - 1)] == x
    if use_ceil:
        expect = np.where(exact, x, up)
    else:
        expect = np.where(exact, x, np.where(x - lo >= up - x, up, lo))
    got = as_float(oracle.fp_quant(ALL16[sel], "f16", 5, 3, allow_subnormal=False, use_ceil=use_ceil), "f16")
    quirk = oracle.floor_log2(ALL16[sel], "f16") != np.floor(np.log2(x.astype(np.float64)))
    assert np.array_equal(got[~quirk], expect[~quirk])
    # in the quirk set the value is 2^(e+1) with half-up and 1.125 * 2^(e+1) with ceil
    e1 = 2.0 ** (np.floor(np.log2(x[quirk].astype(np.float64))) + 1)
    assert np.array_equal(got[quirk], e1 * (1.125 if use_ceil else 1.0))


def test_hbq_without_l2_equals_nvfp(oracle):
    """HBQ with one L2 candidate (l2_sc_bit=0, factor 1) is the FP-scale MX path: both run
    fp_quant(clip(amax / ele_max)) and the same element rounding (src/quantizer.py:505-509, 736-738)."""
    x = to_bits(synth(32, 512, 3, "f16"))
    h = oracle.hbq_qdq(x, "f16", block_size=128, ebit=2, mbit=1, l2_block_size=4, l2_sc_bit=0, l2_scheme="PoT")
    y, s = oracle.mxfp_qdq(x, "f16", block_size=128, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3)
    assert mismatches(h["y"], y, "f16") == 0
    assert mismatches(h["l1"], s, "f16") == 0


@pytest.mark.parametrize("name", ["hbq_a_act", "hbq_a_wgt", "hbq_e_wgt"])
def test_hbq_outputs_on_grid(oracle, name):
    """Every output is sign * element * L2 factor * L1 scale of its block (exact in fp16)."""
    cfg = HBQCFG[name]
    x = to_bits(synth(16, 512, 4, "f16"))
    r = oracle.hbq_qdq(x, "f16", block_size=128, **cfg)
    M = cfg["mbit"]
    elems = sorted({k / 2 ** M for k in range(2 ** M)} | {(1 + k / 2 ** M) * 2 ** e for e in range(3)
                                                           for k in range(2 ** M)})
    y = as_float(r["y"], "f16").reshape(16, 4, 128)
    l1 = as_float(r["l1"], "f16")[..., None]
    l2 = np.repeat(as_float(r["l2val"], "f16"), cfg["l2_block_size"], axis=-1)
    ratio = np.abs(y) / (l1 * l2)
    assert np.all(np.isin(ratio, np.array(elems, np.float32)))


def test_hbq_zero_block(oracle):
    x = np.zeros((2, 256), np.uint16)
    x[1, :] = 0x8000                      # -0 inputs give +0 outputs (src/quantizer.py:241-245)
    r = oracle.hbq_qdq(x, "f16", block_size=128, **HBQCFG["hbq_a_act"])
    assert (r["y"] == 0).all()


def test_hbq_choice_is_near_optimal_exactly(oracle):
    """Recompute every candidate's squared error in exact arithmetic: the oracle's L2 pick per
    sub-block and its scheme pick are within fp16 rounding of the exact minimum (the reference
    compares fp16-rounded sums, so near-ties may go either way, but nothing worse)."""
    cfg = HBQCFG["hbq_a_wgt"]
    rows = 6
    x = synth(rows, 128, 9, "f16", std=0.05)
    r = oracle.hbq_qdq(to_bits(x), "f16", block_size=128, **cfg)
    tab = oracle.l2_table("Mix", 2, "f16")
    tol = 1 + 2.0 ** -8
    for row in range(rows):
        xr = x[row].float()
        amax = float(xr.abs().max())
        per_scheme = []
        for s in range(2):
            em = float(np.float16(6.0 * tab[:, s].max()))
            l1 = float(as_float(oracle.fp_quant(to_bits(torch.tensor([max(amax / em, 2.0 ** -14)]).half()),
                                                "f16", 5, 3, False), "f16")[0])
            t = (x[row] / torch.tensor(l1).half())
            errs = np.zeros((16, 4), dtype=object)
            for j in range(4):
                u = t / torch.tensor(float(tab[j, s])).half()
                q = as_float(oracle.elem_quant(to_bits(u), "f16", 2, 1), "f16")
                d = [Fraction(float(v)) * Fraction(float(tab[j, s])) * Fraction(l1) for v in q]
                e2 = [(Fraction(float(a)) - b) ** 2 for a, b in zip(xr.numpy(), d)]
                for u_ in range(16):
                    errs[u_, j] = sum(e2[u_ * 8:(u_ + 1) * 8])
            per_scheme.append(errs)
        s_pick = int(r["scheme"][row, 0])
        errs = per_scheme[s_pick]
        for u_ in range(16):
            best = min(errs[u_])
            assert errs[u_, int(r["l2idx"][row, 0, u_])] <= best * Fraction(tol) + Fraction(1, 2 ** 40)
        totals = [sum(min(e[u_]) for u_ in range(16)) for e in per_scheme]
        assert totals[s_pick] <= min(totals) * Fraction(tol) + Fraction(1, 2 ** 40)


# ---------------------------------------------------------------------------
# GEMM oracle: closed forms and library arithmetic
# ---------------------------------------------------------------------------
def _h(vals):
    return np.asarray(vals, np.float16).view(np.uint16)


def test_gemm_ones_closed_form(oracle):
    """A = B = 1: each group partial is its length; fp16 sums of group partials are exact here."""
    M, K, N = 3, 300, 5
    A = _h(np.ones((M, K)))
    B = _h(np.ones((K, N)))
    for gk in (16, 32, 64, 128):
        C = as_float(oracle.gemm_fp16_grouped_accum(A, B, gk), "f16")
        assert np.all(C == K)
    assert np.all(as_float(oracle.gemm_fp32_accum(A, B), "f16") == K)


def test_grouped_fp16_rounding_closed_form(oracle):
    """Group partials 2049 (fp16 rounds to 2048 then 2048 + 2048 ...): the grouped result is
    the fp16 running sum of fp16-rounded partials, not the exact total."""
    K, gk = 3 * 128, 128
    A = _h(np.full((1, K), 16.0))
    B = np.full((K, 1), 1.0)
    B[0] = 17.0                                 # group 0: 16*127 + 16*17 = 2304; others 2048
    C = as_float(oracle.gemm_fp16_grouped_accum(A, _h(B), gk), "f16")[0, 0]
    h = np.float16(0)
    for p in (2304.0, 2048.0, 2048.0):
        h = np.float16(h + np.float16(p))
    assert C == float(h)


def test_mxint8_epilogue_known_answer(oracle):
    """One group, GN=4: max |P| = 100.7 -> s = 2^(6-6) = 1; q = rne(P) clamped to +-127."""
    P = np.array([[[100.7, -3.5, 2.5, 0.49]]], np.float32)
    C = as_float(oracle.epilogue(P, "mxint8", 4), "f16")[0]
    assert list(C) == [101.0, -4.0, 2.0, 0.0]
    P = np.array([[[1000.0, 1.0, -1023.9, 4.0]]], np.float32)    # ilogb 9 -> s = 8; -1023.9/8 -> -128 -> -127; 4/8 = 0.5 -> 0
    C = as_float(oracle.epilogue(P, "mxint8", 4), "f16")[0]
    assert list(C) == [1000.0, 0.0, -1016.0, 0.0]


def test_mxfp8_epilogue_known_answer(oracle):
    """E3M4 with s = 2^(ilogb(max) - 3): max 10 -> s = 1; 10 -> 10, 1.03 -> 1.0, 0.2 -> 0.203125."""
    P = np.array([[[10.0, 1.03, 0.2, -0.004]]], np.float32)
    C = as_float(oracle.epilogue(P, "mxfp8", 4), "f16")[0]
    assert C[0] == 10.0 and C[1] == 1.0 and C[2] == np.float16(13 / 64) and C[3] == 0.0


def test_fp16_chain_is_fused(oracle):
    """gemm_fp16_accum rounds a*b + acc once per step: exact rational arithmetic agrees."""
    rng = np.random.default_rng(0)
    A = (rng.standard_normal((4, 40)) * 3).astype(np.float16)
    B = (rng.standard_normal((40, 3)) * 3).astype(np.float16)
    C = as_float(oracle.gemm_fp16_accum(A.view(np.uint16), B.view(np.uint16)), "f16")
    for m in range(4):
        for n in range(3):
            h = np.float16(0)
            for k in range(40):
                exact = Fraction(float(A[m, k])) * Fraction(float(B[k, n])) + Fraction(float(h))
                h = np.float16(float(exact))      # float(exact) is RN to double; exact has < 53 bits here
            assert C[m, n] == float(h)


def test_group_partials_sequential_fmaf(oracle):
    """Group partials equal a sequential fused fp32 chain (fmaf via exact rationals)."""
    rng = np.random.default_rng(1)
    A = rng.standard_normal((2, 64)).astype(np.float16)
    B = rng.standard_normal((64, 2)).astype(np.float16)
    P = oracle.group_partials(A.view(np.uint16), B.view(np.uint16), 32)
    for g in range(2):
        for m in range(2):
            for n in range(2):
                p = np.float32(0)
                for k in range(g * 32, g * 32 + 32):
                    p = np.float32(float(Fraction(float(A[m, k])) * Fraction(float(B[k, n])) + Fraction(float(p))))
                assert P[g, m, n] == p
