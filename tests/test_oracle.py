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
def test_hbq_golden(oracle, golden_hbq, golden_extra, name, inp):
    key = f"{name}_{inp}"
    fx = golden_hbq if key in golden_hbq.files else golden_extra
    dt = "bf16" if inp == "bf16" else "f16"
    r = oracle.hbq_qdq(golden_hbq[f"x_{inp}"], dt, block_size=128, use_quant_kernel=False, **HBQCFG[name])
    assert mismatches(r["y"], fx[key], dt) == 0
    assert mismatches(r["l1"], fx[key + "_l1"], dt) == 0
    assert np.array_equal(r["l2idx"], fx[key + "_l2idx"])
    assert np.array_equal(r["scheme"], fx[key + "_scheme"])
    assert mismatches(r["l2val"], fx[key + "_l2val"], dt) == 0


def test_hbq_golden_ragged(oracle, golden_hbq):
    r = oracle.hbq_qdq(golden_hbq["x_ragged_f16"], "f16", block_size=128, use_quant_kernel=False,
                       **HBQCFG["hbq_a_act"])
    assert mismatches(r["y"], golden_hbq["hbq_a_act_ragged_f16"], "f16") == 0


@pytest.mark.parametrize("dt", ["f16", "bf16"])
@pytest.mark.parametrize("em", [(2, 1), (2, 2), (2, 5)])
def test_elem_quant_compiled_golden_exhaustive(oracle, golden_compiled, golden_elem, dt, em):
    """The torch.compile'd make_fp_quant (GLOBAL_FP_QUANT_CACHE, src/quantizer.py:38-63) over
    every 16-bit pattern.  It differs from the eager function on exactly the values whose
    |m| + 0.5004 rounds across an integer in T but not in fp32: per format 3 positive fp16
    values (and their negatives), 1 bf16 value (and its negative)."""
    key = f"elem_{dt}_e{em[0]}m{em[1]}"
    assert not bool(golden_compiled["compile_fell_back"])
    y = oracle.elem_quant(ALL16, dt, *em, compiled=True)
    assert mismatches(y, golden_compiled[key], dt) == 0
    diff = mismatches(golden_compiled[key], golden_elem[key], dt)
    assert diff == (6 if dt == "f16" else 2)
    # the eager rule would fail here: the compiled oracle is not the eager one renamed
    assert mismatches(oracle.elem_quant(ALL16, dt, *em), golden_compiled[key], dt) == diff


@pytest.mark.parametrize("name", list(HBQCFG))
@pytest.mark.parametrize("inp", ["f16", "f16w", "bf16"])
def test_hbq_compiled_golden(oracle, golden_compiled, golden_hbq, name, inp):
    """HBQQuantizer(use_quant_kernel=True).q, what PTQ builds for every HBQ quantizer
    (src/ptq.py:144-157,198-211; src/quantizer.py:468-469,724)."""
    key = f"{name}_{inp}"
    dt = "bf16" if inp == "bf16" else "f16"
    r = oracle.hbq_qdq(golden_hbq[f"x_{inp}"], dt, block_size=128, use_quant_kernel=True, **HBQCFG[name])
    assert mismatches(r["y"], golden_compiled[key], dt) == 0
    assert mismatches(r["l1"], golden_compiled[key + "_l1"], dt) == 0
    assert np.array_equal(r["l2idx"], golden_compiled[key + "_l2idx"])
    assert np.array_equal(r["scheme"], golden_compiled[key + "_scheme"])


def test_hbq_compiled_differs_from_eager(golden_compiled, golden_hbq):
    """How many HBQ outputs the element rule changes on the fixture tensors (32 x 1024 each).
    Both rules are real: the reference picks one by use_quant_kernel."""
    total = 0
    for name in HBQCFG:
        for inp in ("f16", "f16w", "bf16"):
            key = f"{name}_{inp}"
            if key in golden_hbq.files:
                dt = "bf16" if inp == "bf16" else "f16"
                total += mismatches(golden_compiled[key], golden_hbq[key], dt)
    assert total > 0
    print("HBQ outputs that differ between the compiled and eager element rule:", total)


@pytest.mark.parametrize("name", ["mxfp4", "mxfp8", "nvfp4"])
def test_mxfp_compiled_golden(oracle, golden_compiled, golden_mxfp, name):
    """MXFPQuantizer(activate_dynamo=True).q (src/quantizer.py:464-466)."""
    y, _ = oracle.mxfp_qdq(golden_mxfp["x_f16"], "f16", compiled=True, **MXCFG[name])
    assert mismatches(y, golden_compiled[f"{name}_f16"], "f16") == 0
    y, _ = oracle.mxfp_qdq(golden_mxfp["x_f32"], "f32", compiled=True, **MXCFG[name])
    assert mismatches(y, golden_compiled[f"{name}_f32"], "f32") == 0


def _tensor_scale(x, ebit, mbit, sc_ebit, sc_mbit):
    """MXFPQuantizer.q's per-tensor scale (src/quantizer.py:516-524): a Python float."""
    ele_max = {1: 6.0, 2: 7.0, 5: 7.875}[mbit]
    sc_max = 61440.0 if (sc_ebit, sc_mbit) == (5, 3) else 2.0 ** ((1 << (sc_ebit - 1)) - 1)
    x_max = float(np.abs(x).max())
    return 1.0 if x_max == 0 else x_max / (ele_max * sc_max)


@pytest.mark.parametrize("name", ["nvfp4", "mxfp4"])
def test_mxfp_per_tensor_scale_golden(oracle, golden_extra, name):
    """The per_tensor_scale=True branch (src/quantizer.py:516-524,535-536), off in every
    configuration but part of the interface."""
    for dt, key in (("f16", "x_f16"), ("f32", "x_f32"), ("f16", "x_zero_f16")):
        xb = golden_extra[key]
        ts = _tensor_scale(as_float(xb, dt), 2, MXCFG[name]["mbit"], MXCFG[name]["sc_ebit"], MXCFG[name]["sc_mbit"])
        y, _ = oracle.mxfp_qdq(xb, dt, tensor_scale=ts, **MXCFG[name])
        ref = golden_extra[f"{name}_pts_zero_f16" if key == "x_zero_f16" else f"{name}_pts_{dt}"]
        assert mismatches(y, ref, dt) == 0, (name, key)


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


@pytest.mark.parametrize("compiled", [False, True])
def test_hbq_without_l2_equals_nvfp(oracle, compiled):
    """HBQ with one L2 candidate (l2_sc_bit=0, factor 1) is the FP-scale MX path: both run
    fp_quant(clip(amax / ele_max)) and the same element rounding (src/quantizer.py:505-509, 736-738)."""
    x = to_bits(synth(32, 512, 3, "f16"))
    h = oracle.hbq_qdq(x, "f16", block_size=128, ebit=2, mbit=1, l2_block_size=4, l2_sc_bit=0, l2_scheme="PoT",
                       use_quant_kernel=compiled)
    y, s = oracle.mxfp_qdq(x, "f16", block_size=128, ebit=2, mbit=1, sc_ebit=5, sc_mbit=3, compiled=compiled)
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
                q = as_float(oracle.elem_quant(to_bits(u), "f16", 2, 1, compiled=True), "f16")
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


def _partials_gemm(partials, gk, tail=None):
    """A [1, K] and B [K, N] whose K groups of gk have the given fp32 partials per column:
    A = 1 and one nonzero B entry per (group, column).  Every partial must be an fp16 value,
    so each group partial is exact whatever the sum order inside the group.  tail: length
    of a ragged last group (K = (G - 1) gk + tail)."""
    P = np.asarray(partials, np.float64)
    G, N = P.shape
    K = (G - 1) * gk + (tail if tail else gk)
    A = np.ones((1, K))
    B = np.zeros((K, N))
    for g in range(G):
        B[g * gk] = P[g]
    assert np.array_equal(np.float16(B).astype(np.float64), B)
    return _h(A), _h(B)


def test_grouped_cross_group_sum_is_fp16(oracle):
    """Group partials 2048, 1, 1: the fp16 running sum gives 2048 (2048 + 1 is a tie that
    rounds to even, twice); an fp32 running sum, or one sum rounded at the end, gives 2050
    (gemm.cu:354-377: H = R16(H + R16(P)) per group in ascending order)."""
    for gk in (16, 32, 64, 128):
        A, B = _partials_gemm([[2048.0], [1.0], [1.0]], gk)
        assert as_float(oracle.gemm_fp16_grouped_accum(A, B, gk), "f16")[0, 0] == 2048.0
    # and a tail group of 8 after two full groups of 16 is its own group: merging it into
    # group 1 (partials 2048, 2) would give 2050
    A, B = _partials_gemm([[2048.0], [1.0], [1.0]], 16, tail=8)
    assert as_float(oracle.gemm_fp16_grouped_accum(A, B, 16), "f16")[0, 0] == 2048.0


def test_grouped_partial_rounded_before_add(oracle):
    """Partials 2050 then 2049: R16(2049) = 2048 (tie to even) and 2050 + 2048 = 4098 is a
    tie that rounds to 4096.  Adding the unrounded 2049 (4099) would round to 4100, and so
    would an fp32 running sum."""
    gk = 32
    # 2049 is not an fp16 value: group 1 holds 2048 + 1 (two B entries, exact in fp32)
    K = 2 * gk
    A = np.ones((1, K))
    B = np.zeros((K, 1))
    B[0, 0] = 2050.0
    B[gk, 0] = 2048.0
    B[gk + 1, 0] = 1.0
    C = as_float(oracle.gemm_fp16_grouped_accum(_h(A), _h(B), gk), "f16")[0, 0]
    assert C == 4096.0


def test_fp32_accum_is_sequential_fp32(oracle):
    """gemm_fp32_accum keeps one fp32 accumulator over ascending k (gemm.cu:96-303).  fp16 x
    fp16 products are exact in fp32 (22 significant bits), so fusing the multiply cannot
    change a step; what this pins is the fp32 accumulator and the order:
    4 x 2^22, then 1, 1, then 4 x -2^22: 2^24 + 1 is a tie that stays 2^24, twice, so the sum
    is 0.  Exact or double accumulation gives 2, and so does the descending order."""
    a = np.array([2048.0] * 4 + [1.0, 1.0] + [2048.0] * 4)
    b = np.array([2048.0] * 4 + [1.0, 1.0] + [-2048.0] * 4)
    A, B = _h(a[None, :]), _h(b[:, None])
    assert as_float(oracle.gemm_fp32_accum(A, B), "f16")[0, 0] == 0.0
    A, B = _h(a[None, ::-1]), _h(b[::-1, None])
    assert as_float(oracle.gemm_fp32_accum(A, B), "f16")[0, 0] == 2.0


def test_mxint8_multi_group_known_answer(oracle):
    """Two groups of gk = 64, GN = 4, through the whole GEMM (gemm.cu:1198-1277).
    Group 0 partials [100.75, -3.5, 2.5, 0.5]: s = 2^(ilogb(100.75) - 6) = 1, rne -> [101, -4, 2, 0].
    Group 1 partials [1000, 1, -1020, 4]: s = 2^(9 - 6) = 8; -1020/8 = -127.5 -> -128 -> clamp
    -127 -> -1016; 1/8 and 4/8 -> 0.  H = [1101, -4, -1014, 0].  Quantizing the running sum
    instead (max 1101, s = 16) would give [1104, 0, -1024, 0]."""
    A, B = _partials_gemm([[100.75, -3.5, 2.5, 0.5], [1000.0, 1.0, -1020.0, 4.0]], 64)
    C = as_float(oracle.gemm_blockquant_mxint8(A, B, 64, 4), "f16")[0]
    assert list(C) == [1101.0, -4.0, -1014.0, 0.0]


def test_mxfp8_multi_group_known_answer(oracle):
    """Two groups of gk = 64, GN = 4 (gemm.cu:669-745, 1040-1135).
    Group 0 [10, 1.03125, 0.2001953125, -0.00390625]: s = 2^(3 - 3) = 1; 10 -> 10,
    1.03125 -> 1 (mantissa 0.5 rounds to even 0), 0.2002 -> 13/64, 2^-8 < 2^-7 -> +0.
    Group 1 [-20, 0.375, 100, 3]: s = 2^(6 - 3) = 8; each value is on the E3M4 grid there.
    H = [-10, 1.375, R16(0.203125 + 100) = 100.1875, 3]."""
    P = [[10.0, 1.03125, 0.2001953125, -0.00390625], [-20.0, 0.375, 100.0, 3.0]]
    A, B = _partials_gemm(P, 64)
    C = as_float(oracle.gemm_blockquant_mxfp8(A, B, 64, 4), "f16")[0]
    assert list(C) == [-10.0, 1.375, 100.1875, 3.0]


@pytest.mark.parametrize("op", ["fp32", "fp16", "grouped", "mxint8", "mxfp8"])
def test_gemm_oracle_within_float64_bound(oracle, op):
    """Every oracle GEMM against the float64 product, within the bound its rounding steps
    allow (S = sum_k |a_k b_k| per output, G groups, u_h = 2^-11, u_f = 2^-24):
      fp32:    K u_f S + u_h |C|                        (fp32 chain, one fp16 rounding)
      fp16:    K u_h S                                  (one fp16 rounding per step)
      grouped: (gk u_f + (2G + 1) u_h) S                (partials, their fp16 roundings, the adds)
      mxint8/mxfp8: the grouped bound plus G times half the psum step, max|P_g| 2^-7
               (int8: s/2 = 2^(ilogb - 7)) or 2^-5 (E3M4: 2^(ilogb - 3) spacing / 2 at 15.5).
    A transposed operand, a dropped group or a wrong scale breaks the bound by orders of
    magnitude on this data."""
    rng = np.random.default_rng(5)
    M, K, N, gk, gn = 8, 512, 64, 128, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    B = (rng.standard_normal((K, N)) * 0.05).astype(np.float16)
    Ab, Bb = A.view(np.uint16), B.view(np.uint16)
    Ad, Bd = A.astype(np.float64), B.astype(np.float64)
    ref = Ad @ Bd
    S = np.abs(Ad) @ np.abs(Bd)
    G = K // gk
    uh, uf = 2.0 ** -11, 2.0 ** -24
    if op == "fp32":
        C, bound = oracle.gemm_fp32_accum(Ab, Bb), K * uf * S + uh * np.abs(ref)
    elif op == "fp16":
        C, bound = oracle.gemm_fp16_accum(Ab, Bb), K * uh * S
    else:
        bound = (gk * uf + (2 * G + 1) * uh) * S
        if op == "grouped":
            C = oracle.gemm_fp16_grouped_accum(Ab, Bb, gk)
        else:
            P = np.stack([Ad[:, g * gk:(g + 1) * gk] @ Bd[g * gk:(g + 1) * gk] for g in range(G)])
            pmax = np.abs(P).reshape(G, M, N // gn, gn).max(-1).repeat(gn, axis=-1).sum(0)
            step = 2.0 ** -7 if op == "mxint8" else 2.0 ** -5
            bound = bound + step * pmax * 1.01
            f = oracle.gemm_blockquant_mxint8 if op == "mxint8" else oracle.gemm_blockquant_mxfp8
            C = f(Ab, Bb, gk, gn)
    err = np.abs(as_float(C, "f16").astype(np.float64) - ref)
    assert np.all(err <= bound), float((err / bound).max())
    # the bound is not vacuous: a transposed B (square blocks) lands far outside it
    if op == "grouped":
        Bt = np.ascontiguousarray(B[:N, :].T.astype(np.float16))
        Bt = np.concatenate([Bt] * (K // N), axis=0).astype(np.float16)
        Cbad = as_float(oracle.gemm_fp16_grouped_accum(Ab, Bt.view(np.uint16), gk), "f16")
        assert np.any(np.abs(Cbad.astype(np.float64) - ref) > bound)


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


def test_group_partials_loop_order_is_per_output_chain(oracle):
    """orc_group_partials runs k outside n for speed; each output must still be the
    per-output sequential chain, bit for bit, including a ragged tail group."""
    rng = np.random.default_rng(3)
    A = (rng.standard_normal((3, 200)) * 4).astype(np.float16)
    B = (rng.standard_normal((200, 5)) * 0.1).astype(np.float16)
    P = oracle.group_partials(A.view(np.uint16), B.view(np.uint16), 64)
    for g in range(4):
        for m in range(3):
            for n in range(5):
                one = oracle.group_partial_one(A.view(np.uint16), B.view(np.uint16), m, n, 64 * g, min(64 * g + 64, 200))
                assert np.float32(one) == P[g, m, n]


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
