"""GPU parity of the blockquant_ext GEMMs against the CPU oracle (restatement of gemm.cu).

* Exact-integer inputs: every partial sum is exactly representable, so the MFMA
  summation order cannot matter and the whole GEMM must match bit for bit.
* Epilogues: the fused per-group epilogue applied by the kernel must equal the
  oracle's epilogue applied to the kernel's own fp32 group partials, bit for bit.
* General fp16 inputs: the in-group fp32 sums come from MFMA instead of a
  sequential fmaf chain, so outputs agree to a normwise relative tolerance of
  1e-3 (a one-ulp difference in a partial can move a psum-quantized value by
  one int8 step, so an elementwise bound would be meaningless there).
"""
import numpy as np
import pytest
import torch

from helpers import mismatches, synth, to_bits, to_torch

pytestmark = pytest.mark.gpu


def _ext():
    from hbq_amd import blockquant_ext
    return blockquant_ext


def exact_inputs(M, K, N, seed):
    """Small integers times 1/4 and 1/2: products are multiples of 1/8 below 2^9, so
    group sums over <= 256 terms stay below 2^17 and are exact in fp32."""
    g = torch.Generator().manual_seed(seed)
    A = torch.randint(-15, 16, (M, K), generator=g).half() * 0.25
    B = torch.randint(-15, 16, (K, N), generator=g).half() * 0.5
    return A, B


def b16(t):
    return to_bits(t)


SHAPES = [(128, 256, 128), (200, 320, 136), (64, 1024, 256), (256, 128, 512)]


@pytest.mark.parametrize("shape", SHAPES)
@pytest.mark.parametrize("nk", [False, True])
def test_exact_all_ops(gpu, oracle, shape, nk):
    M, K, N = shape
    print(f"exact ops shape={shape} nk={nk}", flush=True)
    A, B = exact_inputs(M, K, N, 1)
    ext = _ext()
    Ad, Bd = A.to(gpu), (B.t().contiguous() if nk else B).to(gpu)
    a, b = b16(A), b16(B)
    assert mismatches(b16(ext.gemm_fp32_accum(Ad, Bd, b_is_nk=nk)), oracle.gemm_fp32_accum(a, b), "f16") == 0
    for gk in (16, 32, 64, 128):
        got = ext.gemm_fp16_grouped_accum(Ad, Bd, gk, b_is_nk=nk)
        assert mismatches(b16(got), oracle.gemm_fp16_grouped_accum(a, b, gk), "f16") == 0, gk
    for gk in (64, 128, 256):
        if K % gk:
            continue
        for gn in (4, 8, 16, 32):
            if N % gn:
                continue
            got = ext.gemm_blockquant_mxint8(Ad, Bd, gk, gn, b_is_nk=nk)
            assert mismatches(b16(got), oracle.gemm_blockquant_mxint8(a, b, gk, gn), "f16") == 0, (gk, gn)
            got = ext.gemm_blockquant_mxfp8(Ad, Bd, gk, gn, b_is_nk=nk)
            assert mismatches(b16(got), oracle.gemm_blockquant_mxfp8(a, b, gk, gn), "f16") == 0, (gk, gn)


@pytest.mark.parametrize("shape", [(96, 64, 72), (130, 200, 64)])
def test_fp16_accum_exact_chain(gpu, oracle, shape):
    """Pure fp16 accumulation: a fused fp16 FMA per k, in order -> bit-exact for any input."""
    M, K, N = shape
    A = synth(M, K, 3, "f16", outliers=0)
    B = synth(K, N, 4, "f16", std=0.3, outliers=0)
    got = _ext().gemm_fp16_accum(A.to(gpu), B.to(gpu))
    assert mismatches(b16(got), oracle.gemm_fp16_accum(b16(A), b16(B)), "f16") == 0


@pytest.mark.parametrize("mode,gk,gn", [("grouped", 128, 0), ("grouped", 16, 0), ("mxint8", 128, 32),
                                        ("mxint8", 64, 4), ("mxint8", 256, 16), ("mxfp8", 128, 32),
                                        ("mxfp8", 64, 8)])
@pytest.mark.parametrize("nk", [False, True])
def test_epilogue_bitexact_on_kernel_partials(gpu, oracle, mode, gk, gn, nk):
    """The fused epilogue equals the reference epilogue on the kernel's own group partials."""
    print(f"epilogue {mode} gk={gk} gn={gn} nk={nk}", flush=True)
    M, K, N = 256, 512, 384
    A = synth(M, K, 21, "f16")
    B = synth(K, N, 22, "f16", std=0.02)
    ext = _ext()
    Ad, Bd = A.to(gpu), (B.t().contiguous() if nk else B).to(gpu)
    P = ext.group_partials(Ad, Bd, gk, b_is_nk=nk).cpu().numpy()
    if mode == "grouped":
        got = ext.gemm_fp16_grouped_accum(Ad, Bd, gk, b_is_nk=nk)
    elif mode == "mxint8":
        got = ext.gemm_blockquant_mxint8(Ad, Bd, gk, gn, b_is_nk=nk)
    else:
        got = ext.gemm_blockquant_mxfp8(Ad, Bd, gk, gn, b_is_nk=nk)
    ref = oracle.epilogue(P, mode, gn)
    assert mismatches(b16(got), ref, "f16") == 0


def _rel_err(got, ref):
    """Normwise relative error ||got - ref||_F / ||ref||_F, and the fraction of differing elements."""
    g = to_torch(b16(got), "f16").double()
    r = to_torch(ref, "f16").double()
    return ((g - r).norm() / r.norm().clamp_min(1e-30)).item(), (b16(got) != ref).mean()


@pytest.mark.parametrize("op", ["fp32", "grouped", "mxint8"])
def test_general_inputs_tolerance(gpu, oracle, op):
    """N(0,1) activations with outlier channels against N(0, 0.02) weights (configs[2..3] statistics)."""
    M, K, N = 256, 1024, 512
    A = synth(M, K, 31, "f16")
    B = synth(K, N, 32, "f16", std=0.02, outliers=0, laplace_frac=0)
    ext = _ext()
    Ad, Bd = A.to(gpu), B.to(gpu)
    if op == "fp32":
        got, ref = ext.gemm_fp32_accum(Ad, Bd), oracle.gemm_fp32_accum(b16(A), b16(B))
    elif op == "grouped":
        got, ref = ext.gemm_fp16_grouped_accum(Ad, Bd, 128), oracle.gemm_fp16_grouped_accum(b16(A), b16(B), 128)
    else:
        got, ref = ext.gemm_blockquant_mxint8(Ad, Bd, 128, 32), oracle.gemm_blockquant_mxint8(b16(A), b16(B), 128, 32)
    rel, frac = _rel_err(got, ref)
    print(f"{op}: normwise rel err {rel:.2e}, differing elements {frac:.4%}", flush=True)
    assert rel <= 1e-3


def test_hbq_quantized_operands_match(gpu, oracle):
    """HBQ-E quantized activations and weights (configs[3] pipeline at reduced size): psum GEMM vs oracle."""
    from hbq_amd.quantizer import HBQQuantizer
    M, K, N = 512, 1024, 512
    X = synth(M, K, 41, "f16")
    W = synth(N, K, 42, "f16", std=0.02, outliers=0)
    qa = HBQQuantizer(block_size=128, ebit=2, mbit=2, l2_block_size=32, l2_sc_bit=2, l2_scheme="SIG-1")
    qw = HBQQuantizer(block_size=128, ebit=2, mbit=1, l2_block_size=32, l2_sc_bit=2, l2_scheme="Mix")
    Xq = qa.q(X.to(gpu))
    Wq = qw.q(W.to(gpu))
    got = _ext().gemm_blockquant_mxint8_nk(Xq, Wq, 128, 32)
    ref = oracle.gemm_blockquant_mxint8(b16(Xq), b16(Wq.t().contiguous()), 128, 32)
    rel, frac = _rel_err(got, ref)
    print(f"HBQ-E operands: normwise rel err {rel:.2e}, differing elements {frac:.4%}", flush=True)
    assert rel <= 1e-3


def test_error_messages(gpu):
    ext = _ext()
    a = torch.zeros(4, 128, dtype=torch.float16, device=gpu)
    b = torch.zeros(128, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(RuntimeError, match="A must be fp16"):
        ext.gemm_fp32_accum(a.float(), b)
    with pytest.raises(RuntimeError, match="A and B must be 2D"):
        ext.gemm_fp32_accum(a[None], b)
    with pytest.raises(RuntimeError, match="K dimension"):
        ext.gemm_fp32_accum(a, b[:64])
    with pytest.raises(RuntimeError, match=r"group_k must be one of \{16,32,64,128\}"):
        ext.gemm_fp16_grouped_accum(a, b, 256)
    with pytest.raises(RuntimeError, match=r"group_k must be one of \{64,128,256\}"):
        ext.gemm_blockquant_mxint8(a, b, 32, 32)
    with pytest.raises(RuntimeError, match=r"group_n must be one of \{4,8,16,32\}"):
        ext.gemm_blockquant_mxint8(a, b, 128, 64)
    with pytest.raises(RuntimeError, match="K must be divisible by group_k"):
        ext.gemm_blockquant_mxfp8(a[:, :64], b[:64], 128, 32)
    with pytest.raises(RuntimeError, match="N must be divisible by group_n"):
        ext.gemm_blockquant_mxint8(a, b[:, :60], 128, 8)


def test_zero_and_empty(gpu):
    ext = _ext()
    z = ext.gemm_fp16_grouped_accum(torch.zeros(3, 0, dtype=torch.float16, device=gpu),
                                    torch.zeros(0, 5, dtype=torch.float16, device=gpu), 128)
    assert z.shape == (3, 5) and (b16(z) == 0).all()
    a = torch.zeros(64, 128, dtype=torch.float16, device=gpu)
    b = -torch.zeros(128, 64, dtype=torch.float16, device=gpu)
    for C in (ext.gemm_fp32_accum(a, b), ext.gemm_fp16_grouped_accum(a, b, 128),
              ext.gemm_blockquant_mxint8(a, b, 128, 32), ext.gemm_blockquant_mxfp8(a, b, 128, 32)):
        assert (b16(C) == 0).all()   # +0, as the reference's zero-initialised accumulators give


def test_fp16accum_matmul_module(gpu, oracle):
    """FP16AccumMatMul (src/ops.py) dispatch: psum-quantized, grouped, and bias."""
    from hbq_amd.ops import FP16AccumMatMul
    A, B = exact_inputs(64, 256, 96, 5)
    W = B.t().contiguous()
    bias = torch.randn(96).half()
    x = A.view(2, 32, 256).to(gpu)
    y = FP16AccumMatMul(128, 32)(x, W.to(gpu), bias.to(gpu))
    ref = to_torch(oracle.gemm_blockquant_mxint8(b16(A), b16(B), 128, 32), "f16") + bias
    assert y.shape == (2, 32, 96)
    assert mismatches(b16(y.view(64, 96)), b16(ref), "f16") == 0
    y = FP16AccumMatMul(128)(x, W.to(gpu))
    assert mismatches(b16(y.view(64, 96)), oracle.gemm_fp16_grouped_accum(b16(A), b16(B), 128), "f16") == 0
    with pytest.raises(ValueError):
        FP16AccumMatMul(256, 32)(x, W.to(gpu))
    with pytest.raises(ValueError):
        FP16AccumMatMul(128, 64)(x, W.to(gpu))


@pytest.mark.parametrize("op", ["fp32", "grouped", "mxint8", "mxfp8"])
def test_kn_and_nk_layouts_bit_identical(gpu, op):
    """B[K,N] through the 128x128 kernel, W[N,K] through the 256x256 kernel, and B[K,N]
    transposed to W[N,K] by the op: the same bits (same MFMA sequence per output)."""
    from hbq_amd import blockquant_ext as ext
    M, K, N = 320, 1024, 384
    A = synth(M, K, 41, "f16").to(gpu)
    B = synth(K, N, 42, "f16", std=0.02, outliers=0, laplace_frac=0).to(gpu)
    W = B.t().contiguous()
    call = {"fp32": lambda b, nk: ext.gemm_fp32_accum(A, b, b_is_nk=nk),
            "grouped": lambda b, nk: ext.gemm_fp16_grouped_accum(A, b, 128, b_is_nk=nk),
            "mxint8": lambda b, nk: ext.gemm_blockquant_mxint8(A, b, 128, 32, b_is_nk=nk),
            "mxfp8": lambda b, nk: ext.gemm_blockquant_mxfp8(A, b, 64, 16, b_is_nk=nk)}[op]
    old = ext.TRANSPOSE_MIN_MNK
    try:
        ext.TRANSPOSE_MIN_MNK = 1 << 62
        kn = call(B, False)
        ext.TRANSPOSE_MIN_MNK = 0
        kn_t = call(B, False)
    finally:
        ext.TRANSPOSE_MIN_MNK = old
    nk = call(W, True)
    assert torch.equal(kn.view(torch.int16), nk.view(torch.int16))
    assert torch.equal(kn_t.view(torch.int16), nk.view(torch.int16))


@pytest.mark.parametrize("shape", [(1, 1), (7, 130), (64, 64), (200, 72), (4096, 136), (96, 1000)])
def test_transpose16(gpu, shape):
    """The B[K,N] -> W[N,K] helper: exact copy, ragged and unaligned shapes included."""
    from hbq_amd import _lib
    rows, cols = shape
    g = torch.Generator(device=gpu).manual_seed(rows * 1000 + cols)
    src = torch.randint(-32768, 32767, (rows, cols), device=gpu, dtype=torch.int32, generator=g).to(torch.int16)
    dst = torch.empty((cols, rows), device=gpu, dtype=torch.int16)
    _lib.check(_lib.lib().hbq_transpose16(_lib.ptr(src), _lib.ptr(dst), rows, cols, _lib.stream_of(src)))
    assert torch.equal(dst, src.t())


@pytest.mark.parametrize("op,gk,gn", [("fp32", 0, 0), ("grouped", 128, 0), ("mxint8", 128, 32), ("mxint8", 256, 16),
                                      ("mxint8", 128, 4), ("mxfp8", 128, 32), ("mxfp8", 256, 8)])
@pytest.mark.parametrize("K", [256, 512])
@pytest.mark.parametrize("M", [4000, 2000])
def test_large_tile_kernel_bit_identical(gpu, op, gk, gn, K, M):
    """At shapes with enough 256-row tiles to fill the chip W[N,K] runs on the 256-row kernel:
    256 x 256 tiles at M = 4000 (16 x 16 tiles), 256 x 128 tiles at M = 2000 (8 x 32; 256-wide
    tiles would give only 128), the last tile row ragged in both.  B[K,N] without the transpose
    runs on the 128x128 kernel that the oracle tests pin: the same bits."""
    from hbq_amd import blockquant_ext as ext
    N = 4096
    print(f"large tiles {op} gk={gk} gn={gn} K={K} M={M}", flush=True)
    A = synth(M, K, 51, "f16").to(gpu)
    B = synth(K, N, 52, "f16", std=0.02).to(gpu)
    W = B.t().contiguous()
    call = {"fp32": lambda b, nk: ext.gemm_fp32_accum(A, b, b_is_nk=nk),
            "grouped": lambda b, nk: ext.gemm_fp16_grouped_accum(A, b, gk, b_is_nk=nk),
            "mxint8": lambda b, nk: ext.gemm_blockquant_mxint8(A, b, gk, gn, b_is_nk=nk),
            "mxfp8": lambda b, nk: ext.gemm_blockquant_mxfp8(A, b, gk, gn, b_is_nk=nk)}[op]
    old = ext.TRANSPOSE_MIN_MNK
    try:
        ext.TRANSPOSE_MIN_MNK = 1 << 62
        small = call(B, False)
    finally:
        ext.TRANSPOSE_MIN_MNK = old
    big = call(W, True)
    assert torch.isfinite(small.float()).all()
    assert torch.equal(small.view(torch.int16), big.view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(2048, 4096, 14336), (512, 2048, 8192), (300, 1000, 8192)])
def test_fp32_split_k_is_the_sum_of_the_two_halves(gpu, M, N, K):
    """Split-K fp32 accumulation (the prefill's long-K linears): C = R16(P0 + P1) bit for
    bit, P0 and P1 the kernels' own fp32 sums over the two K halves (group partials with
    group_k = K / 2); and within fp32-accumulation tolerance of the unsplit GEMM."""
    from hbq_amd import _lib, blockquant_ext as ext
    print(f"split K {M}x{N}x{K}", flush=True)
    assert _lib.lib().hbq_gemm_fp32_accum_workspace(M, N, K, 1) == 2 * M * N * 4
    g = torch.Generator(device=gpu).manual_seed(M + K)
    A = torch.randn(M, K, device=gpu, generator=g).half()
    W = (torch.randn(N, K, device=gpu, generator=g) * 0.02).half()
    C = ext.gemm_fp32_accum_nk_split(A, W)
    P = ext.group_partials(A, W, K // 2, b_is_nk=True)
    assert P.shape[0] == 2
    ref = (P[0] + P[1]).half()
    assert torch.equal(C.view(torch.int16), ref.view(torch.int16))
    full = ext.gemm_fp32_accum_nk(A, W).float()
    rel = ((C.float() - full).norm() / full.norm()).item()
    assert rel < 1e-3, rel


def test_fp32_split_k_only_for_long_k(gpu):
    """Shapes that fill the chip, or short K, take no workspace (unsplit GEMM)."""
    from hbq_amd import _lib
    L = _lib.lib()
    assert L.hbq_gemm_fp32_accum_workspace(2048, 4096, 4096, 1) == 0      # short K
    assert L.hbq_gemm_fp32_accum_workspace(4096, 4096, 14336, 1) == 0     # more tiles than one round
    assert L.hbq_gemm_fp32_accum_workspace(2048, 4096, 14336, 0) == 0     # B[K, N] layout


@pytest.mark.parametrize("op,gk,gn", [("fp32", 0, 0), ("grouped", 128, 0), ("mxint8", 128, 32)])
def test_wide_tiles_on_short_grids_bit_identical(gpu, op, gk, gn):
    """M = 2000, N = 6144: 192 tiles of 256 x 256 (fewer than the compute units) run in one
    round instead of two rounds of 384 narrower tiles (the prefill's q/k/v shape); the bits
    equal the 128x128 kernel's on B[K, N]."""
    from hbq_amd import blockquant_ext as ext
    M, K, N = 2000, 512, 6144
    print(f"wide tiles, short grid: {op}", flush=True)
    A = synth(M, K, 61, "f16").to(gpu)
    B = synth(K, N, 62, "f16", std=0.02).to(gpu)
    W = B.t().contiguous()
    call = {"fp32": lambda b, nk: ext.gemm_fp32_accum(A, b, b_is_nk=nk),
            "grouped": lambda b, nk: ext.gemm_fp16_grouped_accum(A, b, gk, b_is_nk=nk),
            "mxint8": lambda b, nk: ext.gemm_blockquant_mxint8(A, b, gk, gn, b_is_nk=nk)}[op]
    old = ext.TRANSPOSE_MIN_MNK
    try:
        ext.TRANSPOSE_MIN_MNK = 1 << 62
        small = call(B, False)
    finally:
        ext.TRANSPOSE_MIN_MNK = old
    big = call(W, True)
    assert torch.isfinite(small.float()).all()
    assert torch.equal(small.view(torch.int16), big.view(torch.int16))


@pytest.mark.parametrize("Z,M,N,K", [(8, 8192, 2048, 128), (8, 8192, 128, 2048), (3, 300, 1000, 192)])
def test_fp32_batched_equals_per_problem(gpu, Z, M, N, K):
    """hbq_gemm_fp32_accum_batched (the decoder's attention products: q k^T and P V) gives
    each problem the bits of gemm_fp32_accum on W[N, K] alone."""
    from hbq_amd import _lib, blockquant_ext as ext
    print(f"batched fp32 {Z}x{M}x{N}x{K}", flush=True)
    g = torch.Generator(device=gpu).manual_seed(Z * M + N)
    A = torch.randn(Z, M, K, device=gpu, generator=g).half()
    W = (torch.randn(Z, N, K, device=gpu, generator=g) * 0.1).half()
    C = torch.empty(Z, M, N, device=gpu, dtype=torch.float16)
    _lib.check(_lib.lib().hbq_gemm_fp32_accum_batched(_lib.ptr(A), _lib.ptr(W), _lib.ptr(C), Z, M, N, K, M * K,
                                                      N * K, M * N, _lib.stream_of(A)))
    for z in range(Z):
        ref = ext.gemm_fp32_accum_nk(A[z], W[z])
        assert torch.equal(C[z].view(torch.int16), ref.view(torch.int16)), z


def test_fp32_batched_gqa_rows_into_heads(gpu):
    """hbq_gemm_fp32_accum_batched_ex as the decoder's P V uses it: 8 query heads over 2 kv
    heads (W shared by groups of 4), each head's [T, d] output written at column h * d of
    rows H * d long.  Every head gets the bits of the single GEMM on its own operands."""
    from hbq_amd import _lib, blockquant_ext as ext
    H, kvh, T, d = 8, 2, 256, 128
    g = torch.Generator(device=gpu).manual_seed(78)
    P = torch.rand(H, T, T, device=gpu, generator=g).half()
    VT = (torch.randn(kvh, d, T, device=gpu, generator=g) * 0.5).half()
    out = torch.full((T, H, d), 3.0, device=gpu, dtype=torch.float16)
    _lib.check(_lib.lib().hbq_gemm_fp32_accum_batched_ex(_lib.ptr(P), _lib.ptr(VT), _lib.ptr(out), H, T, d, T, T * T,
                                                         d * T, H // kvh, d, H * d, _lib.stream_of(P)))
    for h in range(H):
        ref = ext.gemm_fp32_accum_nk(P[h], VT[h // (H // kvh)])
        assert torch.equal(out[:, h].view(torch.int16), ref.view(torch.int16)), h


def test_fp32_batched_strides_beyond_one_problem(gpu):
    """Batch strides larger than one problem (problems inside wider buffers, as the ABI
    allows): each problem gets the bits of the single GEMM, and the gaps of C stay as
    they were."""
    from hbq_amd import _lib, blockquant_ext as ext
    Z, M, N, K = 4, 320, 256, 192
    sA, sW, sC = M * K + 136, N * K + 64, M * N + 8
    g = torch.Generator(device=gpu).manual_seed(77)
    A = torch.randn(Z * sA, device=gpu, generator=g).half()
    W = (torch.randn(Z * sW, device=gpu, generator=g) * 0.1).half()
    C = torch.full((Z * sC,), 7.0, device=gpu, dtype=torch.float16)
    _lib.check(_lib.lib().hbq_gemm_fp32_accum_batched(_lib.ptr(A), _lib.ptr(W), _lib.ptr(C), Z, M, N, K, sA, sW,
                                                      sC, _lib.stream_of(A)))
    for z in range(Z):
        a = A[z * sA: z * sA + M * K].view(M, K)
        w = W[z * sW: z * sW + N * K].view(N, K)
        ref = ext.gemm_fp32_accum_nk(a, w)
        got = C[z * sC: z * sC + M * N].view(M, N)
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), z
        assert bool((C[z * sC + M * N: (z + 1) * sC] == 7.0).all()), z
