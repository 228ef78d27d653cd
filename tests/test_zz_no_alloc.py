"""The allocation-free GEMM entry point (hbq_gemm_fp32_accum_noalloc) through the C ABI.

It must give the bits of hbq_gemm_fp32_accum_ws with a caller workspace, on consecutive
calls that share the library's scratch buffer (the second call smaller than the first,
so stale partials of the first would show)."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ws_gemm(L, A, W, M, N, K):
    from hbq_amd import _lib
    need = L.hbq_gemm_fp32_accum_workspace(M, N, K, 1)
    ws = torch.empty(max(need, 4) // 4, dtype=torch.float32, device=A.device)
    C = torch.empty(M, N, dtype=torch.float16, device=A.device)
    _lib.check(L.hbq_gemm_fp32_accum_ws(_lib.ptr(A), _lib.ptr(W), _lib.ptr(C), _lib.ptr(ws), need, M, N, K, 1,
                                        _lib.stream_of(A)))
    return C, need


def test_noalloc_gemm_matches_workspace_entry_point(gpu):
    from hbq_amd import _lib
    L = _lib.lib()
    g = torch.Generator(device=gpu).manual_seed(41)
    # (M, N, K): the prefill down projection (64 MiB of split-K partials, the whole
    # buffer), then a smaller split-K shape (32 MiB), then a shape without split K
    shapes = [(2048, 4096, 14336), (1024, 4096, 8192), (256, 512, 1024)]
    splits_seen = []
    for M, N, K in shapes:
        print(f"noalloc gemm M={M} N={N} K={K}", flush=True)
        A = torch.randn(M, K, device=gpu, generator=g).half()
        W = (torch.randn(N, K, device=gpu, generator=g) * 0.02).half()
        ref, need = _ws_gemm(L, A, W, M, N, K)
        splits_seen.append(need)
        C = torch.full((M, N), float("nan"), dtype=torch.float16, device=gpu)
        rc = L.hbq_gemm_fp32_accum_noalloc(_lib.ptr(A), _lib.ptr(W), _lib.ptr(C), M, N, K, 1, _lib.stream_of(A))
        assert rc == 0, L.hbq_last_error()
        torch.cuda.synchronize()
        assert torch.equal(C.view(torch.int16), ref.view(torch.int16)), (M, N, K)
    # the first two shapes used the scratch buffer (the first one filled it), the last did not
    assert splits_seen[0] == 64 << 20 and 0 < splits_seen[1] < splits_seen[0] and splits_seen[2] == 0

