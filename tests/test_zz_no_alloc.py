"""myelin_gemm_noalloc (static device scratch, no allocation) against
myelin_gemm with a caller workspace of the size the split needs: the same
kernels and split, so the outputs must be equal bit for bit.  Two calls in a
row, the second on a smaller product, so stale scratch contents from the
first call would show.  Captured in a HIP graph, as the process's first
call of the entry point (its device address lookup then runs inside the
capture) and again after eager calls, every replay equals the eager
result bit for bit."""

from __future__ import annotations

import pytest
import torch

from myelin_amd import _lib

pytestmark = pytest.mark.gpu

DEV = torch.device("cuda:0")
MAX_ELEMS = 16 * 1024 * 1024  # MYELIN_NOALLOC_SCRATCH_ELEMS


def _need(M, N, K, prec):
    return int(_lib.load().myelin_gemm_workspace_elems(M, N, K, prec))


def _pair(A, a_dt, B, b_dt, bias, C0, M, N, K, lda, ldb, ta, tb, acc, prec):
    """(no-alloc result, workspace result) from the same inputs."""

    stream = _lib.stream(DEV)
    need = _need(M, N, K, prec)
    ws = torch.empty(max(need, 1), device=DEV)
    ref = C0.clone()
    got = C0.clone()
    _lib.call("myelin_gemm", A.data_ptr(), a_dt, B.data_ptr(), b_dt, _lib.ptr(bias), ref.data_ptr(), M, N, K, lda,
              ldb, N, ta, tb, acc, prec, ws.data_ptr(), need, stream)
    _lib.call("myelin_gemm_noalloc", A.data_ptr(), a_dt, B.data_ptr(), b_dt, _lib.ptr(bias), got.data_ptr(), M, N,
              K, lda, ldb, N, ta, tb, acc, prec, stream)
    torch.cuda.synchronize()
    return got, ref, need


def test_noalloc_gemm_under_graph_capture():
    """Kept first in this file: the capture holds the process's first
    myelin_gemm_noalloc call, whose device-address lookup runs while the
    stream is being captured; a second graph is captured after eager calls.
    Replays run with eager work and synchronisations between them."""

    g = torch.Generator().manual_seed(13)
    bf16 = _lib.DT[torch.bfloat16]
    prec = _lib.PREC["bf16"]
    M, N, K = 784, 2048, 12800  # splits K: the partial planes go to the static array
    assert _need(M, N, K, prec) > 0
    A = torch.randn(K, M, generator=g).to(torch.bfloat16).to(DEV)
    B = torch.randn(K, N, generator=g).to(torch.bfloat16).to(DEV)
    need = _need(M, N, K, prec)
    ws = torch.empty(need, device=DEV)
    ref = torch.empty(M, N, device=DEV)
    _lib.call("myelin_gemm", A.data_ptr(), bf16, B.data_ptr(), bf16, None, ref.data_ptr(), M, N, K, M, N, N, 1, 0,
              0, prec, ws.data_ptr(), need, _lib.stream(DEV))
    torch.cuda.synchronize()
    for which in ("first call inside the capture", "captured after eager calls"):
        print(f"noalloc graph capture: {which}", flush=True)
        out = torch.full((M, N), float("nan"), device=DEV)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            _lib.call("myelin_gemm_noalloc", A.data_ptr(), bf16, B.data_ptr(), bf16, None, out.data_ptr(), M, N,
                      K, M, N, N, 1, 0, 0, prec, _lib.stream(DEV))
        for rep in range(3):
            out.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, ref), f"replay {rep} ({which})"
            # eager work between replays, on the same scratch array
            eager = torch.empty(M, N, device=DEV)
            _lib.call("myelin_gemm_noalloc", A.data_ptr(), bf16, B.data_ptr(), bf16, None, eager.data_ptr(), M,
                      N, K, M, N, N, 1, 0, 0, prec, _lib.stream(DEV))
            torch.cuda.synchronize()
            assert torch.equal(eager, ref)
        del graph


def test_noalloc_gemm_equals_workspace_gemm_two_calls():
    g = torch.Generator().manual_seed(11)
    bf16, f32 = _lib.DT[torch.bfloat16], _lib.DT[torch.float32]
    print("noalloc case 1: bf16 mn-contiguous 784 x 2048 x 12800", flush=True)
    M, N, K = 784, 2048, 12800
    A = torch.randn(K, M, generator=g).to(torch.bfloat16).to(DEV)  # trans_a: stored [K, M]
    B = torch.randn(K, N, generator=g).to(torch.bfloat16).to(DEV)
    C0 = torch.full((M, N), float("nan"), device=DEV)
    got, ref, need = _pair(A, bf16, B, bf16, None, C0, M, N, K, M, N, 1, 0, 0, _lib.PREC["bf16"])
    assert 0 < need <= MAX_ELEMS
    assert torch.equal(got, ref)
    approx = (A.float().t().double() @ B.float().double()).float()
    assert torch.allclose(got, approx, rtol=1e-4, atol=1e-3)

    print("noalloc case 2: fp32 512 x 384 x 4096, bias, accumulate (smaller, after case 1)", flush=True)
    M, N, K = 512, 384, 4096
    A = torch.randn(M, K, generator=g).to(DEV)
    B = torch.randn(K, N, generator=g).to(DEV)
    bias = torch.randn(N, generator=g).to(DEV)
    C0 = torch.randn(M, N, generator=g).to(DEV)
    got, ref, need = _pair(A, f32, B, f32, bias, C0, M, N, K, K, N, 0, 0, 1, _lib.PREC["fp32"])
    assert 0 < need < 12845056
    assert torch.equal(got, ref)
    approx = (C0.double() + A.double() @ B.double() + bias.double()).float()
    assert torch.allclose(got, approx, rtol=1e-4, atol=1e-3)


def test_noalloc_narrow_output_two_calls():
    """Narrow outputs (N <= 32, readout currents and their weight gradient)
    split K into fixed chunks of at most 512 whatever M is; their partial
    planes go to the static array too."""

    g = torch.Generator().manual_seed(12)
    f32 = _lib.DT[torch.float32]
    print("noalloc narrow case 1: fp32 2048 x 20 x 20000", flush=True)
    M, N, K = 2048, 20, 20000
    A = torch.randn(M, K, generator=g).to(DEV)
    B = torch.randn(K, N, generator=g).to(DEV)
    C0 = torch.full((M, N), float("nan"), device=DEV)
    got, ref, need = _pair(A, f32, B, f32, None, C0, M, N, K, K, N, 0, 0, 0, _lib.PREC["fp32"])
    assert 0 < need <= MAX_ELEMS
    assert torch.equal(got, ref)
    approx = (A.double() @ B.double()).float()
    assert torch.allclose(got, approx, rtol=1e-4, atol=1e-3)

    print("noalloc narrow case 2: fp32 300 x 10 x 3000, B stored [N, K], bias, accumulate (smaller)", flush=True)
    M, N, K = 300, 10, 3000
    A = torch.randn(M, K, generator=g).to(DEV)
    B = torch.randn(N, K, generator=g).to(DEV)
    bias = torch.randn(N, generator=g).to(DEV)
    C0 = torch.randn(M, N, generator=g).to(DEV)
    got, ref, need = _pair(A, f32, B, f32, bias, C0, M, N, K, K, K, 0, 1, 1, _lib.PREC["fp32"])
    assert 0 < need < 2048 * 20 * 40
    assert torch.equal(got, ref)
    approx = (C0.double() + A.double() @ B.double().t() + bias.double()).float()
    assert torch.allclose(got, approx, rtol=1e-4, atol=1e-3)


def test_noalloc_gemm_without_split_and_rejection():
    g = torch.Generator().manual_seed(12)
    f32 = _lib.DT[torch.float32]
    M, N, K = 2048, 2048, 128  # short K: no K split, no scratch
    A = torch.randn(M, K, generator=g).to(DEV)
    B = torch.randn(N, K, generator=g).to(DEV)
    C0 = torch.zeros(M, N, device=DEV)
    got, ref, need = _pair(A, f32, B, f32, None, C0, M, N, K, K, K, 0, 1, 0, _lib.PREC["fp32"])
    assert need == 0
    assert torch.equal(got, ref)
    # a product whose split needs more than the static array: rejected on
    # the host before any launch
    M, N, K = 768, 1536, 1 << 20
    assert _need(M, N, K, _lib.PREC["bf16"]) > MAX_ELEMS
    with pytest.raises(ValueError, match="more than"):
        _lib.call("myelin_gemm_noalloc", 1, f32, 1, f32, None, 1, M, N, K, K, N, N, 0, 0, 0, _lib.PREC["bf16"],
                  _lib.stream(DEV))
