"""nwc_gemm_xbf16_noalloc (the product without workspace arguments, its partial sums in the library's static array)
gives the bits nwc_gemm_xbf16 gives with a caller's workspace, through the C ABI: two calls in a row, the second
smaller, both split over K (the array's counters must be zero again after the first), and an unsplit product; a
product whose workspace would not fit the array is refused."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _operands(T, N, K, seed, bias):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    w = (torch.randn(N, K, generator=g) * 0.02).to(torch.bfloat16).cuda()
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).cuda() if bias else None
    return x, w, b


def _noalloc(x, w, b):
    from nwc_amd.nwc_torch import call, ptr, stream
    T, K = x.shape
    N = w.shape[0]
    y = torch.empty(T, N, dtype=torch.bfloat16, device=x.device)
    call("nwc_gemm_xbf16_noalloc", stream(), ptr(x), K, ptr(w), w.stride(0), ptr(b), ptr(y), T, N, K)
    return y


@pytest.mark.parametrize("first,second", [((512, 2560, 9728, True), (300, 1024, 4096, False)),
                                          ((64, 2560, 4096, False), (9, 384, 1344, True))])
def test_noalloc_matches_workspace_entry(cuda, first, second):
    from nwc_amd.nwc_torch import gemm_xbf16, lib
    for i, (T, N, K, bias) in enumerate((first, second)):
        print(f"noalloc call {i}: {T}x{N}x{K} bias {bias} workspace {lib.nwc_gemm_workspace(T, N, K)}", flush=True)
        assert lib.nwc_gemm_workspace(T, N, K) > 0           # split over K: the static array is used
        ops = _operands(T, N, K, seed=T + N + K, bias=bias)
        y = _noalloc(*ops)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), gemm_xbf16(*ops).view(torch.int16))


def test_noalloc_unsplit_and_refused(cuda):
    from nwc_amd.nwc_torch import call, gemm_xbf16, lib, ptr, stream
    print("noalloc unsplit product and refusal", flush=True)
    ops = _operands(512, 6144, 2560, seed=5, bias=False)
    assert lib.nwc_gemm_workspace(512, 6144, 2560) == 0
    assert torch.equal(_noalloc(*ops).view(torch.int16), gemm_xbf16(*ops).view(torch.int16))
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 128, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda")
    with pytest.raises(RuntimeError):                         # K not a multiple of 64
        call("nwc_gemm_xbf16_noalloc", stream(), ptr(x), 128, ptr(w), 128, None, ptr(y), 4, 8, 100)


def test_noalloc_graph_replays(cuda):
    """A captured call replayed three times, eager calls of another shape between the replays: every replay gives
    the eager result."""
    print("noalloc graph replays", flush=True)
    ops = _operands(256, 2560, 9728, seed=7, bias=True)
    want = _noalloc(*ops)
    other = _operands(128, 512, 8192, seed=8, bias=False)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = _noalloc(*ops)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
        _noalloc(*other)
        torch.cuda.synchronize()
