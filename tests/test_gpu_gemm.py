"""The prefill GEMM of the library (nwc_gemm_xbf16, through nwc_amd.nwc_torch.gemm_xbf16) on the GPU: every output
within one BF16 rounding + the fp32 summation bound (2^-20 times the sum of |terms|) of the float64 product; the
two-group kernel (K a multiple of 128) and the one-group kernel, unsplit and split over K (partial tiles added by the
last workgroup of a tile), ragged token counts and rows, an odd row count (element stores), bias, row-strided
weights as dequant() returns them; repeated calls and calls of other shapes in between (the workspace counters)
give the same bits; shapes the kernel cannot take are refused.  NWCLinear's prefill goes through the same GEMM choice
for dequantized and resident weights."""
import pytest
import torch
import torch.nn.functional as F

pytestmark = pytest.mark.gpu


def _operands(T, N, K, seed, pad=0, bias=False):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    wf = (torch.randn(N, K + pad, generator=g) * 0.02).to(torch.bfloat16).cuda()
    b = (torch.randn(N, generator=g) * 0.1).to(torch.bfloat16).cuda() if bias else None
    return x, wf[:, :K], b


def _check(y, x, w, b):
    ref = x.double() @ w.double().t() + (b.double() if b is not None else 0.0)
    tol = 2.0 ** -8 * ref.abs() + 2.0 ** -20 * (x.double().abs() @ w.double().abs().t()) + 1e-6
    err = (y.double() - ref).abs()
    assert bool((err <= tol).all()), f"max error / bound {float((err / tol).max()):.3f}"


SHAPES = [
    # T, N, K, pad, bias
    (512, 2560, 9728, 0, True),      # Qwen3-4B down: split over K, two groups
    (512, 2560, 4096, 0, False),     # o: split
    (512, 6144, 2560, 0, False),     # qkv: one 128 x 128 tile per workgroup, no split
    (300, 2560, 4096, 0, True),      # ragged token tile, split
    (77, 1000, 640, 16, True),       # ragged rows and tokens, row-strided weights
    (9, 2560, 9728, 0, False),       # one token tile: many splits
    (513, 130, 192, 8, True),        # K = 3 stages: one group; 130 rows: element stores
    (200, 384, 1344, 0, False),      # K = 21 stages: one group, split
    (1, 1, 64, 0, False),
]


@pytest.mark.parametrize("T,N,K,pad,bias", SHAPES)
def test_gemm_within_fp32_bound(cuda, T, N, K, pad, bias):
    from nwc_amd.nwc_torch import gemm_xbf16, lib
    print(f"gemm {T}x{N}x{K} pad {pad} bias {bias} workspace {lib.nwc_gemm_workspace(T, N, K)}", flush=True)
    x, w, b = _operands(T, N, K, seed=T + N + K, pad=pad, bias=bias)
    y = gemm_xbf16(x, w, b)
    assert y.shape == (T, N) and y.dtype == torch.bfloat16
    _check(y, x, w, b)
    assert torch.equal(gemm_xbf16(x, w, b).view(torch.int16), y.view(torch.int16))


def test_gemm_workspace_reuse_across_shapes(cuda):
    """Split products of different tile counts share the workspace; each call leaves its counters zero."""
    from nwc_amd.nwc_torch import gemm_xbf16
    print("gemm workspace reuse", flush=True)
    a = _operands(512, 2560, 9728, seed=1)
    c = _operands(64, 2560, 4096, seed=2)
    ya = gemm_xbf16(*a)
    yc = gemm_xbf16(*c)
    for _ in range(3):
        assert torch.equal(gemm_xbf16(*a).view(torch.int16), ya.view(torch.int16))
        assert torch.equal(gemm_xbf16(*c).view(torch.int16), yc.view(torch.int16))
    _check(ya, *a)
    _check(yc, *c)


def test_gemm_in_a_graph(cuda):
    """Replays of a captured split product, with eager work between them, give the eager result each time."""
    from nwc_amd.nwc_torch import gemm_xbf16
    print("gemm graph replay", flush=True)
    x, w, b = _operands(512, 2560, 9728, seed=3, bias=True)
    want = gemm_xbf16(x, w, b)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y = gemm_xbf16(x, w, b)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
        gemm_xbf16(*_operands(128, 256, 8192, seed=4))        # eager work between the replays
        torch.cuda.synchronize()


def test_gemm_refuses_shapes(cuda):
    from nwc_amd.nwc_torch import call, lib, ptr, stream
    print("gemm refusals", flush=True)
    x = torch.zeros(4, 128, dtype=torch.bfloat16, device="cuda")
    w = torch.zeros(8, 128, dtype=torch.bfloat16, device="cuda")
    y = torch.zeros(4, 8, dtype=torch.bfloat16, device="cuda")
    for T, N, K, ldx, ldw in [(4, 8, 100, 128, 128),      # K not a multiple of 64
                              (4, 8, 128, 120, 128),      # row stride below K
                              (4, 8, 128, 128, 132),      # row stride not a multiple of 8
                              (0, 8, 128, 128, 128)]:
        with pytest.raises(RuntimeError):
            call("nwc_gemm_xbf16", stream(), ptr(x), ldx, ptr(w), ldw, None, ptr(y), T, N, K, None, 0)
    need = lib.nwc_gemm_workspace(4, 8, 4096)
    if need:                                               # a split product without its workspace
        xs = torch.zeros(4, 4096, dtype=torch.bfloat16, device="cuda")
        ws = torch.zeros(8, 4096, dtype=torch.bfloat16, device="cuda")
        with pytest.raises(RuntimeError):
            call("nwc_gemm_xbf16", stream(), ptr(xs), 4096, ptr(ws), 4096, None, ptr(y), 4, 8, 4096, None, 0)


@pytest.mark.parametrize("layout", [0, 1])
def test_nwclinear_prefill_uses_one_gemm_choice(cuda, layout, monkeypatch):
    """512 tokens through a down-shaped NWCLinear: the library GEMM on the dequantized matrix, equal to the same GEMM
    on the resident BF16 weights and within the fp32 bound; with NWC_GEMM=hipblaslt, F.linear's result exactly."""
    import nwc_amd.nwc_torch as N
    from tests.helpers import bf16_matrix
    print(f"NWCLinear prefill 512 down layout {layout}", flush=True)
    M, K = 2560, 9728
    w = bf16_matrix(M, K, seed=21 + layout, escapes=False)
    lin = N.NWCLinear(w=N.NWCWeight(w, device="cuda", layout=layout), device="cuda")
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, 512, K, generator=g).to(torch.bfloat16).cuda()
    assert N.gemm_preferred(512, M, K)
    y = lin(x)
    assert torch.equal(y, N.gemm_xbf16(x, w.cuda()))
    _check(y.view(512, M), x.view(512, K), w.cuda(), None)
    monkeypatch.setattr(N, "GEMM", "hipblaslt")
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    assert torch.equal(lin(x), F.linear(x, w.cuda()))
