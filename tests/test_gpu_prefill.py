"""GPU tests of the fused layout-0 prefill (nwc_prefill_xbf16, NWCWeight.prefill): several tokens multiplied with the
compressed matrix without a temporary BF16 copy (decode into LDS, matrix cores).

Bar: every output rounded once, to nearest even, from a value within 1e-3 |ref| + 1e-6 of the float64 product on the
decoded weights, plus the fp32 summation bound (2^-20 times the sum of |terms|) for the matrix cores' accumulation
order (tests/helpers.py check_rne): the kernel's sums are not in a GEMM library's order, so it matches F.linear to
rounding, not bit for bit.  Covers ragged M and K (rows and columns past
the matrix, a half k-step past K16), 1 to 512 tokens (all three token tiles and partial ones), BF16 with escapes, fp8
with row scales, bias, and NWCLinear's opt-in dispatch (NWC_PREFILL=fused)."""
import pytest
import torch
import torch.nn.functional as F

from tests.helpers import bf16_matrix, check_rne, fp8_source

pytestmark = pytest.mark.gpu


def _weight(M, K, elem, seed):
    from nwc_amd.nwc_torch import NWCWeight
    w = fp8_source(M, K, seed=seed) if elem == "fp8" else bf16_matrix(M, K, seed=seed, escapes=True)
    return NWCWeight(w, device="cuda", elem=elem, layout=0)


def _check(c, x, y, bias):
    wd = c.dequant().double()
    if c.scale is not None:
        wd = wd * c.scale.double()[:, None]
    ref = x.double() @ wd.t()
    if bias is not None:
        ref = ref + bias.double()
    terms = x.double().abs() @ wd.abs().t()
    tol = 1e-3 * ref.abs() + 2.0 ** -20 * terms + 1e-6
    check_rne(y, ref.cpu().numpy(), tol.cpu().numpy(), "prefill")


@pytest.mark.parametrize("M,K,T,elem,with_bias", [
    (300, 1000, 12, "bf16", True),      # ragged M and K: K16 = 1008 ends in a half k-step
    (300, 1000, 37, "bf16", False),
    (64, 512, 1, "bf16", True),         # one token
    (8, 16, 5, "bf16", True),           # one row group, one 16-column chunk
    (1000, 2600, 70, "bf16", True),     # two token tiles of 64
    (257, 1024, 100, "fp8", True),      # fp8 with row scales, 129 rows past a tile
    (2000, 1536, 300, "fp8", False),    # 64-token tiles, the last with 44 tokens
    (8200, 1024, 300, "bf16", True),    # 256-token tiles (129 row tiles, the last with one row group)
])
def test_prefill_matches_float64(cuda, M, K, T, elem, with_bias):
    print(f"prefill {M}x{K} T={T} {elem} bias={with_bias}", flush=True)
    c = _weight(M, K, elem, seed=M + K + T)
    g = torch.Generator().manual_seed(T)
    x = torch.randn(T, K, generator=g).to(torch.bfloat16).cuda()
    b = ((torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)).cuda() if with_bias else None
    y = c.prefill(x, b)
    assert y.shape == (T, M) and y.dtype == torch.bfloat16
    _check(c, x, y, b)


@pytest.mark.parametrize("name,M,K", [("qkv", 6144, 2560), ("down", 2560, 9728)])
def test_prefill_qwen3_4b_512_tokens(cuda, name, M, K):
    """configs[2]'s 512-token prefill at two Qwen3-4B shapes (128- and 64-token tiles)."""
    print(f"prefill 512 tokens {name} {M}x{K}", flush=True)
    from nwc_amd.nwc_torch import NWCWeight
    g = torch.Generator().manual_seed(M)
    w = (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=0)
    x = torch.randn(512, K, generator=g).to(torch.bfloat16).cuda()
    y = c.prefill(x, None)
    _check(c, x, y, None)
    # and against the dequantization + hipBLASLt path on the same weights, to the same bound
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    _check(c, x, F.linear(x, c.dequant()), None)


def test_nwclinear_fused_prefill_dispatch(cuda, monkeypatch):
    """NWC_PREFILL=fused sends more than NWC_BATCH_MAX BF16 tokens of a layout-0 matrix to the fused kernel; the
    default keeps the temporary matrix and F.linear (bit-identical to it)."""
    import nwc_amd.nwc_torch as nt
    M, K = 384, 1536
    c = _weight(M, K, "bf16", seed=5)
    g = torch.Generator().manual_seed(6)
    b = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)
    lin = nt.NWCLinear(w=c, bias=b, device="cuda")
    x = torch.randn(2, 20, K, generator=g).to(torch.bfloat16).cuda()
    monkeypatch.setattr(nt, "PREFILL", "dequant")
    y_dq = lin(x)
    assert torch.equal(y_dq, F.linear(x, c.dequant(), b.cuda()))
    monkeypatch.setattr(nt, "PREFILL", "fused")
    y_f = lin(x)
    assert y_f.shape == (2, 20, M)
    assert torch.equal(y_f.view(40, M), c.prefill(x.view(40, K), b.cuda()))
    _check(c, x.view(40, K), y_f.view(40, M), b.cuda())


def test_prefill_zero_tokens_and_refusals(cuda):
    from nwc_amd.nwc_torch import NWCWeight
    c = _weight(64, 512, "bf16", seed=1)
    y = c.prefill(torch.empty(0, 512, dtype=torch.bfloat16, device="cuda"), None)
    assert y.shape == (0, 64)
    c1 = NWCWeight(bf16_matrix(64, 512, seed=2), device="cuda", layout=1)
    with pytest.raises(ValueError):
        c1.prefill(torch.zeros(3, 512, dtype=torch.bfloat16, device="cuda"), None)
