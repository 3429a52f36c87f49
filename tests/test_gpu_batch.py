"""The layout-0 batched token path (nwc_linear_xbf16_batch, NWCWeight.linear_batch, NWCLinear on 2..8 tokens): each
vector's result bit-identical to the single-vector kernel's, rounded to nearest even from within 1e-3 of float64
(tests/helpers.py check_rne), on the Qwen3-4B
matrices, a ragged shape, escape-heavy rows that decode from global memory, a vocabulary-sized matrix (several
residency rounds), and fp8 with its row scale and a bias; NWCLinear's batched forward against its decompress +
F.linear path."""
import numpy as np
import pytest
import torch

from tests.helpers import bf16_matrix, check_rne, token_tol

pytestmark = pytest.mark.gpu


def _nwc():
    from nwc_amd.nwc_torch import NWCWeight, NWCLinear, quantize_fp8
    return NWCWeight, NWCLinear, quantize_fp8


def _check(y, y64, terms=None):
    check_rne(y, y64, token_tol(y64, terms), "batched token path")


@pytest.mark.parametrize("M,K,escapes", [(6144, 2560, "none"), (2560, 4096, "none"), (19456, 2560, "none"),
                                         (2560, 9728, "none"), (1003, 1100, "none"), (2560, 9728, "heavy"),
                                         (151936, 1024, "none")])
@pytest.mark.parametrize("T", [2, 3, 4, 7])
def test_batch_equals_single_vector(cuda, M, K, escapes, T):
    NWCWeight, _, _ = _nwc()
    print(f"batch {T} x {M}x{K} {escapes}", flush=True)
    w = bf16_matrix(M, K, seed=M + K)
    if escapes == "heavy":
        sign = torch.randint(0, 2, (24, K), generator=torch.Generator().manual_seed(5)) * 2 - 1
        w[0:24] = (sign * 1e30).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=0)
    X = torch.randn(T, K, generator=torch.Generator().manual_seed(T)).to(torch.bfloat16).cuda()
    Y = c.linear_batch(X, None)
    single = torch.stack([c.linear_bf16(X[t], None) for t in range(T)])
    assert torch.equal(Y, single)
    wd = w.cuda().double()
    _check(Y[T - 1], (wd @ X[T - 1].double()).cpu().numpy(), (wd.abs() @ X[T - 1].double().abs()).cpu().numpy())


def test_batch_fp8_scale_bias_and_module(cuda):
    """fp8 weights (row scale) with a bias through linear_batch, and NWCLinear's forward on [1, T, K] inputs for
    T = 1..9: batched (2..8) and single-token results against the decompress + F.linear path of the same module."""
    NWCWeight, NWCLinear, quantize_fp8 = _nwc()
    M, K = 2560, 4096
    w = bf16_matrix(M, K, seed=3, escapes=False).float()
    q, scale = quantize_fp8(w)
    c = NWCWeight(w, device="cuda", elem="fp8", layout=0)
    g = torch.Generator().manual_seed(7)
    bias = torch.randn(M, generator=g).to(torch.bfloat16).cuda()
    X = torch.randn(4, K, generator=g).to(torch.bfloat16).cuda()
    Y = c.linear_batch(X, bias)
    assert torch.equal(Y, torch.stack([c.linear_bf16(X[t], bias) for t in range(4)]))
    y64 = (q.double() @ X[2].double().cpu()) * scale.double() + bias.double().cpu()
    _check(Y[2], y64.numpy())
    lin = NWCLinear(w=NWCWeight(bf16_matrix(M, K, seed=4), device="cuda", layout=0), bias=bias, device="cuda")
    for T in range(1, 10):
        x = torch.randn(1, T, K, generator=g).to(torch.bfloat16).cuda()
        got = lin(x)
        want = torch.nn.functional.linear(x, lin.w.dequant(), lin.bias)
        assert got.shape == want.shape
        d = (got.float() - want.float()).abs().max().item()
        assert d <= 2.0 ** -7 * want.float().abs().max().item() + 1e-3, (T, d)
