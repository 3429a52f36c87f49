"""The product's host encoder (nwc_amd/csrc/encode.cpp, multithreaded) against the oracle's serial restatement of
the reference encoder (oracle/nwc_oracle.c, nwc_ops.cu:175-348): every output byte identical -- data (incl. the
data length and slack), bases, hdr, the raw plane, psym and the decode table -- on the reference tests' shapes and
stressors (tests/test_format_cpu.py:117-131, test_fp8.py:19) and on exponent-spread matrices with many escapes.
CPU only: the encoder is a host entry point of the C ABI."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_matrix, bits16, fp8_source

BF16_CASES = [(8, 512, 0.02), (13, 40, 0.02), (3, 4097, 0.02), (100, 1000, 1.0), (64, 2048, 0.02), (17, 520, 0.02),
              (1, 1, 0.02), (300, 3000, 0.02)]
FP8_CASES = [(8, 512), (13, 40), (3, 4097), (101, 1000)]


def _nwc():
    from nwc_amd.nwc_torch import NWCWeight, quantize_fp8
    return NWCWeight, quantize_fp8


def _assert_identical(c, e):
    assert c.data.numel() == e["dl"] + 64
    assert np.array_equal(c.data.numpy()[: e["dl"]], e["data"][: e["dl"]])
    assert not c.data.numpy()[e["dl"]:].any()                       # slack bytes are zero
    assert np.array_equal(c.bases.numpy().view(np.uint32), e["bases"])
    assert np.array_equal(c.hdr.numpy(), e["hdr"])
    assert np.array_equal(c.lut.numpy().view(np.uint32), e["lut"])
    assert np.array_equal(c.low.numpy()[: e["n_low"]], e["low"][: e["n_low"]])


def _spread(M, K, seed):
    """Signs random, magnitudes 2^U(-40, 40): ~80 exponent values, so ranks >= 15 (escapes) are common."""
    g = torch.Generator().manual_seed(seed)
    mag = torch.exp2(torch.rand(M, K, generator=g) * 80 - 40)
    sign = torch.where(torch.rand(M, K, generator=g) < 0.5, -1.0, 1.0)
    return (mag * sign).to(torch.bfloat16)


@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,K,sigma", BF16_CASES)
def test_bf16_encoder_matches_oracle(layout, M, K, sigma):
    NWCWeight, _ = _nwc()
    w = bf16_matrix(M, K, seed=M * 7 + K, scale=sigma)
    c = NWCWeight(w, device="cpu", layout=layout)
    _assert_identical(c, O.encode(bits16(w), O.ELEM_BF16, layout))


@pytest.mark.parametrize("layout", [0, 1])
def test_bf16_encoder_escape_heavy(layout):
    NWCWeight, _ = _nwc()
    w = _spread(40, 1000, seed=5)
    c = NWCWeight(w, device="cpu", layout=layout)
    e = O.encode(bits16(w), O.ELEM_BF16, layout)
    _assert_identical(c, e)
    assert np.array_equal(O.decode(e), bits16(w))


@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,K", FP8_CASES)
def test_fp8_encoder_matches_oracle(layout, M, K):
    NWCWeight, quantize_fp8 = _nwc()
    w = fp8_source(M, K, seed=M)
    c = NWCWeight(w, device="cpu", elem="fp8", layout=layout)
    q, scale = quantize_fp8(w)
    _assert_identical(c, O.encode(q.view(torch.uint8).numpy(), O.ELEM_FP8, layout))
    assert torch.equal(c.scale, scale)
