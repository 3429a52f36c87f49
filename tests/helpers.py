"""Shared test inputs: seeded matrices with the reference tests' stressors (escapes, fp8 outliers) and the
oracle-side references."""
import numpy as np
import torch

from oracle import oracle as O


def bf16_matrix(M, K, seed=0, scale=0.02, escapes=True):
    """N(0, scale^2) BF16; every floor(MK/50)-th weight set to 1e30 (tests/test_format_cpu.py:117)."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(M, K, generator=g) * scale).to(torch.bfloat16)
    if escapes:
        w.view(-1)[:: max(1, M * K // 50)] = torch.tensor(1e30, dtype=torch.bfloat16)
    return w


def fp8_source(M, K, seed=0):
    """N(0, 0.02^2) with every 97th weight x40 (tests/test_fp8.py:19), as BF16."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(M, K, generator=g) * 0.02
    w.view(-1)[::97] *= 40
    return w.to(torch.bfloat16)


def bits16(t):
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def oracle_encoding(c):
    """The oracle's view of an NWCWeight's tensors (for or_decode / or_linear)."""
    return {"data": c.data.cpu().numpy(), "bases": c.bases.cpu().numpy().view(np.uint32), "hdr": c.hdr.cpu().numpy(),
            "lut": c.lut.cpu().numpy().view(np.uint32), "low": c.low.cpu().numpy(), "M": c.out_features,
            "K": c.in_features, "elem": c.elem, "layout": c.layout}


def ref_matvec64(w_bits, x, scale=None, bias_bits=None):
    """float64 matvec on decoded BF16 weights (the closed form the kernels are checked against)."""
    y = O.bf16_to_f64(w_bits) @ np.asarray(x, np.float64)
    if scale is not None:
        y = y * np.asarray(scale, np.float64)
    if bias_bits is not None:
        y = y + O.bf16_to_f64(bias_bits)
    return y
