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
    """The oracle's view of an NWCWeight's stored tensors (for or_decode / or_linear): the checkpoint form, with
    layout 0's streams packed back from their fixed slots."""
    t = c.tensors()
    return {"data": t["data"].cpu().numpy(), "bases": t["bases"].cpu().numpy().view(np.uint32),
            "hdr": t["hdr"].cpu().numpy(), "lut": t["lut"].cpu().numpy().view(np.uint32), "low": t["low"].cpu().numpy(),
            "M": c.out_features, "K": c.in_features, "elem": c.elem, "layout": c.layout}


BF16_MAX = float.fromhex("0x1.fep127")


def rne_bf16(v):
    """float64 -> the nearest BF16 value (ties to even), rounded once from float64 and returned as float64.  For
    v = m * 2^e (0.5 <= |m| < 1) the BF16 quantum is 2^(e - 8) (8 significant bits), never below the subnormal
    quantum 2^-133; magnitudes that round past the largest finite BF16 become +-inf; inf and NaN pass through."""
    v = np.asarray(v, np.float64)
    with np.errstate(over="ignore", invalid="ignore"):
        _, e = np.frexp(v)
        q = np.maximum(e - 8, -133)
        r = np.ldexp(np.rint(np.ldexp(v, -q)), q)          # np.rint: round half to even
        r = np.where(np.abs(r) > BF16_MAX, np.copysign(np.inf, v), r)
    return np.where(np.isfinite(v), r, v)


def token_tol(y64, terms=None, absolute=1e-5):
    """The north star's bar before rounding: 1e-3 |y64| + 1e-5, plus 2^-20 sum|w x| where `terms` is given (the fp32
    summation error that cancellation exposes when escapes make the terms much larger than the sum)."""
    t = 1e-3 * np.abs(y64) + absolute
    return t if terms is None else t + 2.0 ** -20 * np.asarray(terms, np.float64)


def check_rne(y, y64, tol, what="token path"):
    """A BF16 output rounded once, to nearest even, from a value within tol of y64: RNE is monotone, so
    RNE(y64 - tol) <= y <= RNE(y64 + tol) (the reference's finalize, nwc_ops.cu:553-565).  A truncating finish, or one
    that rounds before the bias, falls outside this interval for a large share of outputs.  y: BF16 tensor or float
    array; y64: float64 array."""
    if isinstance(y, torch.Tensor):
        y = y.float().cpu().double().numpy()
    y = np.asarray(y, np.float64).ravel()
    y64 = np.asarray(y64, np.float64).ravel()
    tol = np.asarray(tol, np.float64)
    tol = tol.ravel() if tol.size == y64.size else np.broadcast_to(tol, y64.shape)
    lo, hi = rne_bf16(y64 - tol), rne_bf16(y64 + tol)
    bad = ~((y >= lo) & (y <= hi))
    if bad.any():
        i = np.flatnonzero(bad)[:4]
        raise AssertionError(f"{what}: {int(bad.sum())} of {y.size} outputs outside [RNE(y64 - tol), RNE(y64 + tol)], "
                             f"e.g. index {i.tolist()}: y {y[i].tolist()} y64 {y64[i].tolist()} tol {tol[i].tolist()}")


def ref_matvec64(w_bits, x, scale=None, bias_bits=None):
    """float64 matvec on decoded BF16 weights (the closed form the kernels are checked against)."""
    y = O.bf16_to_f64(w_bits) @ np.asarray(x, np.float64)
    if scale is not None:
        y = y * np.asarray(scale, np.float64)
    if bias_bits is not None:
        y = y + O.bf16_to_f64(bias_bits)
    return y


def ref_terms64(w_bits, x, scale=None):
    """sum_k |w x| per row (times |scale|), the size of the terms an fp32 sum adds (cancellation bound)."""
    t = np.abs(O.bf16_to_f64(w_bits)) @ np.abs(np.asarray(x, np.float64))
    return t if scale is None else t * np.abs(np.asarray(scale, np.float64))
