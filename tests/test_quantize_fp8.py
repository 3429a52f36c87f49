"""Weight-only fp8 quantization pinned bit for bit: nwc_amd.quantize_fp8 (the product, torch ops, reference
nwc/nwc_torch.py:88-94) against the oracle's restatement, whose e4m3 rounding is a brute-force nearest-code search
with ties to the even code (oracle/nwc_oracle.c or_f32_to_e4m3, itself pinned against the e4m3fn definition in
test_oracle_kat.py).

Inputs: the reference test's outlier matrices (tests/test_fp8.py:19), rows whose scale is a power of two so that
every value is an exact midpoint between two e4m3 codes (ties), rows whose scaled maximum lands above 448 before
the clamp, all-zero rows (the 1e-12 floor), tiny rows below the floor, subnormal codes and signed zeros.  The GPU
test runs the same check on CUDA-resident weights, since convert() on a GPU model quantizes there."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import fp8_source

E4M3_POS = np.array([O.lib().or_e4m3_to_f32(c) for c in range(127)], np.float64)   # finite non-negative codes


def _nwc_quantize():
    pytest.importorskip("nwc_amd.nwc_torch", reason="the HIP library is not built")
    from nwc_amd.nwc_torch import quantize_fp8
    return quantize_fp8


def crafted_rows(seed=0):
    """float32 [R, 256] rows that exercise the rounding and the scale rules."""
    rng = np.random.default_rng(seed)
    rows = []
    # ties: scale 2^-k exactly (absmax 448 * 2^-k), every adjacent-code midpoint times 2^-k, both signs
    mids = (E4M3_POS[:-1] + E4M3_POS[1:]) / 2
    for k in (0, 3, 7, 12):
        r = np.zeros(256, np.float64)
        r[0] = 448.0
        r[1:1 + mids.size] = mids
        r[1 + mids.size:1 + 2 * mids.size] = -mids[::-1]
        rows.append((r * 2.0 ** -k).astype(np.float32))
    # just above and below each midpoint (one fp32 ulp)
    for d in (+1, -1):
        m32 = (mids * 2.0 ** -4).astype(np.float32)
        r = np.zeros(256, np.float32)
        r[0] = np.float32(448.0 * 2.0 ** -4)
        r[1:1 + m32.size] = np.nextafter(m32, np.float32(d * np.inf))
        rows.append(r)
    # scaled maximum above 448 before the clamp: fl(a / fl(a / 448)) = 448.00003 for these a
    a = rng.uniform(0.001, 1, 20000).astype(np.float32)
    over = a[(a / (a / np.float32(448))).astype(np.float32) > 448][:255]
    r = np.zeros(256, np.float32)
    r[0] = over.max()
    r[1:1 + over.size] = -over
    rows.append(r)
    # the 1e-12 floor: an all-zero row and a row far below the floor; signed zeros
    rows.append(np.zeros(256, np.float32))
    rows.append((rng.standard_normal(256) * 1e-14).astype(np.float32))
    r = np.zeros(256, np.float32)
    r[0], r[1], r[2] = 1.0, -0.0, 0.0
    rows.append(r)
    # subnormal codes (m * 2^-9 in the scaled domain) and values around them
    r = np.zeros(256, np.float32)
    r[0] = 448.0
    sub = np.arange(1, 8) * 2.0 ** -9
    r[1:8], r[8:15] = sub, -sub
    r[15:22], r[22:29] = sub * 0.74, sub * 1.26
    r[29:33] = [2.0 ** -10, 3 * 2.0 ** -10, 2.0 ** -11, 2.0 ** -30]
    rows.append(r)
    # Gaussian rows with the reference's x40 outliers
    r = (rng.standard_normal((8, 256)) * 0.02).astype(np.float32)
    r.reshape(-1)[::97] *= 40
    rows.extend(r)
    return np.stack(rows).astype(np.float32)


def check_against_oracle(w, device="cpu"):
    quantize_fp8 = _nwc_quantize()
    wf = torch.from_numpy(np.ascontiguousarray(w, np.float32))
    q, scale = quantize_fp8(wf.to(device))
    q_o, scale_o = O.quantize_fp8(w)
    np.testing.assert_array_equal(scale.cpu().numpy().view(np.uint32), scale_o.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().view(torch.uint8).numpy(), q_o)


def test_crafted_rows_bit_exact():
    check_against_oracle(crafted_rows())


def test_ties_go_to_the_even_code():
    """The crafted tie rows: every midpoint quantizes to the even code of its two neighbours (the pin itself)."""
    w = crafted_rows()[:4]
    q, _ = O.quantize_fp8(w)
    n = E4M3_POS.size - 1
    for row in q:
        pos, neg = row[1:1 + n], row[1 + n:1 + 2 * n][::-1]
        lo = np.arange(n)
        assert np.all(pos == np.where(lo % 2 == 0, lo, lo + 1))
        assert np.all(neg == (0x80 | np.where(lo % 2 == 0, lo, lo + 1)))


def test_floor_and_clamp_rows():
    w = crafted_rows()
    q, scale = O.quantize_fp8(w)
    zero = np.nonzero(~w.any(axis=1))[0][0]
    assert scale[zero] == np.float32(np.float32(1e-12) / np.float32(448.0)) and not q[zero].any()
    clamp_row = 6
    assert q[clamp_row][0] == 0x7E and np.all(q[clamp_row][1:] & 0x7F <= 0x7E)


@pytest.mark.parametrize("M,K,seed", [(64, 2048, 0), (257, 1024, 9), (96, 1000, 3)])
def test_reference_fp8_sources_bit_exact(M, K, seed):
    check_against_oracle(fp8_source(M, K, seed=seed).float().numpy())


@pytest.mark.gpu
@pytest.mark.parametrize("M,K,seed", [(257, 1024, 9), (1024, 2560, 4)])
def test_gpu_resident_quantization_bit_exact(cuda, M, K, seed):
    print(f"quantize_fp8 on cuda {M}x{K}", flush=True)
    check_against_oracle(fp8_source(M, K, seed=seed).float().numpy(), device="cuda")
    check_against_oracle(crafted_rows(seed), device="cuda")
