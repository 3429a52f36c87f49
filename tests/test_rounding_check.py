"""CPU pins of the BF16 output check the token-path tests use (tests/helpers.py check_rne): the host rounding
rne_bf16 against torch's float32 -> bfloat16 conversion (round to nearest even) and hand-derived ties, and the
check itself against planted finishing mistakes (a truncating finish, rounding before the bias), which it must
reject, while the reference's finish (one RNE after scale and bias, nwc_ops.cu:553-565) passes."""
import numpy as np
import torch

from tests.helpers import check_rne, rne_bf16, token_tol


def _torch_rne(v32):
    return torch.from_numpy(np.asarray(v32, np.float32)).to(torch.bfloat16).double().numpy()


def test_rne_matches_torch_on_float32_values():
    g = np.random.default_rng(0)
    v = np.concatenate([g.standard_normal(200000) * 10.0 ** g.integers(-40, 38, 200000),
                        g.standard_normal(20000) * 1e-39,            # float32 subnormals
                        np.array([0.0, -0.0, 3.3895e38, -3.3895e38, 3.4e38, 1e-45, -1e-45])])
    v32 = v.astype(np.float32)
    assert np.array_equal(rne_bf16(v32.astype(np.float64)), _torch_rne(v32), equal_nan=True)


def test_rne_ties_and_single_rounding():
    u = 2.0 ** -7                                               # BF16 spacing in [1, 2)
    assert rne_bf16(1 + u / 2) == 1.0                          # tie -> even mantissa
    assert rne_bf16(1 + 3 * u / 2) == 1 + 2 * u                # tie -> even mantissa (up)
    assert rne_bf16(-(1 + u / 2)) == -1.0
    # one rounding from float64: just above a tie rounds up, although float32 would first round it onto the tie
    v = 1 + u / 2 + 2.0 ** -30
    assert rne_bf16(v) == 1 + u
    assert _torch_rne(np.float32(v))[()] == 1.0
    assert rne_bf16(2.0 ** -133) == 2.0 ** -133 and rne_bf16(2.0 ** -134) == 0.0 and rne_bf16(1.5 * 2.0 ** -134) == 2.0 ** -133
    assert np.isinf(rne_bf16(3.4e38)) and rne_bf16(3.3895e38) == float.fromhex("0x1.fep127")
    assert np.isnan(rne_bf16(np.nan)) and rne_bf16(-np.inf) == -np.inf


def _sums(n=20000, K=2560, seed=1):
    """float64 results and fp32-accumulated sums of N(0, 0.02^2) BF16 rows times N(0, 1) BF16 activations."""
    g = torch.Generator().manual_seed(seed)
    w = (torch.randn(n // 100, K, generator=g) * 0.02).to(torch.bfloat16)
    x = torch.randn(100, K, generator=g).to(torch.bfloat16)
    y64 = (w.double() @ x.double().T).numpy().ravel()
    s32 = (w.float() @ x.float().T).numpy().ravel()
    bias = (torch.rand(y64.size, generator=g) - 0.5).to(torch.bfloat16).double().numpy()
    return y64, s32, bias


def test_check_accepts_the_reference_finish():
    y64, s32, bias = _sums()
    y = _torch_rne(s32.astype(np.float64) + bias)              # fp32 sum + bias, one RNE
    check_rne(y, y64 + bias, token_tol(y64 + bias))


def test_check_rejects_a_truncating_finish():
    y64, s32, _ = _sums()
    trunc = (s32.astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32).astype(np.float64)
    try:
        check_rne(trunc, y64, token_tol(y64))
    except AssertionError as e:
        assert "outside" in str(e)
    else:
        raise AssertionError("a truncating finish passed the check")


def test_check_rejects_rounding_before_the_bias():
    y64, s32, bias = _sums()
    early = _torch_rne(_torch_rne(s32) + bias)                  # RNE(RNE(sum) + bias): two roundings
    try:
        check_rne(early, y64 + bias, token_tol(y64 + bias))
    except AssertionError:
        pass
    else:
        raise AssertionError("rounding before the bias passed the check")
