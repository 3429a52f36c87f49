"""GPU parity at the BASELINE.json config workloads, at their real sizes, through the C ABI.

  configs[0]  9728 x 2560 BF16 layout 0 (the reference CPU path's single layer)
  configs[1]  the Qwen3-0.6B matrices, layout 0, token path with the row index and the 13-bit table
  configs[2]  the Qwen3-4B matrices, 512-token prefill in layouts 0 and 1, plus the tied 151936 x 2560 lm_head
  configs[3]  the Qwen3-4B gate_up and down as weight-only fp8, layouts 0 and 1
  configs[4]  64 seeded token ids gathered from a 152064 x 3584 embedding table, layouts 0, 1 and 2
and the reference's own token entry point nwc_linear_bf16, bound with the reference bridge's argument types
(nwc/nwc_torch.py:58-77), for every layout and element type with scale and bias.

Bars: decoded weights and gathered rows bit-exact against the original weights (and, for configs[0], against the
oracle's decode of the same tensors); token path rounded to nearest even from within 1e-3 |y| + 1e-5 of a float64
matvec on the decoded weights (RNE(y64 - tol) <= y <= RNE(y64 + tol)); fp32 path within 1e-3 |y| + 1e-5; prefill equal to the same GEMM on the original BF16 weights (the same
GEMM on bit-identical operands)."""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as O
from tests.helpers import bits16, check_rne, fp8_source, oracle_encoding, ref_matvec64, token_tol

pytestmark = pytest.mark.gpu

QWEN3_06B = {"qkv": (4096, 1024), "o": (1024, 2048), "gate_up": (6144, 1024), "down": (1024, 3072)}
QWEN3_4B = {"qkv": (6144, 2560), "o": (2560, 4096), "gate_up": (19456, 2560), "down": (2560, 9728)}


def _nwc():
    from nwc_amd.nwc_torch import NWCLinear, NWCWeight, quantize_fp8
    return NWCWeight, NWCLinear, quantize_fp8


def gaussian_bf16(M, K, seed):
    """The north star's weights: N(0, 0.02^2) from a seed, as BF16."""
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(M, K, generator=g) * 0.02).to(torch.bfloat16)


def activations(K, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(K, generator=g).to(torch.bfloat16)


def y_exact(w_cuda_bf16, x, scale=None, bias=None):
    """float64 matvec on the GPU over the decoded weights (rocBLAS dgemv; exact to ~1e-16 relative), for matrices too
    large for a host float64 copy."""
    y = w_cuda_bf16.double() @ x.cuda().double()
    if scale is not None:
        y = y * scale.cuda().double()
    if bias is not None:
        y = y + bias.cuda().double()
    return y.cpu().numpy()


def check_token(y_bf16, y64):
    check_rne(y_bf16, y64, token_tol(y64))


def check_f32(y, y64):
    err = np.abs(y.cpu().double().numpy() - y64)
    tol = 1e-3 * np.abs(y64) + 1e-5
    assert np.all(err <= tol), f"fp32 path: worst excess {np.max(err - tol):.3e}"


def test_config0_single_layer(cuda):
    """decoded W bit-exact (original and oracle decode), y = W x with N(0,1) x."""
    NWCWeight, _, _ = _nwc()
    print("configs[0] 9728x2560 layout 0", flush=True)
    w = gaussian_bf16(9728, 2560, seed=7)
    c = NWCWeight(w, device="cuda", layout=0)
    d = c.dequant()
    assert torch.equal(d.cpu().view(torch.int16), w.view(torch.int16))
    assert np.array_equal(O.decode(oracle_encoding(c)), bits16(w))
    x = activations(2560, seed=8)
    y64 = y_exact(d, x.float())
    check_token(c.linear_bf16(x.cuda(), None), y64)            # BF16 x, row index + 13-bit table
    check_token(c.linear_bf16(x.float().cuda(), None), y64)    # fp32 x, the reference entry point
    check_f32(c.matvec(x.float().cuda()), y64)
    # the oracle's own CPU decode + fp32 matvec (the CPU baseline's path) meets the same bar
    check_f32(torch.from_numpy(O.linear(oracle_encoding(c), x.float().numpy())), y64)


@pytest.mark.parametrize("name", list(QWEN3_06B))
def test_config1_qwen3_06b_matrices(cuda, name):
    """each Qwen3-0.6B matrix through nwc_linear_xbf16 with the row index and the 13-bit table."""
    NWCWeight, _, _ = _nwc()
    M, K = QWEN3_06B[name]
    print(f"configs[1] 0.6B {name} {M}x{K}", flush=True)
    w = gaussian_bf16(M, K, seed=M + K)
    c = NWCWeight(w, device="cuda", layout=0)
    assert c.row_index() is not None and c.seq_table() is not None
    d = c.dequant()
    assert torch.equal(d.cpu().view(torch.int16), w.view(torch.int16))
    g = torch.Generator().manual_seed(3)
    for _ in range(3):
        x = torch.randn(K, generator=g).to(torch.bfloat16)
        bias = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)
        check_token(c.linear_bf16(x.cuda(), bias.cuda()), y_exact(d, x.float(), bias=bias.float()))


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("name", list(QWEN3_4B))
def test_config2_prefill_512(cuda, name, layout):
    """a 512-token prefill (dequantization + the GEMM NWCLinear picks for the shape) equals the same GEMM
    on the resident BF16 weights."""
    from nwc_amd.nwc_torch import linear_dequantized
    NWCWeight, NWCLinear, _ = _nwc()
    M, K = QWEN3_4B[name]
    print(f"configs[2] prefill 512 {name} {M}x{K} layout {layout}", flush=True)
    w = gaussian_bf16(M, K, seed=M * 3 + K + layout)
    lin = NWCLinear(w=NWCWeight(w, device="cuda", layout=layout), device="cuda")
    g = torch.Generator().manual_seed(11)
    x = torch.randn(1, 512, K, generator=g).to(torch.bfloat16).cuda()
    torch.backends.cuda.preferred_blas_library("hipblaslt")
    assert torch.equal(lin(x), linear_dequantized(x, w.cuda()))
    check_token(lin(x[:, :1]).view(-1), y_exact(w.cuda(), x[0, 0].float().cpu()))


def test_config2_tied_lm_head(cuda):
    """The tied 151936 x 2560 embedding / lm_head of Qwen3-4B, the largest matvec of a token: token path with BF16
    and fp32 activations, fp32 path, bit-exact decode, and the tied lookup."""
    NWCWeight, NWCLinear, _ = _nwc()
    from nwc_amd.nwc_torch import NWCEmbedding
    M, K = 151936, 2560
    print(f"configs[2] lm_head {M}x{K}", flush=True)
    w = gaussian_bf16(M, K, seed=2024)
    c = NWCWeight(w, device="cuda", layout=0)
    d = c.dequant()
    assert torch.equal(d.view(torch.int16), w.cuda().view(torch.int16))
    x = activations(K, seed=5)
    y64 = y_exact(d, x.float())
    lin = NWCLinear(w=c, device="cuda")
    check_token(lin(x.view(1, 1, K).cuda()).view(-1), y64)
    check_token(c.linear_bf16(x.float().cuda(), None), y64)
    check_f32(c.matvec(x.float().cuda()), y64)
    emb = NWCEmbedding(w=c)
    ids = torch.tensor([0, M - 1, M // 2, 151643, 151645, 12345], dtype=torch.int64)
    assert torch.equal(emb(ids.cuda()).cpu().view(torch.int16), w[ids].view(torch.int16))


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("name", ["gate_up", "down"])
def test_config3_fp8_large(cuda, name, layout):
    """weight-only fp8 at the 4B gate_up and down shapes: codes bit-exact, token (with and without a bias)
    and fp32 paths."""
    NWCWeight, _, quantize_fp8 = _nwc()
    M, K = QWEN3_4B[name]
    print(f"configs[3] fp8 {name} {M}x{K} layout {layout}", flush=True)
    w = gaussian_bf16(M, K, seed=M + 2 * K)
    q, scale = quantize_fp8(w)
    c = NWCWeight(w, device="cuda", elem="fp8", layout=layout)
    d = c.dequant()
    assert torch.equal(d.cpu().view(torch.int16), q.to(torch.bfloat16).view(torch.int16))
    q2, s2 = c.dequant_fp8()
    assert torch.equal(q2.cpu().view(torch.uint8), q.view(torch.uint8)) and torch.equal(s2.cpu(), scale)
    x = activations(K, seed=6)
    y64 = y_exact(d, x.float(), scale=scale)
    check_token(c.linear_bf16(x.cuda(), None), y64)
    check_f32(c.matvec(x.float().cuda()), y64)
    bias = (torch.rand(M, generator=torch.Generator().manual_seed(K)) - 0.5).to(torch.bfloat16)
    check_token(c.linear_bf16(x.cuda(), bias.cuda()), y_exact(d, x.float(), scale=scale, bias=bias.float()))


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_config4_embedding_gather_64(cuda, layout):
    """64 uniform-random (seeded) ids from the untied 152064 x 3584 Qwen2.5-7B table."""
    NWCWeight, _, _ = _nwc()
    M, K = 152064, 3584
    print(f"configs[4] gather 64 of {M}x{K} layout {layout}", flush=True)
    w = gaussian_bf16(M, K, seed=77)
    c = NWCWeight(w, device="cuda", layout=layout)
    g = torch.Generator().manual_seed(64)
    ids = torch.randint(0, M, (64,), generator=g)
    assert torch.equal(c.gather(ids.cuda()).cpu().view(torch.int16), w[ids].view(torch.int16))
    ids2 = torch.tensor([0, M - 1, M // 2, 1, M - 2])
    assert torch.equal(c.gather(ids2.cuda()).cpu().view(torch.int16), w[ids2].view(torch.int16))


def _reference_binding():
    """nwc_linear_bf16 bound the way the reference bridge binds it (nwc/nwc_torch.py:58-77 with ELEM): eleven
    pointers, then n, block, K and elem."""
    from nwc_amd._abi import LIB_PATH
    lib = ctypes.CDLL(LIB_PATH)
    P, U64, U32 = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32
    lib.nwc_linear_bf16.restype = ctypes.c_int
    lib.nwc_linear_bf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, U64, U32, U32, ctypes.c_int]
    return lib


@pytest.mark.parametrize("elem", ["bf16", "fp8"])
@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,K", [(1001, 1000), (2560, 4096)])
def test_reference_entry_point_all_layouts(cuda, M, K, layout, elem):
    """The reference's token entry point with its own argument conventions: layout 0 takes fp32 x [K16], layouts
    1/2 BF16 x [K32] through the same float pointer; scale (fp8), bias and the reference's scratch buffer passed."""
    NWCWeight, _, quantize_fp8 = _nwc()
    print(f"nwc_linear_bf16 layout {layout} {elem} {M}x{K}", flush=True)
    lib = _reference_binding()
    w = gaussian_bf16(M, K, seed=M + layout)
    c = NWCWeight(w, device="cuda", elem=elem, layout=layout)
    g = torch.Generator().manual_seed(9)
    x = torch.randn(K, generator=g).to(torch.bfloat16)
    bias = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16).cuda()
    if layout == 0:
        xin = F.pad(x.float(), (0, c.K16 - K)).cuda()
    else:
        xin = F.pad(x, (0, -K % 32)).cuda()
    y = torch.empty(M, dtype=torch.bfloat16, device="cuda")
    p = lambda t: None if t is None else ctypes.c_void_p(t.data_ptr())
    rc = lib.nwc_linear_bf16(ctypes.c_void_p(torch.cuda.current_stream().cuda_stream), p(c.data), p(c.bases), p(c.hdr),
                             p(c.lut), p(c.low), p(xin), p(bias), p(c.scale), p(c.scratch), p(y), c.n, c.block, K,
                             c.code)
    assert rc == 0
    ref_w = c.dequant()
    if elem == "bf16":
        assert torch.equal(ref_w.cpu().view(torch.int16), w.view(torch.int16))
    else:
        assert torch.equal(ref_w.cpu().view(torch.int16), quantize_fp8(w)[0].to(torch.bfloat16).view(torch.int16))
    check_token(y, y_exact(ref_w, x.float(), scale=c.scale, bias=bias.float()))


BASELINE_SHAPES = dict(QWEN3_4B, lm_head=(151936, 2560))


@pytest.mark.parametrize("name", list(BASELINE_SHAPES))
def test_uncompressed_baselines_at_config_sizes(cuda, name):
    """The uncompressed matvecs the compressed path is measured against, at the sizes bench.py times them, against
    float64: nwc_ref_fp8 on the quantized weights (its bandwidth plans at these shapes: <4,2> qkv, <4,1> o, <8,2>
    gate_up, <4,3> down, <8,5> lm_head) and nwc_ref_bf16 on the BF16 weights; also ragged shapes that take the
    byte-wise fallbacks."""
    from nwc_amd.nwc_torch import quantize_fp8, ref_bf16_matvec, ref_fp8_matvec
    M, K = BASELINE_SHAPES[name]
    print(f"baselines {name} {M}x{K}", flush=True)
    w = gaussian_bf16(M, K, seed=M + 5 * K)
    x = activations(K, seed=K)
    wc = w.cuda()
    y64 = y_exact(wc, x.float())
    check_rne(ref_bf16_matvec(wc, x.cuda()), y64, token_tol(y64), "nwc_ref_bf16")
    q, scale = quantize_fp8(wc)
    y64 = y_exact(q.to(torch.bfloat16), x.float(), scale=scale)
    check_rne(ref_fp8_matvec(q, scale, x.float().cuda()), y64, token_tol(y64), "nwc_ref_fp8")


@pytest.mark.parametrize("M,K", [(13, 40), (3, 4097), (1001, 1000), (257, 1030)])
def test_uncompressed_baselines_ragged(cuda, M, K):
    from nwc_amd.nwc_torch import quantize_fp8, ref_bf16_matvec, ref_fp8_matvec
    w = gaussian_bf16(M, K, seed=M * K)
    x = activations(K, seed=M)
    y64 = y_exact(w.cuda(), x.float())
    check_rne(ref_bf16_matvec(w.cuda(), x.cuda()), y64, token_tol(y64), "nwc_ref_bf16")
    q, scale = quantize_fp8(w.cuda())
    y64 = y_exact(q.to(torch.bfloat16), x.float(), scale=scale)
    check_rne(ref_fp8_matvec(q, scale, x.float().cuda()), y64, token_tol(y64), "nwc_ref_fp8")
