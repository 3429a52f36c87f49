"""GPU parity of the gfx950 kernels against the oracle and against closed forms, through the C ABI (nwc_amd).

Bars:
  * decoded weights bit-exact: dequant and gather equal the original BF16 / fp8 values and the oracle's decode;
  * fp32 path (nwc_matvec): |y - y64| <= 1e-3 |y64| + 1e-5 * (sigma / 0.02), y64 = float64 matvec on the decoded
    weights (sigma = weight scale of the test matrix; 1e-5 absolute at the north star's N(0, 0.02^2));
  * token path (BF16 out): rounded once, to nearest even, from a value within 1e-3 |y64| + the same absolute term
    of y64: RNE(y64 - tol) <= y <= RNE(y64 + tol) (tests/helpers.py check_rne; the reference's finalize,
    nwc_ops.cu:553-565).
Shapes and stressors follow the reference tests (tests/test_format_cpu.py:127-131, test_k.py:10-11, test_fp8.py:19,44).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_matrix, bits16, check_rne, fp8_source, oracle_encoding, ref_matvec64, token_tol

pytestmark = pytest.mark.gpu

SHAPES = [(8, 512, 0.02), (13, 40, 0.02), (3, 4097, 0.02), (100, 1000, 1.0), (64, 2048, 0.02), (17, 520, 0.02),
          (1001, 1000, 0.02), (8, 16, 0.02), (1, 1, 0.02)]
FP8_SHAPES = [(8, 512), (13, 40), (3, 4097), (1001, 1000), (2560, 4096), (6144, 2560)]   # tests/test_fp8.py:45
LAYOUTS = [0, 1, 2]


def _nwc():
    from nwc_amd.nwc_torch import NWCWeight, ref_fp8_matvec, quantize_fp8
    return NWCWeight, ref_fp8_matvec, quantize_fp8


def _check_f32(y, y64, sigma):
    err = np.abs(np.asarray(y, np.float64) - y64)
    tol = 1e-3 * np.abs(y64) + 1e-5 * max(1.0, sigma / 0.02)
    assert np.all(err <= tol), f"fp32 path: worst excess {np.max(err - tol):.3e}"


def _check_bf16(y_bf16, y64, sigma):
    check_rne(y_bf16, y64, token_tol(y64, absolute=1e-5 * max(1.0, sigma / 0.02)))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("M,K,sigma", SHAPES)
def test_bf16_all_paths(cuda, layout, M, K, sigma):
    NWCWeight, _, _ = _nwc()
    print(f"bf16 layout {layout} {M}x{K}", flush=True)
    w = bf16_matrix(M, K, seed=M * 7 + K, scale=sigma)
    c = NWCWeight(w, device="cuda", layout=layout)
    wb = bits16(w)
    # decoded weights: bit-exact against the original and against the oracle decoding the same tensors
    d = c.dequant().cpu()
    assert torch.equal(d.view(torch.int16), w.view(torch.int16))
    assert np.array_equal(O.decode(oracle_encoding(c)), wb)
    # token path with bias
    g = torch.Generator().manual_seed(1)
    x = torch.randn(K, generator=g).to(torch.bfloat16)
    bias = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)
    y = c.linear_bf16(x.cuda(), bias.cuda())
    y64 = ref_matvec64(wb, x.float().numpy(), bias_bits=bits16(bias))
    _check_bf16(y, y64, sigma)
    # token path with fp32 activations (reference ABI for layout 0) and without bias
    y2 = c.linear_bf16(x.float().cuda(), None)
    _check_bf16(y2, ref_matvec64(wb, x.float().numpy()), sigma)
    # fp32 path with non-BF16 activations
    xf = torch.rand(K, generator=g) - 0.5
    y32 = c.matvec(xf.cuda()).cpu().numpy()
    _check_f32(y32, ref_matvec64(wb, xf.numpy()), sigma)
    # gather, including the first, last and middle rows
    ids = torch.cat([torch.tensor([0, M - 1, M // 2]), torch.randint(0, M, (13,), generator=g)])
    rows = c.gather(ids.cuda()).cpu()
    assert torch.equal(rows.view(torch.int16), w[ids].view(torch.int16))


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("M,K", FP8_SHAPES)
def test_fp8_all_paths(cuda, layout, M, K):
    NWCWeight, ref_fp8_matvec, quantize_fp8 = _nwc()
    print(f"fp8 layout {layout} {M}x{K}", flush=True)
    w = fp8_source(M, K, seed=M)
    q, scale = quantize_fp8(w)
    ref_vals = q.to(torch.bfloat16)                     # unscaled fp8 values, exact in BF16
    c = NWCWeight(w, device="cuda", elem="fp8", layout=layout)
    assert torch.equal(c.dequant().cpu().view(torch.int16), ref_vals.view(torch.int16))
    q2, s2 = c.dequant_fp8()
    assert torch.equal(q2.cpu().view(torch.uint8), q.view(torch.uint8))
    assert torch.equal(s2.cpu(), scale)
    assert np.array_equal(O.decode(oracle_encoding(c)), bits16(ref_vals))
    g = torch.Generator().manual_seed(2)
    x = torch.randn(K, generator=g)
    vb = bits16(ref_vals)
    y64 = ref_matvec64(vb, x.to(torch.bfloat16).float().numpy(), scale=scale.numpy())
    _check_bf16(c.linear_bf16(x.to(torch.bfloat16).cuda(), None), y64, 0.02)
    y32 = c.matvec(x.cuda()).cpu().numpy()
    _check_f32(y32, ref_matvec64(vb, x.numpy(), scale=scale.numpy()), 0.02)
    ids = torch.randint(0, M, (7,), generator=g)
    assert torch.equal(c.gather(ids.cuda()).cpu().view(torch.int16), ref_vals[ids].view(torch.int16))
    yr = ref_fp8_matvec(q.cuda().contiguous(), scale.cuda(), x.cuda())
    _check_bf16(yr, ref_matvec64(vb, x.numpy(), scale=scale.numpy()), 0.02)


def test_fp8_nan_rejected():
    NWCWeight, _, _ = _nwc()
    bad = torch.full((8, 512), float("nan")).to(torch.float8_e4m3fn)
    with pytest.raises(ValueError):
        NWCWeight(bad, device="cpu", elem="fp8", scale=torch.ones(8))


def test_fp8_hardware_conversion_exhaustive(cuda):
    """The native fp8 baseline converts with v_cvt_pk_f32_fp8; every finite e4m3fn code must give its exact value
    (closed form from the definition, oracle or_e4m3_to_f32)."""
    _, ref_fp8_matvec, _ = _nwc()
    codes = np.array([c for c in range(256) if (c & 0x7F) != 0x7F], np.uint8)
    M, K = codes.size, 32
    w = np.zeros((M, K), np.uint8)
    w[:, 5] = codes
    x = torch.zeros(K)
    x[5] = 1.0
    y = ref_fp8_matvec(torch.from_numpy(w).cuda().view(torch.float8_e4m3fn), torch.ones(M).cuda(), x.cuda()).cpu()
    exact = O.e4m3_to_f32(codes)
    # values, not bits: a matvec returns +0 for the -0 code (0x80)
    assert np.array_equal(y.float().numpy(), exact)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_full_size_qwen3_4b_gate_up(cuda, layout):
    """BASELINE config 3's largest matrix at its real shape: dequant bit-exact and the token path against a torch
    fp32 matvec on the GPU (size-independent checks; the oracle covers the small shapes)."""
    NWCWeight, _, _ = _nwc()
    M, K = 19456, 2560
    print(f"full size layout {layout}", flush=True)
    w = bf16_matrix(M, K, seed=11, escapes=False)
    c = NWCWeight(w, device="cuda", layout=layout)
    wc = w.cuda()
    assert torch.equal(c.dequant().view(torch.int16), wc.view(torch.int16))
    x = torch.randn(K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).cuda()
    y = c.linear_bf16(x, None).double().cpu().numpy()
    y64 = (wc.double() @ x.double()).cpu().numpy()
    check_rne(y, y64, token_tol(y64))
    y32 = c.matvec(x.float()).double().cpu().numpy()
    assert np.all(np.abs(y32 - y64) <= 1e-3 * np.abs(y64) + 1e-5)


def _row_index_cpu(w, lut):
    """Bit positions of rows 2, 4, 6 in every layout-0 lane stream, from the code lengths (rank r: r + 2 bits, rank
    >= 15: 24-bit escape, fillers past M or K: rank 0; docs/format.md section 3) with exp_of_rank read back from the
    table as the decoders do."""
    M, K = w.shape
    K16, CB = (K + 15) // 16 * 16, (K + 511) // 512
    Mp = (M + 7) // 8 * 8
    hb = np.zeros((Mp, CB * 512), np.int64)
    hb[:M, :K] = (bits16(w).reshape(M, K).astype(np.int64) >> 8) & 0x7F
    lut = lut.astype(np.uint32)
    eor = []
    for q in range(15):
        src = (1 << (11 - q)) if q < 11 else (q - 11) >> 1
        sh = 8 if (q < 11 or (q & 1)) else 16
        eor.append(int((lut[src] >> sh) & 0x7F))
    rank = np.full(128, 15)
    for r in range(14, -1, -1):
        rank[eor[r]] = r
    ln = np.where(rank[hb] < 15, rank[hb] + 2, 24)
    ln[M:, :] = 2                                                      # filler weights are coded as rank 0, sign 0
    ln[:, K:] = 2
    ln = ln.reshape(Mp // 8, 8, CB, 32, 16).sum(-1)                 # bits per (group, row, block column, lane)
    cum = np.cumsum(ln, axis=1)                                        # after rows 0..r
    pos = cum[:, [1, 3, 5], :, :]                                      # starts of rows 2, 4, 6
    return pos.transpose(0, 2, 1, 3).reshape(-1, 3, 32), K16           # [block = group * CB + cb][j][lane]


def _code_lengths(w, lut, rows):
    """Code length of every weight, padded to whole row groups and column blocks (fillers: 2 bits)."""
    M, K = w.shape
    CB = (K + 511) // 512
    Mp = (M + rows - 1) // rows * rows
    hb = np.zeros((Mp, CB * 512), np.int64)
    hb[:M, :K] = (bits16(w).reshape(M, K).astype(np.int64) >> 8) & 0x7F
    lut = lut.astype(np.uint32)
    eor = []
    for q in range(15):
        src = (1 << (11 - q)) if q < 11 else (q - 11) >> 1
        sh = 8 if (q < 11 or (q & 1)) else 16
        eor.append(int((lut[src] >> sh) & 0x7F))
    rank = np.full(128, 15)
    for r in range(14, -1, -1):
        rank[eor[r]] = r
    ln = np.where(rank[hb] < 15, rank[hb] + 2, 24)
    ln[M:, :] = 2
    ln[:, K:] = 2
    return ln


def _row_index_cpu_l1(w, lut):
    """Bit positions of super-chunks 4, 8, 12 in every layout-1 lane stream (lane L = (r, q) codes, per super-chunk,
    16 weights of rows r and r + 8: docs/format.md section 4c), or the lane's end where the block codes fewer."""
    M, K = w.shape
    K16, CB = (K + 15) // 16 * 16, (K + 511) // 512
    nsl = ((K16 - (CB - 1) * 512) // 16 + 1) // 2
    ln = _code_lengths(w, lut, 16)
    G = ln.shape[0] // 16
    L5 = ln.reshape(G, 16, CB, 16, 32)                                 # [group, row, block column, super-chunk, column]
    bits = np.zeros((G, CB, 16, 8, 4), np.int64)                       # [group, cb, sc, r, q]
    for j in range(16):
        roff = 8 * ((j >> 1) & 1)
        coff = 4 * ((j >> 3) & 1) + 2 * ((j >> 2) & 1) + (j & 1)
        for q in range(4):
            bits[:, :, :, :, q] += L5[:, roff:roff + 8, :, :, 8 * q + coff].transpose(0, 2, 3, 1)
    bits[:, CB - 1, nsl:] = 0                                          # super-chunks the last block does not code
    cum = np.cumsum(bits, axis=2).reshape(G, CB, 16, 32)               # after super-chunks 0..sc, lane 4r + q
    pos = cum[:, :, [3, 7, 11], :]
    return pos.reshape(-1, 3, 32)


@pytest.mark.parametrize("M,K,escapes", [(64, 2048, False), (100, 1000, True), (13, 40, True), (300, 2560, False)])
def test_row_index_values_layout1(cuda, M, K, escapes):
    NWCWeight, _, _ = _nwc()
    w = bf16_matrix(M, K, seed=M + K + 1, escapes=escapes)
    c = NWCWeight(w, device="cuda", layout=1)
    got = c.row_index().cpu().numpy().view(np.uint16).reshape(-1, 3, 32).astype(np.int64)
    want = _row_index_cpu_l1(w, c.lut.cpu().numpy().view(np.uint32))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("M,K,escapes", [(64, 2048, False), (100, 1000, True), (13, 40, True), (300, 2560, False)])
def test_row_index_values(cuda, M, K, escapes):
    NWCWeight, _, _ = _nwc()
    w = bf16_matrix(M, K, seed=M + K, escapes=escapes)
    c = NWCWeight(w, device="cuda", layout=0)
    got = c.row_index().cpu().numpy().view(np.uint16).reshape(-1, 3, 32).astype(np.int64)
    want, K16 = _row_index_cpu(w, c.lut.cpu().numpy().view(np.uint32))
    CB = (K + 511) // 512
    lane_ok = (np.arange(CB)[:, None] * 512 + np.arange(32)[None, :] * 16) < K16        # lanes with columns
    mask = np.broadcast_to(np.tile(lane_ok, ((M + 7) // 8, 1))[:, None, :], want.shape)
    assert np.array_equal(got[mask], want[mask])


@pytest.mark.parametrize("layout,M,K,split,escapes", [
    (0, 2560, 4096, 2, "none"), (0, 6144, 2560, 2, "none"), (0, 1003, 1100, 4, "none"), (0, 2560, 4096, 2, "sparse"),
    (0, 2560, 4096, 2, "dense"), (0, 6144, 2560, 2, "dense"), (0, 1003, 1100, 4, "dense"), (0, 2560, 4096, 2, "heavy"),
    (0, 6144, 2560, 2, "heavy"), (0, 19456, 2560, 1, "heavy"), (0, 2560, 9728, 1, "dense"), (0, 151936, 256, 1, "none"),
    (0, 9728, 2560, 2, "none"), (0, 9728, 2560, 2, "heavy"),  # two per CU, two half-waves per block on 30 half-waves
    (1, 2560, 4096, 4, "none"), (1, 6144, 2560, 4, "none"), (1, 19456, 2560, 2, "none"), (1, 1003, 1100, 4, "none"),
    (1, 2560, 4096, 4, "dense"), (1, 1003, 1100, 4, "dense"),
    (1, 2560, 9728, 4, "none"), (1, 2560, 9728, 4, "dense"), (1, 1003, 9000, 4, "none"), (1, 2560, 4096, 4, "heavy"),
    (1, 2560, 9728, 4, "heavy"), (1, 151936, 2560, 2, "none")])
def test_token_path_with_and_without_row_index(cuda, layout, M, K, split, escapes):
    """The split decode (layout 0: four or two half-waves per block, each reducing 2 or 4 rows; layout 1: super-chunk
    ranges 4 or 8 long, and for K > 8192 several such items per half-wave) against the whole-block decode: o_proj, qkv_proj, gate_up and down shapes on 256 CUs,
    ragged matrices (layout 1: a last column block of three or two super-chunks), and escape runs (24-bit codes) dense
    enough ("heavy": three whole row groups) that tiles do not fit their LDS region and decode from global memory."""
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    NWCWeight, _, _ = _nwc()
    w = bf16_matrix(M, K, seed=77, escapes=escapes == "sparse")
    if escapes == "dense":                    # 24-bit codes: whole lanes of rows 0-7, 9, 13 and 16-23 are escapes
        big = torch.tensor(1e30, dtype=torch.bfloat16)
        w[0:8, 0:64] = big
        w[9, 512:700] = -big
        w[13, 1024:1100] = big
        w[16:24, 16:32] = -big
    if escapes == "heavy":                    # rows 0-23 all escapes: the first workgroups' streams exceed their region
        sign = torch.randint(0, 2, (24, K), generator=torch.Generator().manual_seed(5)) * 2 - 1
        w[0:24] = (sign * 1e30).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=layout)
    assert _lib.nwc_token_split(c.n, K, c.code, 1) == split
    assert _lib.nwc_token_split(c.n, K, c.code, 0) == 1
    x = torch.randn(K, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16).cuda()
    xin = c._padded(x).contiguous()                             # zero-padded to K16 (layout 0) or K32 (layout 1)
    ys = []
    host = torch.zeros(c.seq_table().numel(), dtype=torch.int32)
    lut = c.lut.cpu()
    assert _lib.nwc_seq_table(_ptr(lut), c.code, _ptr(host)) == 0
    assert torch.equal(c.seq_table().cpu(), host)            # the device copy of the 13-bit table is the host build
    combos = [(c.row_index(), None), (None, None), (c.row_index(), c.seq_table()), (None, c.seq_table())]
    for ri, st in combos:
        y = torch.empty(M, dtype=torch.bfloat16, device="cuda")
        err = _lib.nwc_linear_xbf16(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                                    _ptr(ri) if ri is not None else None, _ptr(st) if st is not None else None,
                                    _ptr(xin), None, None, _ptr(y), c.n, K, c.code)
        assert err == 0
        ys.append(y.double().cpu().numpy())
    assert np.array_equal(ys[2], ys[0]) and np.array_equal(ys[3], ys[1])   # the table changes no sum: bit-identical
    if layout == 0:                         # nor does layout 0's split: each row's lanes and blocks are summed in one order
        assert np.array_equal(ys[0], ys[1])
    y64 = (w.cuda().double() @ x.double()).cpu().numpy()
    for y in ys:
        check_rne(y, y64, token_tol(y64))


@pytest.mark.parametrize("M,K,elem,escapes", [
    (2560, 4096, "bf16", "none"), (2560, 9728, "bf16", "dense"), (2560, 9728, "fp8", "none"), (2560, 1000, "bf16", "sparse"),
    (2880, 2048, "bf16", "none"), (2880, 9728, "bf16", "heavy"), (2600, 4096, "fp8", "dense"), (2050, 512, "bf16", "none")])
def test_split_tail_plan(cuda, M, K, elem, escapes):
    """Matrices of one to two row groups per CU take k_layout0t (one whole row group per CU, the rest cut into
    quarters or halves of their rows): results bit-identical to the whole-block decode without the row index (every
    row's lanes and column blocks are summed in one order), and rounded from within 1e-3 of float64, with scale and
    bias; shapes with 320 row groups (quarters), 360 (halves), ragged K, escapes that overflow the staged region, and
    fp8.  Dequantization takes the same plan: the original bits, equal to the whole-block kernel's."""
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    NWCWeight, _, quantize_fp8 = _nwc()
    print(f"tail plan {M}x{K} {elem} {escapes}", flush=True)
    w = bf16_matrix(M, K, seed=M + K + 3, escapes=escapes == "sparse")
    if escapes == "dense":
        big = torch.tensor(1e30, dtype=torch.bfloat16)
        w[M - 20:M - 12, 0:64] = big
        w[M - 7, 512:700] = -big
    if escapes == "heavy":                    # the last 24 rows all escapes: the tail's streams exceed their region
        sign = torch.randint(0, 2, (24, K), generator=torch.Generator().manual_seed(5)) * 2 - 1
        w[M - 24:M] = (sign * 1e30).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=0, elem=elem)
    assert _lib.nwc_token_split(c.n, K, c.code, 3) >= 1
    g = torch.Generator().manual_seed(8)
    x = torch.randn(K, generator=g).to(torch.bfloat16).cuda()
    bias = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16).cuda()
    xin = c._padded(x).contiguous()
    ys = []
    for ri in (c.row_index(), None):
        y = torch.empty(M, dtype=torch.bfloat16, device="cuda")
        assert _lib.nwc_linear_xbf16(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                                     _ptr(ri) if ri is not None else None, _ptr(c.seq_table()), _ptr(xin), _ptr(bias),
                                     _ptr(c.scale), _ptr(y), c.n, K, c.code) == 0
        ys.append(y.cpu())
    assert torch.equal(ys[0].view(torch.int16), ys[1].view(torch.int16))
    # dequantization through the same plan (nwc_dequant_seq) against the whole-block kernel without the row index
    # (nwc_dequant) and, for BF16, against the encoded bits
    plain = torch.empty(M, c.K16, dtype=torch.bfloat16, device="cuda")
    assert _lib.nwc_dequant(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low), _ptr(plain),
                            c.n, c.block, K, c.code) == 0
    got = c.dequant()
    assert torch.equal(got.cpu().view(torch.int16), plain[:, :K].cpu().view(torch.int16))
    if elem == "bf16":
        assert torch.equal(got.cpu().view(torch.int16), w.view(torch.int16))
    wd = got.double()
    if c.scale is not None:
        wd = wd * c.scale.double()[:, None]
    y64 = (wd @ x.double() + bias.double()).cpu().numpy()
    terms = (wd.abs() @ x.double().abs()).cpu().numpy()
    check_rne(ys[0], y64, token_tol(y64, terms))


@pytest.mark.parametrize("M,K,escapes", [(4608, 3584, "none"), (3584, 3584, "dense"), (1003, 1100, "dense"),
                                          (16, 512, "none"), (2000, 3000, "dense"), (37888, 3584, "dense"),
                                          (3584, 18944, "none"), (1000, 17000, "dense")])
def test_layout2_split_token_path(cuda, M, K, escapes):
    """Layout 2's token path on matrices with few 16-row groups per CU, where a block's 16 super-chunks go to four or
    two half-waves (qkv / o of Qwen2.5-7B, ragged shapes), and on gate_up / down of Qwen2.5-7B (tiles with more
    blocks than half-waves; 37 column blocks), against float64 on the decoded weights and against the
    fp32 path's whole-block kernel; "dense" places runs of exceptions (ranks past the table) in several super-chunks of
    one lane, so each part must add exactly the exceptions of its own range."""
    NWCWeight, _, _ = _nwc()
    w = bf16_matrix(M, K, seed=11, escapes=False)
    if escapes == "dense":
        big = torch.tensor(1e30, dtype=torch.bfloat16)
        w[0, 0:512:3] = big                                   # one lane-row, many super-chunks
        w[9, 600:700] = -big
        w[M - 1, K - 40:K] = big
    c = NWCWeight(w, device="cuda", layout=2)
    x = torch.randn(K, generator=torch.Generator().manual_seed(12)).to(torch.bfloat16)
    y = c.linear_bf16(x.cuda(), None).double().cpu().numpy()
    y64 = (w.double() @ x.double()).numpy()
    check_rne(y, y64, token_tol(y64))
    y32 = c.matvec(x.float().cuda()).double().cpu().numpy()       # fp32 path: the whole-block kernel
    check_rne(y, y32, token_tol(y32) + 1e-3 * np.abs(y64) + 1e-5)   # both paths' summation errors
    assert np.all(np.abs(y32 - y64) <= 1e-3 * np.abs(y64) + 1e-5)


@pytest.mark.parametrize("layout,M,K,escapes", [
    (0, 64, 20000, "none"), (0, 4160, 16400, "none"), (0, 1003, 1100, "heavy"), (0, 19456, 2560, "none"),
    (0, 2560, 9728, "heavy"), (1, 64, 20000, "none"), (1, 1003, 1100, "heavy"), (2, 1003, 1100, "none")])
def test_dequant_with_and_without_table(cuda, layout, M, K, escapes):
    """nwc_dequant and nwc_dequant_seq (13-bit decode table for layouts 0/1, row index for layout 0) both return the
    original BF16 bits: matrices wider than one round of blocks (K = 20000: 40 column blocks, the two-buffer kernel
    with one row group per workgroup; 4160 x 16400: 33 column blocks, two row groups per workgroup), gate_up and down
    of Qwen3-4B, and escape rows whose streams exceed their LDS region.  The token path on the wide matrices (the
    two-buffer kernel) against float64."""
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    NWCWeight, _, _ = _nwc()
    print(f"dequant layout {layout} {M}x{K} {escapes}", flush=True)
    w = bf16_matrix(M, K, seed=M + K, escapes=False)
    if escapes == "heavy":
        sign = torch.randint(0, 2, (24, K), generator=torch.Generator().manual_seed(5)) * 2 - 1
        w[0:24] = (sign * 1e30).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=layout)
    st = c.seq_table() if layout <= 1 else None
    outs = []
    for seq in (False, True):
        out = torch.full((M, c.K16), -1, dtype=torch.int16, device="cuda")
        if seq:
            ri = c.row_index() if layout <= 1 else None
            err = _lib.nwc_dequant_seq(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                                       _ptr(ri) if ri is not None else None, _ptr(st) if st is not None else None,
                                       _ptr(out), c.n, K, c.code)
        else:
            err = _lib.nwc_dequant(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                                   _ptr(out), c.n, c.block, K, c.code)
        assert err == 0
        outs.append(out[:, :K].cpu())
    for o in outs:
        assert torch.equal(o, w.view(torch.int16))
    if K > 16384:
        x = torch.randn(K, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16)
        y = c.linear_bf16(x.cuda(), None).double().cpu().numpy()
        y64 = (w.double() @ x.double()).numpy()
        check_rne(y, y64, token_tol(y64))


REF_TEST_K_SHAPES = [(8192, 4608), (4096, 11008), (1024, 3600), (2048, 2064), (512, 16384), (19456, 2560), (1024, 9728),
                     (1001, 1000), (13, 40), (8, 16), (3, 4097)]


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("M,K", REF_TEST_K_SHAPES)
def test_reference_test_k_shapes(cuda, layout, M, K):
    """The reference's tests/test_k.py shapes (:10-11: K not a multiple of 512 or 16, M not a multiple of 8), with
    seeded N(0, 0.02^2) weights instead of its data/W.raw (absent here) and its activations (rand - 0.5) and bias:
    dequant bit-exact; token path rounded to nearest even from within 1e-3 of float64 (the reference accepts 2e-2
    against F.linear); fp32
    path within 1e-3 relative (the reference: 1e-4 relative to |ref| + 1e-2)."""
    NWCWeight, _, _ = _nwc()
    print(f"test_k shape layout {layout} {M}x{K}", flush=True)
    w = bf16_matrix(M, K, seed=M + 3 * K)
    c = NWCWeight(w, device="cuda", layout=layout)
    assert torch.equal(c.dequant().cpu().view(torch.int16), w.view(torch.int16))
    g = torch.Generator().manual_seed(1)
    xb = (torch.rand(K, generator=g) - 0.5).to(torch.bfloat16)
    bias = (torch.rand(M, generator=g) - 0.5).to(torch.bfloat16)
    y = c.linear_bf16(xb.cuda(), bias.cuda())
    wd = w.cuda().double()
    y64 = (wd @ xb.cuda().double() + bias.cuda().double()).cpu().numpy()
    _check_bf16(y, y64, 0.02)
    y32 = c.matvec(xb.float().cuda()).double().cpu().numpy()
    _check_f32(y32, (wd @ xb.cuda().double()).cpu().numpy(), 0.02)


@pytest.mark.parametrize("layout", LAYOUTS)
@pytest.mark.parametrize("M,K", [(4096, 2560), (8192, 4608), (151936 // 8, 2560), (2048, 2064), (1001, 1000), (13, 40)])
def test_reference_gather_shapes(cuda, layout, M, K):
    """The reference's tests/test_gather.py shapes (:12) and ids (64, including 0, M - 1 and M / 2, :18): rows
    bit-exact; ids outside [0, M) leave their output rows untouched."""
    NWCWeight, _, _ = _nwc()
    print(f"gather shape layout {layout} {M}x{K}", flush=True)
    w = bf16_matrix(M, K, seed=5 * M + K)
    c = NWCWeight(w, device="cuda", layout=layout)
    g = torch.Generator().manual_seed(2)
    ids = torch.cat([torch.tensor([0, M - 1, M // 2]), torch.randint(0, M, (61,), generator=g)])
    assert torch.equal(c.gather(ids.cuda()).cpu().view(torch.int16), w[ids].view(torch.int16))
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    bad = torch.tensor([-1, M, 0, M + 7], dtype=torch.int64, device="cuda")
    out = torch.full((4, c.K16), 0x1234, dtype=torch.int16, device="cuda")
    assert _lib.nwc_gather(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low), _ptr(bad), 4,
                           _ptr(out), c.n, c.block, K, c.code) == 0
    out = out.cpu()
    assert torch.all(out[[0, 1, 3]] == 0x1234)
    assert torch.equal(out[2, :K], w[0].view(torch.int16))


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("M,K,elem", [(1000, 2600, "bf16"), (300, 1000, "fp8"), (19, 40, "bf16"), (4096, 3584, "bf16")])
def test_gather_xindex_matches_reference_entry_point(cuda, M, K, elem, layout):
    """The row-index gather (layout 0: from the row pair that holds each row; layout 1: four half-waves per block, one
    per quarter of the super-chunks) against the reference's entry point nwc_gather on the same ids, with the 13-bit
    table and with the stored LUT: every row of a row group (ids 0..15 and random ones), ragged K (a last column block
    of 40 or 16 columns), fp8, escapes; ids outside [0, M) leave their output rows untouched."""
    NWCWeight, _, _ = _nwc()
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    print(f"gather xindex layout {layout} {M}x{K} {elem}", flush=True)
    w = fp8_source(M, K, seed=M + K) if elem == "fp8" else bf16_matrix(M, K, seed=M + K, escapes=True)
    c = NWCWeight(w, device="cuda", elem=elem, layout=layout)
    if c.row_index() is None:
        pytest.skip("no row index for this layout-1 shape")
    g = torch.Generator().manual_seed(K)
    ids = torch.cat([torch.arange(min(16, M)), torch.randint(0, M, (64,), generator=g), torch.tensor([-1, M, M + 9])])
    ids = ids.cuda()
    n = ids.numel()
    ref = torch.full((n, c.K16), 0x1234, dtype=torch.int16, device="cuda")
    assert _lib.nwc_gather(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low), _ptr(ids), n,
                           _ptr(ref), c.n, c.block, K, c.code) == 0
    for table in (c.seq_table(), None):
        out = torch.full((n, c.K16), 0x1234, dtype=torch.int16, device="cuda")
        assert _lib.nwc_gather_xindex(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low),
                                      _ptr(c.row_index()), _ptr(table), _ptr(ids), n, _ptr(out), c.n, K, c.code) == 0
        assert torch.equal(out.cpu(), ref.cpu())
    torch.cuda.synchronize()
    assert torch.all(ref[-3:].cpu() == 0x1234)
    d = c.dequant().cpu().view(torch.int16)
    assert torch.equal(ref[:-3, :K].cpu(), d[ids[:-3].cpu(), :K])


@pytest.mark.parametrize("elem", ["bf16", "fp8"])
def test_layout2_gather_exception_rows(cuda, elem):
    """Layout 2's gather (four half-waves per block, each patching only the exceptions of its own super-chunks) on rows
    dense in exceptions: a whole row, every third column of another, a run across a super-chunk boundary and the ragged
    last column block; rows bit-exact against the original weights."""
    NWCWeight, _, quantize_fp8 = _nwc()
    M, K = 48, 1000
    if elem == "fp8":
        w = fp8_source(M, K, seed=3)
        w[5] *= 40.0                                         # whole rows of outliers (exceptions after quantization)
        w[21, ::3] *= 40.0
        w[40, 500:520] *= 40.0
        ref = quantize_fp8(w)[0].to(torch.bfloat16)
    else:
        w = bf16_matrix(M, K, seed=3, escapes=False)
        sign = torch.tensor([1e30, -1e30], dtype=torch.bfloat16).repeat(K // 2)
        w[5] = sign
        w[21, ::3] = torch.tensor(1e30, dtype=torch.bfloat16)
        w[40, 500:520] = torch.tensor(-1e30, dtype=torch.bfloat16)
        w[40, 990:1000] = torch.tensor(3e29, dtype=torch.bfloat16)
        ref = w
    c = NWCWeight(w, device="cuda", elem=elem, layout=2)
    ids = torch.tensor([5, 21, 40, 0, 47, 13, 29, 5, 40, 21, 8, 16])
    print(f"layout-2 gather exception rows {elem}", flush=True)
    assert torch.equal(c.gather(ids.cuda()).cpu().view(torch.int16), ref[ids].view(torch.int16))


def _random_shapes(n, seed):
    """Seeded log-uniform shapes (M up to 3000, K up to 20000): ragged K16/K32 tails, column-block counts from 1 to 40,
    row counts that leave partial row groups."""
    g = np.random.default_rng(seed)
    return [(int(np.exp(g.uniform(0, np.log(3000)))), int(np.exp(g.uniform(0, np.log(20000)))),
             int(g.integers(0, 3)), ["bf16", "fp8"][int(g.integers(0, 2))]) for _ in range(n)]


def _large_shapes(n, seed):
    """Seeded tall shapes (30000-160000 rows, at most 2e8 weights) whose row groups do not fit one residency round:
    the multi-round tiles of layouts 0 and 1 and layout 2's round-robin ranges."""
    g = np.random.default_rng(seed)
    out = []
    for i in range(n):
        M = int(np.exp(g.uniform(np.log(30000), np.log(160000))))
        K = int(np.exp(g.uniform(np.log(256), np.log(min(6000, 2e8 / M)))))
        out.append((M, K, i % 3, ["bf16", "fp8"][(i // 3) % 2]))
    return out


@pytest.mark.parametrize("M,K,layout,elem", _random_shapes(24, 20261202) + _large_shapes(6, 20261203))
def test_random_shapes_all_paths(cuda, M, K, layout, elem):
    """Seeded random shapes through every path: dequant (bit-exact against the source for BF16; both entry points
    agree), gather, token path (BF16 x) rounded to nearest even from within 1e-3 of float64 on the decoded weights
    (fp8: times the row scale), fp32 path within 1e-3."""
    from nwc_amd._abi import lib as _lib, ptr as _ptr, stream as _stream
    NWCWeight, _, _ = _nwc()
    print(f"random shape {M}x{K} layout {layout} {elem}", flush=True)
    src = fp8_source(M, K, seed=M * 31 + K) if elem == "fp8" else bf16_matrix(M, K, seed=M * 31 + K)
    try:
        c = NWCWeight(src, device="cuda", layout=layout, elem=elem)
    except (RuntimeError, ValueError):
        # a matrix the format cannot code (a lane stream over 255 words, or over 255 layout-2 exceptions): the
        # oracle's restatement of the reference encoder refuses it too
        _, _, quantize_fp8 = _nwc()
        codes = quantize_fp8(src)[0].view(torch.uint8).numpy() if elem == "fp8" else bits16(src)
        assert O.encode(codes, int(elem == "fp8"), layout)["dl"] < 0
        return
    d = c.dequant()
    w = d.float() * c.scale[:, None] if elem == "fp8" else d.float()
    if elem == "bf16":
        assert torch.equal(d.cpu().view(torch.int16), src.view(torch.int16))
    out = torch.empty(M, c.K16, dtype=torch.bfloat16, device="cuda")
    assert _lib.nwc_dequant(_stream(), _ptr(c.data), _ptr(c.bases), _ptr(c.hdr), _ptr(c.lut), _ptr(c.low), _ptr(out),
                            c.n, c.block, K, c.code) == 0
    assert torch.equal(out[:, :K], d)
    ids = torch.randint(0, M, (9,), generator=torch.Generator().manual_seed(K))
    rows = c.gather(ids.cuda())                                 # fp8: the unscaled values, as dequant()
    assert torch.equal(rows.view(torch.int16), d[ids.cuda()].view(torch.int16))
    x = torch.randn(K, generator=torch.Generator().manual_seed(M)).to(torch.bfloat16).cuda()
    y = c.linear_bf16(x, None).double().cpu().numpy()
    y64 = (w.double() @ x.double()).cpu().numpy()
    # fp32 accumulation error is bounded by the sum of |terms|, not by |y|: two 1e30 escapes whose products cancel
    # leave y64 ~ 1 while any fp32 sum returns ~0 (23x1289, x seed 23, row 12)
    cancel = 2.0 ** -20 * (w.double().abs() @ x.double().abs()).cpu().numpy()
    check_rne(y, y64, token_tol(y64) + cancel)
    y32 = c.matvec(x.float()).double().cpu().numpy()
    assert np.all(np.abs(y32 - y64) <= 1e-3 * np.abs(y64) + 1e-5 + cancel)


@pytest.mark.parametrize("layout", LAYOUTS)
def test_special_values_round_trip(cuda, layout):
    """BF16 specials survive bit for bit: +-0, +-inf, NaNs with several payloads, subnormals, the largest finite
    values, scattered through an N(0, 0.02^2) matrix (dequant, gather, and the oracle's decode of the same tensors)."""
    NWCWeight, _, _ = _nwc()
    M, K = 64, 1100
    w = bf16_matrix(M, K, seed=99, escapes=False)
    bits = w.view(torch.int16).view(-1)
    specials = [0x0000, 0x8000, 0x7F80, 0xFF80, 0x7FC0, 0xFFC1, 0x7F81, 0x0001, 0x8001, 0x007F, 0x7F7F, 0xFF7F, 0x3F80]
    g = torch.Generator().manual_seed(3)
    pos = torch.randint(0, M * K, (400,), generator=g)
    for i, p in enumerate(pos.tolist()):
        v = specials[i % len(specials)]
        bits[p] = v - 0x10000 if v >= 0x8000 else v
    if layout == 2:
        try:
            c = NWCWeight(w, device="cuda", layout=layout)
        except ValueError:
            pytest.skip("a lane stream has more than 255 layout-2 exceptions")
    else:
        c = NWCWeight(w, device="cuda", layout=layout)
    assert torch.equal(c.dequant().cpu().view(torch.int16), w.view(torch.int16))
    assert np.array_equal(O.decode(oracle_encoding(c)), bits16(w))
    ids = torch.unique(pos // K)[:16]
    assert torch.equal(c.gather(ids.cuda()).cpu().view(torch.int16), w[ids].view(torch.int16))


def _finish_rows():
    """Rows whose fp32 sums are exact in any order (few nonzero weights, x = 1) and land on or near BF16 ties, with the
    bias each row needs; the expected output is RNE(sum + bias) computed exactly on the host.  u = 2^-7 is the BF16
    spacing in [1, 2)."""
    u = 2.0 ** -7
    return [([1.0, u / 2], 0.0),                   # tie -> even: 1
            ([1.0, 3 * u / 2], 0.0),               # tie -> even: 1 + 2u (a truncating finish gives 1 + u)
            ([-1.0, -u / 2], 0.0),                 # -1
            ([1.0, u / 2, 2.0 ** -20], 0.0),       # just above the tie: 1 + u
            ([1.0, u / 4, u / 16], u / 4),         # 1 + 0.3125u, + 0.25u: 1 + u (rounding before the bias gives 1)
            ([2.0 ** 100, 2.0 ** 92], 0.0),        # tie at 2^100: 2^100
            ([1.0, 1.0, 1.0, u], -0.5),            # 2.5 + u: exact, 2.5078125
            ([0.75, u / 8], 0.0)]                  # 0.75 + u/8, below the tie in [0.5, 1): 0.75


@pytest.mark.parametrize("layout", LAYOUTS)
def test_token_path_rounds_once_after_the_bias(cuda, layout):
    """The finish is the reference's (nwc_ops.cu:553-565): the row's sum over column blocks, plus the bias, rounded
    once to nearest even.  Each row's few weights sit in different column blocks of a 16 x 1536 matrix; every output
    must equal the host's RNE(sum + bias) bit for bit (the batched kernel and fp32 activations too, layout 0)."""
    from tests.helpers import rne_bf16
    NWCWeight, _, _ = _nwc()
    M, K = 16, 1536
    rows = _finish_rows()
    w = torch.zeros(M, K, dtype=torch.float64)
    bias = torch.zeros(M, dtype=torch.float64)
    cols = [3, 700, 1100, 1400]
    for r, (vals, b) in enumerate(rows):
        for v, col in zip(vals, cols):
            w[r, col] = v
        bias[r] = b
    wb, bb = w.to(torch.bfloat16), bias.to(torch.bfloat16)
    assert torch.equal(wb.double(), w) and torch.equal(bb.double(), bias)     # every value exact in BF16
    want = rne_bf16(w.sum(1).numpy() + bias.numpy())
    c = NWCWeight(wb, device="cuda", layout=layout)
    x = torch.ones(K, dtype=torch.bfloat16, device="cuda")
    outs = [c.linear_bf16(x, bb.cuda()), c.linear_bf16(x.float(), bb.cuda())]
    if layout == 0:
        outs.append(c.linear_batch(torch.stack([x, x]), bb.cuda())[1])
    for y in outs:
        assert np.array_equal(y.double().cpu().numpy(), want), (y.double().cpu().numpy()[:8], want[:8])


@pytest.mark.parametrize("layout", LAYOUTS)
def test_token_path_nan_and_inf_rows(cuda, layout):
    """Rows whose sums are not finite: an inf - inf pair and a NaN weight give a quiet NaN, one infinite weight gives
    +-inf (positive activations), in the token path, the batched kernel and the fp32 path; every other row is
    unaffected.  A NaN sum stays NaN (the quiet bit set): the reference's unguarded bias rounding (nwc_ops.cu:562-564)
    gives the same bits for a NaN with a zero low half, which is what BF16 operands produce, and would turn a NaN
    with low payload bits into +-inf or -0."""
    NWCWeight, _, _ = _nwc()
    M, K = 64, 1100
    w = bf16_matrix(M, K, seed=21, escapes=False)
    inf, nan = float("inf"), float("nan")
    w[3, 10], w[3, 700] = inf, -inf
    w[7, 100] = nan
    w[11, 5] = inf
    w[12, 1099] = -inf
    w[40, 513], w[40, 514] = -inf, inf
    x = (torch.rand(K, generator=torch.Generator().manual_seed(2)) + 0.25).to(torch.bfloat16)
    c = NWCWeight(w, device="cuda", layout=layout)
    assert torch.equal(c.dequant().cpu().view(torch.int16), w.view(torch.int16))
    outs = [c.linear_bf16(x.cuda(), None), c.matvec(x.float().cuda())]
    if layout == 0:
        outs.append(c.linear_batch(torch.stack([x, x]).cuda(), None)[0])
    finite = [r for r in range(M) if r not in (3, 7, 11, 12, 40)]
    wf = w[finite].double()
    y64 = (wf @ x.double()).numpy()
    for i, y in enumerate(outs):
        yc = y.cpu()
        for r in (3, 7, 40):
            assert torch.isnan(yc[r]), (i, r, yc[r])
            if yc.dtype == torch.bfloat16:
                assert int(yc[r:r + 1].view(torch.int16)) & 0x7FC0 == 0x7FC0
        assert yc[11].item() == inf and yc[12].item() == -inf
        if yc.dtype == torch.bfloat16:
            check_rne(yc[finite], y64, token_tol(y64))
        else:
            assert np.all(np.abs(yc[finite].double().numpy() - y64) <= 1e-3 * np.abs(y64) + 1e-5)
