"""Pins the C oracle (oracle/nwc_oracle.c) to values derived by hand from the format definition
(docs/format.md sections 2-4d, nwc_ops.cu:87-348) and to closed forms, so that a dropped term, a wrong shift or a
transposed index in the oracle fails here.  The reference's own tests hold no stored vectors (all seeded at run time,
tests/test_format_cpu.py), so these known answers, the exhaustive fp8 tables and the round trips are the pins.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.helpers import bf16_matrix, bits16, fp8_source

FLAG = 1 << 30


def enc_const(M, K, value_bits, layout, elem=0):
    w = np.full((M, K), value_bits, dtype=np.uint16 if elem == 0 else np.uint8)
    return O.encode(w, elem, layout)


# ---------------------------------------------------------------------------------------------------------------
# known answers from the code definition: a constant matrix
def test_constant_block_layout0():
    """8x512 of 0.02 (BF16 0x3CA4: symbol 0x3C, raw 0xA4, sign 0): every weight is the rank-0 code '1' + sign '0', so
    every lane stream is 128 x '10' = 256 bits = 8 words of 0xAAAAAAAA."""
    e = enc_const(8, 512, 0x3CA4, 0)
    assert e["dl"] == 32 * 8 * 4 + 64
    assert list(e["bases"]) == [0]
    assert list(e["hdr"]) == [8] * 32
    assert np.all(e["data"][:1024].view("<u4") == 0xAAAAAAAA)
    assert np.all(e["low"][:8 * 512] == 0xA4) and np.all(e["low"][8 * 512:] == 0)
    # exchange sort with one used symbol: ord[0] <-> ord[0x3C] swapped, all other ranks keep their index
    assert list(e["psym"][:16]) == [0x3C] + list(range(1, 16))
    neg = enc_const(8, 512, 0xBCA4, 0)
    assert np.all(neg["data"][:1024].view("<u4") == 0xFFFFFFFF)          # '1' + sign '1'


def test_constant_block_layout1_and_2():
    e1 = enc_const(16, 512, 0x3CA4, 1)
    assert list(e1["hdr"]) == [16] * 32                                  # 256 codes x 2 bits per lane
    assert np.all(e1["data"][:32 * 64].view("<u4") == 0xAAAAAAAA)
    e2 = enc_const(16, 512, 0x3CA4, 2)
    assert e2["dl"] == 64 and list(e2["hdr"]) == [0] * 32                # no exceptions
    nib = 16 * 32 * 8
    assert np.all(e2["low"][:nib] == 0)                                  # [sign 0 | rank 0]
    assert np.all(e2["low"][nib:nib + 16 * 32 * 16] == 0xA4)
    # rank tables: rank 0 = 0x3C, ranks 1..6 the unused symbols 1..6 in index order, rank 7 = 0
    assert e2["lut"][0] == 0x3C | 1 << 8 | 2 << 16 | 3 << 24
    assert e2["lut"][1] == 4 | 5 << 8 | 6 << 16
    assert e2["lut"][2] == 0 and e2["lut"][3] == 0


# ---------------------------------------------------------------------------------------------------------------
# the decode table, entry by entry
def _lut(psym, elem=0):
    p = np.zeros(1024, np.uint16)
    p[:len(psym)] = psym
    lut = np.zeros(4096, np.uint32)
    O.lib().or_build_tab(O._p(p), elem, O._p(lut))
    return lut


PS = [10 + r for r in range(16)]            # distinct, recognisable table bytes


@pytest.mark.parametrize("pat,expect", [
    (0b101000000000, 4 | PS[0] << 8 | PS[0] << 16),                         # '10' '10': two rank-0 codes, c = 4
    (0b011100000000, 5 | (0x80 | PS[1]) << 8 | PS[0] << 16),                # '011' rank 1 sign 1, '10'
    (0b001011000000, 6 | PS[2] << 8 | (0x80 | PS[0]) << 16),                # '0010' rank 2, '11' rank 0 sign 1
    (0b110000000000, FLAG | 2 | (0x80 | PS[0]) << 8 | 1 << 24),             # one code, then 10 zeros (incomplete)
    (0b000000000010, FLAG | 12 | PS[10] << 8 | 1 << 24),                    # rank 10 fills the window exactly
    (0b000000000001, FLAG | PS[11] << 8 | PS[12] << 16),                    # entry 1: ranks 13/14 -> see below
])
def test_lut_entries_bf16(pat, expect):
    lut = _lut(PS)
    if pat == 1:
        assert lut[1] == FLAG | PS[13] << 8 | PS[14] << 16
        assert lut[0] == FLAG | PS[11] << 8 | PS[12] << 16
    else:
        assert lut[pat] == expect


def test_lut_rank_readback():
    """exp_of_rank for ranks 0..10 sits in byte 1 of entry 1 << (11 - r) (pattern: r zeros, one, sign 0)."""
    lut = _lut(PS)
    for r in range(11):
        assert (lut[1 << (11 - r)] >> 8) & 0x7F == PS[r]
        assert lut[1 << (11 - r)] & 0xFF == (r + 2 if r < 5 else lut[1 << (11 - r)] & 0xFF)


def test_lut_fp8_has_ten_ranks():
    lut = _lut(PS, elem=1)
    assert lut[0b000000000010] == FLAG                                      # rank 10 does not exist for fp8
    assert lut[0b000000000100] == FLAG | 11 | PS[9] << 8 | 1 << 24          # rank 9: 9 zeros, one, sign
    assert lut[0] == FLAG | PS[11] << 8 | PS[12] << 16


# ---------------------------------------------------------------------------------------------------------------
def test_escape_code_bits():
    """17 symbols with distinct counts: ranks follow the counts; ranks 15 and 16 are escapes = 15 zeros, a one and
    the whole byte (24 bits).  The first weight of lane 0 is the rarest symbol, so lane 0 starts 0x000138 (byte 0x38)."""
    syms = np.arange(40, 57)
    counts = np.arange(300, 283, -1)                                        # 40 most frequent ... 56 rarest
    flat = np.concatenate([np.full(c, s) for s, c in zip(syms, counts)])
    rng = np.random.default_rng(0)
    rng.shuffle(flat)
    M, K = 8, 4096 // 8 * 2
    w = np.zeros(M * K, np.uint16)
    w[:flat.size] = flat
    # put the rare symbol first in lane 0 (row 0, column 0) by swapping
    j = int(np.nonzero(w == 56)[0][0])
    w[0], w[j] = w[j], w[0]
    # fill the rest with the most frequent symbol, keeping the counts ordered
    rest = w == 0
    w[rest] = 40
    w = (w << 8) | 0x11
    e = O.encode(w.reshape(M, K), 0, 0)
    assert list(e["psym"][:16]) == list(range(40, 56))
    first = int(e["data"][:4].view("<u4")[0])
    assert first >> 8 == 0x000138
    assert np.array_equal(O.decode(e), w.reshape(M, K))


# ---------------------------------------------------------------------------------------------------------------
# fp8 splits against the e4m3fn definition (exhaustive)
def e4m3_value(b):
    s, e, m = b >> 7, (b >> 3) & 15, b & 7
    v = m / 512.0 if e == 0 else 2.0 ** (e - 7) * (1 + m / 8)
    return -v if s else v


def f32_of_bits(u):
    return float(np.array([u], np.uint32).view(np.float32)[0])


BYTE3 = [60, 61, 62, 63, 64, 65, 66, 67, 59, 0]          # docs/format.md 4b: table byte of symbols 0..9


def test_fp8_split_exhaustive():
    for b in range(256):
        sym, nib = ctypes_u8(), ctypes_u8()
        rc = O.lib().or_fp8_split(b, sym.ref, nib.ref)
        if (b & 0x7F) == 0x7F:
            assert rc == -1
            continue
        assert rc == 0 and sym.v < 10 and nib.v < 16
        # decoded fp32 = [s | byte3][nibble << 4][0][0] must be the exact value
        u = (b >> 7) << 31 | BYTE3[sym.v] << 24 | nib.v << 20
        assert f32_of_bits(u) == e4m3_value(b)


def test_fp8_split2_exhaustive():
    for b in range(256):
        sym, m3 = ctypes_u8(), ctypes_u8()
        rc = O.lib().or_fp8_split2(b, sym.ref, m3.ref)
        if (b & 0x7F) == 0x7F:
            assert rc == -1
            continue
        assert rc == 0 and sym.v < 20 and m3.v < 8
        hb, lb = O.lib().or_fp8_hb2(sym.v), O.lib().or_fp8_lb2(sym.v)
        u = ((b >> 7) << 15 | hb << 8 | lb | m3.v << 4) << 16
        assert f32_of_bits(u) == e4m3_value(b)
    # the symbol numbering fixes the exchange sort's tie order: normals are their exponent, then the subnormal groups
    assert [O.lib().or_fp8_hb2(s) for s in range(20)] == [0, 60, 61, 61, 62, 62, 63, 63, 64, 64, 65, 65, 66, 66, 67, 67, 60, 59, 59, 0]


class ctypes_u8:
    def __init__(self):
        import ctypes
        self._c = ctypes.c_uint8(0)
        self.ref = ctypes.byref(self._c)

    @property
    def v(self):
        return self._c.value


def test_e4m3_quantizer_matches_definition():
    for b in range(256):
        if (b & 0x7F) == 0x7F:
            continue
        assert O.lib().or_f32_to_e4m3(e4m3_value(b)) == b or (e4m3_value(b) == 0 and (b & 0x7F) == 0)
    # ties between neighbours go to the even code: 1 + 1/16 lies between 1.0 (0x38) and 1.125 (0x39)
    assert O.lib().or_f32_to_e4m3(1.0625) == 0x38
    assert O.lib().or_f32_to_e4m3(1.1875) == 0x3A                            # between 0x39 and 0x3A -> even 0x3A
    assert O.lib().or_f32_to_e4m3(448.0) == 0x7E and O.lib().or_f32_to_e4m3(-448.0) == 0xFE
    assert O.lib().or_f32_to_e4m3(2.0 ** -10) == 0x00                        # half of the smallest subnormal, tie -> 0
    assert O.lib().or_f32_to_e4m3(3 * 2.0 ** -10) == 0x02                    # 1.5 x 2^-9 ties to the even code 2


# ---------------------------------------------------------------------------------------------------------------
def test_fragment_order_matches_format_text():
    """docs/format.md 4c: lane (r, q) holds columns 8q..8q+7 of rows r and r+8; h = j >> 3 picks columns +0..3 or
    +4..7; inside an mma the a-registers are (row r, +0,+1), (row r+8, +0,+1), (row r, +2,+3), (row r+8, +2,+3)."""
    seen = set()
    for L in range(32):
        r, q = L >> 2, L & 3
        for j in range(16):
            h, a, e = j >> 3, (j >> 1) & 3, j & 1
            row = r + (8 if a in (1, 3) else 0)
            col = 8 * q + 4 * h + (2 if a in (2, 3) else 0) + e
            assert O.lib().or_frag_row(L, j) == row and O.lib().or_frag_col(L, j) == col
            seen.add((row, col))
    assert len(seen) == 16 * 32


@pytest.mark.parametrize("M,K,elem,layout,expect", [
    (19456, 2560, 0, 0, [12160, 19456 * 2560, 19456 * 5, 2560]),
    (2560, 4096, 0, 0, [2560, 2560 * 4096, 2560 * 8, 4096]),
    (6144, 2560, 0, 1, [1920, 6144 * 2560, 6144 * 5, 2560]),
    (3, 4097, 0, 0, [9, 3 * 4112, 8 * 9, 4112]),
    (3, 4097, 0, 1, [9, 129 * 32 * 16, 16 * 9, 4112]),
    (3, 4097, 1, 1, [9, 129 * 32 * 8, 16 * 9, 4112]),
    (3, 4097, 0, 2, [9, 129 * 32 * 8 + 129 * 32 * 16, 16 * 9, 4112]),
    (3, 4097, 1, 2, [9, 129 * 32 * 8 + 65 * 3 * 32 * 4, 16 * 9, 4112]),
    (3, 4097, 1, 0, [9, 3 * 2056, 8 * 9, 4112]),
])
def test_layout_arithmetic(M, K, elem, layout, expect):
    assert O.layout_info(M, K, elem, layout) == expect


def test_layout_rejects():
    out = np.zeros(4, np.uint64)
    for M, K in [(0, 5), (5, 0), (1 << 32, 5)]:
        assert O.lib().or_layout(M, K, 0, O._p(out)) == -1


# ---------------------------------------------------------------------------------------------------------------
# error codes of the encoder (nwc_ops.cu:185, :219-220, :248, :311)
def test_encoder_error_codes():
    w = bits16(bf16_matrix(8, 512))
    assert O.encode(w, 0, 0, cap=100)["dl"] == -1                             # capacity
    nan = np.full((8, 512), 0x7F, np.uint8)
    assert O.encode(nan, 1, 0)["dl"] == -2
    assert O.encode(nan, 1, 2)["dl"] == -2
    # layout 2: lane 0 of a 16x512 block made of 10 rare symbols -> 256 exceptions in one lane
    M, K = 16, 512
    w = np.zeros((M, K), np.uint16)
    for L in range(32):
        for j in range(256):
            sc, jj = j >> 4, j & 15
            row = (L >> 2) + 8 * ((jj >> 1) & 1)
            col = sc * 32 + 8 * (L & 3) + 4 * ((jj >> 3) & 1) + 2 * ((jj >> 2) & 1) + (jj & 1)
            sym = 47 + (j % 10) if L == 0 else 40 + (j % 7)
            w[row, col] = sym << 8
    assert O.encode(w, 0, 2)["dl"] == -3
    assert O.encode(w, 0, 0)["dl"] > 0                                        # layouts 0/1 code it fine


# ---------------------------------------------------------------------------------------------------------------
SHAPES = [(8, 512, 0.02), (13, 40, 0.02), (3, 4097, 0.02), (100, 1000, 1.0), (64, 2048, 0.02), (17, 520, 0.02), (1, 1, 0.02)]


@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,K,sigma", SHAPES)
def test_roundtrip_bf16(layout, M, K, sigma):
    w = bits16(bf16_matrix(M, K, seed=M + K, scale=sigma))
    assert np.array_equal(O.decode(O.encode(w, 0, layout)), w)


@pytest.mark.parametrize("layout", [0, 1, 2])
@pytest.mark.parametrize("M,K", [(8, 512), (13, 40), (3, 4097), (101, 1000)])
def test_roundtrip_fp8(layout, M, K):
    from nwc_amd.nwc_torch import quantize_fp8
    q, _ = quantize_fp8(fp8_source(M, K, seed=M))
    qb = q.view(torch.uint8).numpy()
    expect = bits16(q.to(torch.bfloat16))
    assert np.array_equal(O.decode(O.encode(qb, 1, layout)), expect)


def test_decoder_rejects_malformed():
    e = O.encode(bits16(bf16_matrix(8, 512)), 0, 0)
    bad = dict(e)
    bad["hdr"] = e["hdr"].copy()
    bad["hdr"][0] = 1                                                         # lane 0 stream cut short
    with pytest.raises(ValueError):
        O.decode(bad)


def test_matvec_closed_form():
    """The oracle's fp32 matvec against float64 on the same BF16 weights (1e-3 rel / 1e-5 abs, the north star's bar),
    and the end-to-end or_linear equal to decode + matvec."""
    w = bits16(bf16_matrix(96, 3000, seed=5, escapes=False))
    x = np.random.default_rng(1).standard_normal(3000).astype(np.float32)
    y = O.matvec_f32(w, x)
    y64 = O.bf16_to_f64(w) @ x.astype(np.float64)
    assert np.all(np.abs(y - y64) <= 1e-3 * np.abs(y64) + 1e-5)
    for layout in (0, 1, 2):
        assert np.array_equal(O.linear(O.encode(w, 0, layout), x), y)
