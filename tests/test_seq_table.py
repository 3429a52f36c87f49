"""The 13-bit token-path decode table (nwc_seq_table, nwc_amd/csrc/encode.cpp): not part of the format, derived from
the stored LUT.  Pinned two ways, CPU only:
  * against the stored 12-bit LUT (itself byte-identical to the oracle's, tests/test_encoder.py): every 13-bit window
    whose first 12 bits hold two complete codes must give the same two bytes and length, and no window may give a
    pair longer than 13 bits or an entry outside the step encoding;
  * end to end: decoding layout-0 lane streams with the kernel's step rule (two table reads per four codes, else four
    codes by the code definition) must reproduce the high byte (sign + exponent) of every BF16 weight, on N(0, 0.02^2)
    weights with escapes and on an exponent-spread matrix where escapes and long codes are common."""
import numpy as np
import pytest
import torch

from tests.helpers import bf16_matrix, fp8_source

SLOW = 0x40000000
FLAG = 1 << 30
BYTE0 = 16              # a fast entry's byte 0 is BYTE0 - c (c = bits of its two codes): the kernel's step encoding


def _nwc():
    from nwc_amd.nwc_torch import NWCWeight, SEQ_TABLE_WORDS
    from nwc_amd._abi import lib as _lib, ptr as _ptr
    return NWCWeight, _lib, _ptr, SEQ_TABLE_WORDS


def _table(c):
    _, lib, ptr, words = _nwc()
    out = torch.zeros(words, dtype=torch.int32)
    assert lib.nwc_seq_table(ptr(c.lut.contiguous()), c.code, ptr(out)) == 0
    return out.numpy().view(np.uint32)


def _spread(M, K, seed):
    g = torch.Generator().manual_seed(seed)
    mag = torch.exp2(torch.rand(M, K, generator=g) * 80 - 40)
    sign = torch.where(torch.rand(M, K, generator=g) < 0.5, -1.0, 1.0)
    return (mag * sign).to(torch.bfloat16)


@pytest.mark.parametrize("elem", ["bf16", "fp8"])
@pytest.mark.parametrize("kind", ["normal", "spread"])
def test_seq_table_agrees_with_stored_lut(elem, kind):
    NWCWeight, _, _, _ = _nwc()
    if elem == "fp8":
        c = NWCWeight(fp8_source(64, 1024, seed=3), device="cpu", elem="fp8", layout=0)
    else:
        w = bf16_matrix(64, 1024, seed=4) if kind == "normal" else _spread(64, 1024, seed=4)
        c = NWCWeight(w, device="cpu", layout=0)
    lut = c.lut.numpy().view(np.uint32)
    t = _table(c)
    seq = t[:8192]
    fast = seq != SLOW
    assert np.all((seq[fast] >> 24) == 0)
    assert np.all((seq[fast] & 0xFF) >= BYTE0 - 13) and np.all((seq[fast] & 0xFF) <= BYTE0 - 4)   # 4 <= c <= 13
    p = np.arange(8192)
    e12 = lut[p >> 1]
    pair12 = (e12 & FLAG) == 0
    pair12[:4] = False                                   # patterns 0..3 map to entries 0/1 (exp_of_rank carriers)
    assert np.all(fast[pair12])
    assert np.array_equal(seq[pair12] & 0xFFFF00, e12[pair12] & 0xFFFF00)
    assert np.array_equal(BYTE0 - (seq[pair12] & 0xFF), e12[pair12] & 0xFF)
    # the 13-bit table decodes strictly more windows: some pair is 13 bits long
    assert fast.sum() > pair12.sum()
    # exp_of_rank words: byte q is the symbol the stored LUT gives rank q with sign 0
    eor = t[8192:].view(np.uint8)
    for q in range(11):
        e = lut[1 << (11 - q)]
        if not (e & FLAG) or (e >> 24) & 0xFF:           # a complete first code
            assert eor[q] == (e >> 8) & 0x7F


def _decode_lanes(c, seq):
    """Decode every lane stream of a layout-0 matrix with the kernel's step rule; returns the coded bytes per weight
    in the matrix's [M, K16] order."""
    data = c.data.numpy()
    bases = c.bases.numpy().view(np.uint32)
    hdr = c.hdr.numpy()
    eor = seq[8192:].view(np.uint8)
    M, K16 = c.out_features, c.K16
    CB = (K16 + 511) // 512
    groups = (M + 7) // 8
    out = np.zeros((groups * 8, CB * 512), np.int64)
    for b in range(groups * CB):
        g, cb = divmod(b, CB)
        n = hdr[b * 32:(b + 1) * 32].astype(np.int64)
        start = np.concatenate([[0], np.cumsum(n)[:-1]])
        for L in range(32):
            if cb * 512 + 16 * L >= K16:
                continue
            off = int(bases[b]) + 4 * int(start[L])
            words = data[off:off + 4 * int(n[L]) + 16].view("<u4")
            bits = "".join(format(int(x), "032b") for x in words) + "0" * 64
            pos, got = 0, []
            while len(got) < 128:
                e1 = int(seq[int(bits[pos:pos + 13], 2)])
                if e1 != SLOW:
                    c1 = BYTE0 - (e1 & 0xFF)
                    e2 = int(seq[int(bits[pos + c1:pos + c1 + 13], 2)])
                    if e2 != SLOW:
                        got += [(e1 >> 8) & 0xFF, (e1 >> 16) & 0xFF, (e2 >> 8) & 0xFF, (e2 >> 16) & 0xFF]
                        pos += c1 + BYTE0 - (e2 & 0xFF)
                        continue
                for _ in range(4):                       # the slow path: four codes by the code definition
                    z = len(bits[pos:]) - len(bits[pos:].lstrip("0"))
                    if z < 15:
                        got.append(int(bits[pos + z + 1]) << 7 | int(eor[z]))
                        pos += z + 2
                    else:
                        got.append(int(bits[pos + 16:pos + 24], 2))
                        pos += 24
            assert pos <= 32 * int(n[L])
            blk = np.array(got).reshape(8, 16)
            out[g * 8:g * 8 + 8, cb * 512 + 16 * L:cb * 512 + 16 * L + 16] = blk
    return out[:M, :K16]


@pytest.mark.parametrize("kind,M,K", [("normal", 24, 1100), ("spread", 16, 600)])
def test_seq_table_decodes_streams(kind, M, K):
    NWCWeight, _, _, _ = _nwc()
    w = bf16_matrix(M, K, seed=M + K) if kind == "normal" else _spread(M, K, seed=7)
    c = NWCWeight(w, device="cpu", layout=0)
    seq = _table(c)
    hi = _decode_lanes(c, seq)[:, :K]
    want = (w.contiguous().view(torch.int16).numpy().view(np.uint16) >> 8).astype(np.int64)
    assert np.array_equal(hi, want)


def test_weight_seq_table_is_the_host_build():
    NWCWeight, _, _, _ = _nwc()
    c = NWCWeight(bf16_matrix(16, 1024, seed=2), device="cpu", layout=0)
    assert np.array_equal(c.seq_table().numpy().view(np.uint32), _table(c))
    assert NWCWeight(bf16_matrix(16, 1024, seed=2), device="cpu", layout=2).seq_table() is None


def test_seq_table_rejects_layout2():
    NWCWeight, lib, ptr, words = _nwc()
    c = NWCWeight(bf16_matrix(8, 512, seed=1), device="cpu", layout=2)
    out = torch.zeros(words, dtype=torch.int32)
    assert lib.nwc_seq_table(ptr(c.lut.contiguous()), c.code, ptr(out)) == -1
