"""Layouts 0/1 in fixed slots (NWCWeight._to_slots, done when a matrix is placed on a GPU): every block's lane streams
start at byte b * stride, so the token kernels compute a block's offset instead of reading bases[b] before they can
request the streams.  The slot tensors must remain a valid tensor set of the format (the oracle's restatement of the
reference decoder reads them as it reads the packed ones), tensors() must give back the packed bytes exactly, and
matrices the slots do not suit stay packed.  The library's check of the stride bits of `elem` is covered here too.
CPU only (the move is plain tensor work; the kernels' use of it is compared with the packed form on the GPU)."""
import ctypes

import numpy as np
import pytest
import torch

from tests.helpers import bf16_matrix


def _weight(M, K, elem="bf16", seed=5, w=None, layout=0):
    pytest.importorskip("nwc_amd.nwc_torch", reason="the HIP library is not built")
    from nwc_amd.nwc_torch import NWCWeight, quantize_fp8
    w = bf16_matrix(M, K, seed=seed) if w is None else w
    if elem == "fp8":
        q, s = quantize_fp8(w.float())
        return NWCWeight(q, device="cpu", elem="fp8", scale=s, layout=layout)
    return NWCWeight(w, device="cpu", layout=layout)


def _oracle_decode(c, data, bases):
    from oracle import oracle as O
    enc = {"data": data.numpy(), "bases": bases.numpy().view(np.uint32), "hdr": c.hdr.numpy(),
           "lut": c.lut.numpy().view(np.uint32), "low": c.low.numpy(), "M": c.out_features, "K": c.in_features,
           "elem": c.elem, "layout": c.layout}
    return O.decode(enc)


@pytest.mark.parametrize("M,K,elem,layout", [(64, 512, "bf16", 0), (48, 2560, "bf16", 0), (24, 2560, "fp8", 0),
                                             (16, 33, "bf16", 0), (64, 2560, "bf16", 1), (32, 4096, "fp8", 1),
                                             (32, 33, "bf16", 1)])
def test_slots_round_trip(M, K, elem, layout):
    from nwc_amd.nwc_torch import LANES, SLOT_TAIL
    c = _weight(M, K, elem, layout=layout)
    packed = {k: v.clone() for k, v in c.tensors().items()}
    code, size_bytes = c.code, c.bytes
    c._to_slots()
    nb = packed["bases"].numel()
    start = packed["bases"].to(torch.int64)
    size = c.hdr.view(-1, LANES).to(torch.int64).sum(1) * 4
    stride = c._slot
    assert stride % 16 == 0 and int(size.max()) <= stride < int(size.max()) + 16
    assert c.data.numel() == nb * stride + SLOT_TAIL
    assert torch.equal(c.bases.to(torch.int64), torch.arange(nb, dtype=torch.int64) * stride)
    used = torch.zeros(c.data.numel(), dtype=torch.bool)
    for b in range(nb):
        n = int(size[b])
        assert torch.equal(c.data[b * stride:b * stride + n], packed["data"][int(start[b]):int(start[b]) + n])
        used[b * stride:b * stride + n] = True
    assert not c.data[~used].any()                                  # padding and tail are zero
    assert c.code == code | (stride // 16) << 8 and c.bytes == size_bytes
    back = c.tensors()                                              # the checkpoint form: the packed bytes exactly
    for name, t in packed.items():
        assert torch.equal(back[name], t), name
    # the slot tensors are a valid tensor set of the format: the oracle decodes them to the same weights
    assert np.array_equal(_oracle_decode(c, c.data, c.bases), _oracle_decode(c, packed["data"], packed["bases"]))


def test_ragged_blocks_keep_packed():
    """K = 530 leaves a last column block of 18 columns: slots sized for the full blocks would hold far more bytes
    than the packed streams (past the 15% allowed), so the matrix stays packed."""
    from nwc_amd.nwc_torch import LANES, SLOT_OVERHEAD
    c = _weight(40, 530)
    size = c.hdr.view(-1, LANES).to(torch.int64).sum(1) * 4
    assert size.numel() * (-(-int(size.max()) // 16) * 16) > SLOT_OVERHEAD * c.data.numel()
    before = c.data.clone()
    c._to_slots()
    assert c._slot == 0 and torch.equal(c.data, before)


def test_nonzero_gap_byte_keeps_packed():
    """A byte outside every block's streams that is not zero (a foreign writer's padding) could not be restored by
    tensors(): such a matrix stays packed."""
    from nwc_amd.nwc_torch import LANES
    c = _weight(48, 2560)
    start = c.bases.to(torch.int64)
    end = start + c.hdr.view(-1, LANES).to(torch.int64).sum(1) * 4
    gap = int(end[-1])                                              # the slack after the last block
    data = c.data.clone()
    data[gap] = 7
    c.data = data
    c._to_slots()
    assert c._slot == 0 and torch.equal(c.data, data) and c.code == 0


def test_wide_blocks_keep_packed():
    """Near-uniform exponents code long: blocks past the largest stride stay packed."""
    from nwc_amd.nwc_torch import LANES, SLOT_MAX
    g = torch.Generator().manual_seed(3)
    bits = torch.randint(-32768, 32767, (16, 1024), generator=g, dtype=torch.int32).to(torch.int16)
    bits[(bits & 0x7F80) == 0x7F80] = 0                             # no inf / NaN
    c = _weight(16, 1024, w=bits.view(torch.bfloat16))
    assert int(c.hdr.view(-1, LANES).to(torch.int64).sum(1).max()) * 4 > SLOT_MAX[0]
    before = c.data.clone()
    c._to_slots()
    assert c._slot == 0 and torch.equal(c.data, before)


def _lib():
    from nwc_amd.nwc_torch import _LIB_PATH
    lib = ctypes.CDLL(_LIB_PATH)
    lib.nwc_token_split.restype = ctypes.c_int
    lib.nwc_token_split.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
    lib.nwc_linear_xbf16.restype = ctypes.c_int
    P, U64, U32, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
    lib.nwc_linear_xbf16.argtypes = [P] * 12 + [U64, U32, I]
    return lib


@pytest.mark.parametrize("M,K,elem,ok", [
    (2560, 4096, 0x00 | 94 << 8, True),          # layout 0, stride 1504
    (2560, 4096, 0x01 | 108 << 8, True),         # fp8, stride 1728 (the largest)
    (2560, 4096, 0x00 | 109 << 8, False),        # stride 1744: past layout 0's largest
    (2560, 4096, 0x10 | 186 << 8, True),         # layout 1, stride 2976
    (2560, 4096, 0x11 | 190 << 8, True),         # layout 1 fp8, stride 3040 (the largest)
    (2560, 4096, 0x10 | 191 << 8, False),        # stride 3056: past layout 1's largest
    (2560, 4096, 0x20 | 94 << 8, False),         # layout 2 has no slots
    (2560, 4096, 0x00 | 1 << 16, False),         # unknown bits
    ((1 << 27) - 8, 16, 0x00 | 17 << 8, False),  # 2^24 - 1 blocks of 272-byte slots pass 2^32 bytes
    ((1 << 27) - 8, 16, 0x00 | 15 << 8, True),
])
def test_stride_bits_checked(M, K, elem, ok):
    """Bits 8-15 of elem (stride / 16) are accepted for layout 0 up to the largest stride whose slots stay within
    32-bit offsets, and refused otherwise, before any device call (nwc_token_split plans without launching)."""
    lib = _lib()
    got = lib.nwc_token_split(M * K, K, elem, 0)
    assert (got != -1) == ok
    if not ok:
        assert lib.nwc_linear_xbf16(None, *([None] * 11), M * K, K, elem) == -1
