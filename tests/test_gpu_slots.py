"""Layouts 0/1 in fixed slots against the same matrix packed, on the GPU: every entry point (token path with BF16
and fp32 activations, with scale and bias; dequantization with and without the 13-bit table; the batched token
kernel and the fused prefill of layout 0; both gathers; the row-index build) gives the same bits from either
placement, over the plans the Qwen3-4B shapes take (layout 0: k_layout0p with four and eight rows per half-wave, the
split tail k_layout0t, one workgroup per CU, and the two-buffer plan of a wide matrix; layout 1: k_layout1sp with
the 12-bit LUT and the 13-bit table, and the multi-item k_layout1mp).  The packed twin is rebuilt from the slot
weight's checkpoint tensors with the slots switched off, so both decode the same bytes."""
import numpy as np
import pytest
import torch

from tests.helpers import bf16_matrix, oracle_encoding
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [
    (6144, 2560, "bf16", 0),     # qkv: k_layout0p, four rows per half-wave
    (2560, 4096, "bf16", 0),     # o: split tail, two rows per half-wave of a whole row group + quarters
    (19456, 2560, "bf16", 0),    # gate_up: k_layout0p, eight rows per half-wave
    (2560, 9728, "fp8", 0),      # down as fp8 (row scale): split tail, eight rows + quarters
    (64, 20480, "bf16", 0),      # 40 column blocks: the two-buffer plan
    (1000, 2560, "fp8", 0),
    (6144, 2560, "bf16", 1),     # layout 1 qkv
    (19456, 2560, "bf16", 1),    # layout 1 gate_up (12-bit LUT)
    (2560, 9728, "bf16", 1),     # layout 1 down: the multi-item kernel
    (2560, 4096, "fp8", 1),
]


def _twins(M, K, elem, monkeypatch, layout=0):
    import nwc_amd.nwc_torch as N
    # fp8 without the 1e30 stressors: a row holding one quantizes to zeros, and the spread of block sizes that such
    # row groups add can keep a matrix packed (2560x9728 would need a 1744-byte stride, past the largest)
    w = bf16_matrix(M, K, seed=M + K, escapes=elem != "fp8")
    if elem == "fp8":
        q, s = N.quantize_fp8(w.float())
        c = N.NWCWeight(q, device="cuda:0", elem="fp8", scale=s, layout=layout)
    else:
        c = N.NWCWeight(w, device="cuda:0", layout=layout)
    assert c._slot, "expected fixed slots for this matrix"
    t = c.tensors()
    with monkeypatch.context() as m:
        m.setattr(N, "FIXED_SLOTS", False)
        p = N.NWCWeight.from_tensors(M, K, c.block, t["data"], t["bases"], t["hdr"], t["lut"], t["low"],
                                     device="cuda:0", elem=elem, scale=t.get("scale"), layout=layout)
    assert p._slot == 0 and p.code == c.code & 0xFF
    return c, p


def _same(a, b, what):
    assert torch.equal(a.view(torch.int16) if a.dtype == torch.bfloat16 else a,
                       b.view(torch.int16) if b.dtype == torch.bfloat16 else b), what


@pytest.mark.parametrize("M,K,elem,layout", SHAPES)
def test_slots_match_packed(cuda, M, K, elem, layout, monkeypatch):
    print(f"slots vs packed {M}x{K} {elem} layout {layout}", flush=True)
    c, p = _twins(M, K, elem, monkeypatch, layout)
    assert torch.equal(c.row_index(), p.row_index())
    g = torch.Generator().manual_seed(7)
    x = torch.randn(K, generator=g).to(torch.bfloat16).to(cuda)
    bias = (torch.randn(M, generator=g) * 0.1).to(torch.bfloat16).to(cuda)
    for b in (None, bias):
        _same(c.linear_bf16(x, b), p.linear_bf16(x, b), "token path, BF16 x")
        _same(c.linear_bf16(x.float(), b), p.linear_bf16(x.float(), b), "token path, fp32 x")
    _same(c.matvec(x.float()), p.matvec(x.float()), "fp32 path")
    d = c.dequant()
    _same(d, p.dequant(), "dequantization")
    ids = torch.randint(0, M, (9,), generator=g).to(cuda)
    _same(c.gather(ids), p.gather(ids), "gather")
    if K <= 16384 and layout == 0:
        xs = torch.randn(3, K, generator=g).to(torch.bfloat16).to(cuda)
        _same(c.linear_batch(xs, bias), p.linear_batch(xs, bias), "batched token path")
        xt = torch.randn(5, K, generator=g).to(torch.bfloat16).to(cuda)
        _same(c.prefill(xt, bias), p.prefill(xt, bias), "fused prefill")
    if M * K <= 4096 * 2560:
        assert np.array_equal(d.cpu().view(torch.int16).numpy().view(np.uint16), O.decode(oracle_encoding(c))), \
            "dequantization != oracle"


def test_dequant_without_table_matches(cuda, monkeypatch):
    """nwc_dequant (the reference's entry point: no row index, no 13-bit table) on slots and packed."""
    import nwc_amd.nwc_torch as N
    c, p = _twins(2560, 4096, "bf16", monkeypatch)
    outs = []
    for w in (c, p):
        out = torch.empty(w.out_features, w.K16, dtype=torch.bfloat16, device=cuda)
        N.call("nwc_dequant", N.stream(), *w._streams(), N.ptr(out), w.n, w.block, w.in_features, w.code)
        outs.append(out)
    _same(outs[0], outs[1], "nwc_dequant")
    _same(outs[0], c.dequant(), "nwc_dequant against nwc_dequant_seq")


@pytest.mark.parametrize("layout,elem", [(0, "bf16"), (1, "bf16"), (0, "fp8")])
def test_checkpoint_tensors_are_the_packed_encoding(cuda, layout, elem):
    """A matrix placed on the GPU in fixed slots gives back, through tensors() (what save_pretrained writes), exactly
    the tensors the same matrix has on the CPU, where it stays packed as the encoder wrote it."""
    import nwc_amd.nwc_torch as N
    w = bf16_matrix(2560, 4096, seed=11, escapes=elem != "fp8")
    if elem == "fp8":
        q, s = N.quantize_fp8(w.float())
        g = N.NWCWeight(q, device="cuda:0", elem="fp8", scale=s, layout=layout)
        h = N.NWCWeight(q, device="cpu", elem="fp8", scale=s, layout=layout)
    else:
        g = N.NWCWeight(w, device="cuda:0", layout=layout)
        h = N.NWCWeight(w, device="cpu", layout=layout)
    assert g._slot and not h._slot and g.bytes == h.bytes
    tg, th = g.tensors(), h.tensors()
    assert tg.keys() == th.keys()
    for name in th:
        assert torch.equal(tg[name].cpu(), th[name]), name
