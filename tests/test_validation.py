"""Stored tensors are checked before any kernel reads them (NWCWeight.from_tensors): a checkpoint whose block bases
go backwards, are not 8-byte aligned, or whose streams overlap the next block or run past `data` is refused with
ValueError on the host.  The kernels size their LDS copies from consecutive bases (a base that goes backwards would
wrap the copy's length), so these tensors must never reach the GPU.  CPU only."""
import pytest
import torch

from tests.helpers import bf16_matrix


def _weight(layout, elem="bf16"):
    pytest.importorskip("nwc_amd.nwc_torch", reason="the HIP library is not built")
    from nwc_amd.nwc_torch import NWCWeight, quantize_fp8
    w = bf16_matrix(40, 1100, seed=5)
    if elem == "fp8":
        q, s = quantize_fp8(w.float())
        return NWCWeight(q, device="cpu", elem="fp8", scale=s, layout=layout)
    return NWCWeight(w, device="cpu", layout=layout)


def _rebuild(c, **changes):
    from nwc_amd.nwc_torch import NWCWeight
    t = {k: v.clone() for k, v in c.tensors().items()}
    t.update(changes)
    return NWCWeight.from_tensors(c.out_features, c.in_features, c.block, t["data"], t["bases"], t["hdr"], t["lut"],
                                  t["low"], device="cpu", elem="fp8" if c.elem else "bf16", scale=t.get("scale"),
                                  layout=c.layout)


@pytest.mark.parametrize("layout,elem", [(0, "bf16"), (1, "bf16"), (2, "bf16"), (0, "fp8"), (2, "fp8")])
def test_intact_tensors_accepted(layout, elem):
    c = _weight(layout, elem)
    d = _rebuild(c)
    for name, t in c.tensors().items():
        assert torch.equal(t, d.tensors()[name])


@pytest.mark.parametrize("layout", [0, 1, 2])
def test_bases_going_backwards_refused(layout):
    c = _weight(layout)
    bases = c.bases.clone()
    assert bases.numel() >= 3
    bases[2] = bases[0]                    # block 2 claims the bytes of block 0
    with pytest.raises(ValueError):
        _rebuild(c, bases=bases)


@pytest.mark.parametrize("layout", [0, 2])
def test_misaligned_base_refused(layout):
    c = _weight(layout)
    bases = c.bases.clone()
    bases[1] += 4
    with pytest.raises(ValueError):
        _rebuild(c, bases=bases)


def test_streams_overlapping_next_block_refused():
    c = _weight(0)
    hdr = c.hdr.clone()
    hdr[0] = min(255, int(hdr[0]) + 40)    # lane 0 of block 0 now runs into block 1
    with pytest.raises(ValueError):
        _rebuild(c, hdr=hdr)


@pytest.mark.parametrize("layout", [0, 2])
def test_last_block_past_data_refused(layout):
    c = _weight(layout)
    with pytest.raises(ValueError):
        _rebuild(c, data=c.data[:int(c.bases[-1]) - 8].clone())     # the last block starts past the end


def test_wrong_sizes_refused():
    c = _weight(0)
    with pytest.raises(ValueError):
        _rebuild(c, bases=c.bases[:-1].clone())
    with pytest.raises(ValueError):
        _rebuild(c, low=c.low[:-7].clone())


@pytest.mark.parametrize("name,dtype", [("bases", torch.int64), ("hdr", torch.int32), ("lut", torch.int64),
                                        ("data", torch.int8), ("low", torch.int16), ("bases", torch.float32)])
def test_wrong_dtype_refused(name, dtype):
    """The kernels read data/hdr/low as bytes and bases/lut as 32-bit words: a tensor of another dtype (values kept,
    bytes reinterpreted) would move every offset and code length the validation checked, so it is refused."""
    c = _weight(0)
    t = getattr(c, name).clone()
    if t.element_size() == torch.tensor([], dtype=dtype).element_size() and not dtype.is_floating_point:
        t = t.view(dtype)
    else:
        t = t.to(dtype)
    with pytest.raises(ValueError, match=name):
        _rebuild(c, **{name: t})


def test_fp8_needs_float_scale():
    c = _weight(0, "fp8")
    with pytest.raises(ValueError):
        _rebuild(c, scale=c.scale.to(torch.int32))
    with pytest.raises(ValueError):
        _rebuild(c, scale=c.scale[:-1].clone())
