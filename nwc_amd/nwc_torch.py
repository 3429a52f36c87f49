"""PyTorch side of NWC on AMD Instinct MI355X: modules that keep BF16 (or weight-only fp8) weights losslessly
compressed in HBM and multiply through the gfx950 library.

    one token (batch 1)  -> fused decode-matvec kernel, weights decoded in registers (nwc_linear_xbf16)
    several tokens       -> the matrix decompressed into a temporary BF16 buffer, then F.linear (hipBLASLt)

The public names, arguments, buffer contracts and exceptions are those of the reference bridge (parda21/NWC
nwc/nwc_torch.py: NWCWeight :126-269, NWCLinear :306-327, NWCEmbedding :330-344, fuse :360-386, convert :389-445,
quantize_fp8 :88-94, RefFP8Linear :272-290), so code written against `nwc` runs against `nwc_amd`.  The structure
below is this package's own.  There is no CPU fallback: compute methods need the HIP library and a GPU; the host
encoder needs only the library.
"""
import os
from typing import NamedTuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import _abi
from ._abi import call, lib, ptr, stream

_LIB_PATH = _abi.LIB_PATH
VERSION, NSTATE, TAB_WORDS, HDR_BLOCK, FIXED_BLOCK = (_abi.VERSION, _abi.NSTATE, _abi.TAB_WORDS, _abi.HDR_BLOCK,
                                                      _abi.FIXED_BLOCK)
ELEM, LAYOUT1, LAYOUT2 = _abi.HAS_ELEM, _abi.HAS_LAYOUT1, _abi.HAS_LAYOUT2
V9 = VERSION >= 9
X_FP32 = True                     # the reference ABI's layout-0 token path takes x as fp32

LANES = 32                        # lane streams per block
NPAIR = 1024                      # length of the encoder's freq/psym buffers
RAW_SLACK = 512                   # bytes after the raw plane `low` that the kernels may read
DATA_SLACK = 64                   # zero bytes kept after the encoder's output in `data`
SEQ_TABLE_WORDS = 8196            # 13-bit decode table + exp_of_rank
ELEM_BF16, ELEM_FP8 = 0, 1
ELEMS = {"bf16": ELEM_BF16, "fp8": ELEM_FP8}
LAYOUTS = (0, 1, 2)
_default_layout = int(os.environ.get("NWC_LAYOUT", "0"))
LAYOUT_DEFAULT = {ELEM_BF16: _default_layout, ELEM_FP8: _default_layout}
SEQ_TABLE = os.environ.get("NWC_SEQ_TABLE", "1") != "0"   # layouts 0/1: stage the 13-bit decode table
# layouts 0/1 on a GPU: each block's streams in a slot of one fixed stride, so the token kernels compute a block's
# offset instead of reading it before they can request the streams (Qwen3-4B layout-0 sweep 1577 -> 1523 us per token)
FIXED_SLOTS = os.environ.get("NWC_FIXED_SLOTS", "1") != "0"
SLOT_MAX = {0: 1728, 1: 3040}     # the library's largest stride per layout (nwc_format.h kSlotMax0 / kSlotMax1)
SLOT_OVERHEAD = 1.15              # slots only where they hold at most 15% more bytes than the packed streams
SLOT_TAIL = 2 * DATA_SLACK        # zero bytes after the last slot (the packed form keeps 64 + DATA_SLACK)
ROW_INDEX = os.environ.get("NWC_ROW_INDEX", "1") != "0"   # layouts 0/1: build the row index for the token path
# layout 0: inputs of 2..BATCH_MAX tokens go through the fused kernel (four vectors per launch) instead of a
# temporary BF16 matrix + F.linear
BATCH_MAX = int(os.environ.get("NWC_BATCH_MAX", "8"))
BATCH_LAUNCH = 4                                           # vectors per nwc_linear_xbf16_batch launch
# more tokens, layout 0: "dequant" (default) decompresses into a temporary BF16 matrix and multiplies it with
# linear_dequantized (hipBLASLt, or the library's GEMM where that is faster); "fused" runs nwc_prefill_xbf16 (decode
# into LDS + matrix cores, no temporary matrix; correct, but slower on MI355X at 512 tokens: 19 ms against 8.0 ms
# per Qwen3-4B stack)
PREFILL = os.environ.get("NWC_PREFILL", "dequant")
# the prefill GEMM on the temporary matrix: "auto" (default) the library's split-K matrix-core kernel
# (nwc_gemm_xbf16) for the shapes where it measured faster than hipBLASLt on MI355X, torch's F.linear for the rest;
# "nwc" the library kernel wherever it applies; "hipblaslt" F.linear always
GEMM = os.environ.get("NWC_GEMM", "auto")
FP8_MAX = 448.0


def _check_layout(layout):
    if layout not in LAYOUTS:
        raise ValueError(f"unknown layout {layout}")


def _need_gpu(t):
    if t.device.type != "cuda":
        raise RuntimeError("NWC kernels run on the GPU: move the NWCWeight to a cuda device")


# ---------------------------------------------------------------------------------------------------------------
# weight-only fp8

def _absmax_scale(wf):
    """Per-row fp32 scale: absmax / 448, with absmax floored at 1e-12 so all-zero rows divide safely.  The divisor
    is a tensor, not a Python number: torch on the GPU multiplies by the rounded reciprocal of a host scalar, which
    is one ulp off the quotient for some rows, while a tensor divisor gives the correctly rounded quotient on every
    device, as the CPU does."""
    amax = wf.abs().amax(dim=1).clamp_min(1e-12)
    return amax / torch.full_like(amax, FP8_MAX)


def quantize_fp8(w: torch.Tensor):
    """[out, in] BF16 or float -> (float8_e4m3fn codes, fp32 scale[out]).  Each row is divided by its scale,
    clamped to +-448 and rounded to nearest even e4m3 (reference nwc_torch.py:88-94)."""
    wf = w.detach().float()
    scale = _absmax_scale(wf)
    scaled = torch.clamp(wf / scale.unsqueeze(1), min=-FP8_MAX, max=FP8_MAX)
    return scaled.to(torch.float8_e4m3fn), scale


def ref_fp8_matvec(w8: torch.Tensor, scale: torch.Tensor, x_f32: torch.Tensor) -> torch.Tensor:
    """Uncompressed fp8 weight-only matvec of the library (the bandwidth baseline): BF16 y = scale * (W8 x)."""
    _need_gpu(w8)
    rows, cols = w8.shape
    y = torch.empty(rows, dtype=torch.bfloat16, device=w8.device)
    pad = -x_f32.numel() % 16
    xin = (F.pad(x_f32, (0, pad)) if pad else x_f32).contiguous()
    call("nwc_ref_fp8", stream(), ptr(w8.view(torch.uint8)), ptr(scale), ptr(xin), ptr(y), rows, cols)
    return y


def ref_bf16_matvec(w: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
    """Uncompressed BF16 matvec of the library (a bandwidth baseline next to hipBLASLt): BF16 y = RNE(W x), fp32
    accumulation; w BF16 [out, in] row-major, x BF16 [in]."""
    _need_gpu(w)
    rows, cols = w.shape
    y = torch.empty(rows, dtype=torch.bfloat16, device=w.device)
    wc, xc = w.contiguous(), x.to(torch.bfloat16).contiguous()
    call("nwc_ref_bf16", stream(), ptr(wc), ptr(xc), ptr(y), rows, cols)
    return y


# device index -> workspace of nwc_gemm_xbf16 (its counters are zero between calls).  Calls on one device share it,
# so they must not run concurrently on two streams.  A workspace that a larger one replaces stays allocated: graphs
# captured earlier keep its address.
_GEMM_WS = {}
_GEMM_WS_RETIRED = []


def gemm_usable(x: torch.Tensor, weight: torch.Tensor) -> bool:
    """Whether gemm_xbf16 takes this product: BF16 on the GPU, K a multiple of 64, rows of 16-byte multiples."""
    return (x.dtype == torch.bfloat16 and weight.dtype == torch.bfloat16 and x.is_cuda and x.device == weight.device
            and weight.dim() == 2 and weight.shape[1] % 64 == 0 and weight.stride(1) == 1
            and weight.stride(0) % 8 == 0 and weight.data_ptr() % 16 == 0)


def gemm_preferred(tokens: int, out_features: int, in_features: int) -> bool:
    """Where nwc_gemm_xbf16 beats hipBLASLt on MI355X (graph-timed against F.linear, 16-2048 tokens on the Qwen3-4B
    projection shapes): K of 8192 or more at 128-768 tokens (the down projection, 2560 x 9728: 1.08-1.70x), where the
    output has few 128 x 128 tiles and the split over K fills the CUs.  Everywhere else hipBLASLt was faster."""
    return in_features >= 8192 and 128 <= tokens <= 768


def linear_dequantized(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor = None) -> torch.Tensor:
    """The prefill product on a dequantized matrix, F.linear(x, weight, bias): the library GEMM (gemm_xbf16) where
    NWC_GEMM and gemm_preferred choose it, torch's F.linear (hipBLASLt) otherwise.  The choice depends on the shapes
    only, so a dequantized matrix and the same matrix resident in BF16 go through the same GEMM."""
    chosen = GEMM == "nwc" or (GEMM == "auto" and gemm_preferred(x.numel() // weight.shape[1], *weight.shape))
    if chosen and gemm_usable(x, weight) and (bias is None or bias.device == weight.device):
        return gemm_xbf16(x, weight, bias)
    return F.linear(x, weight, bias)


def gemm_xbf16(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor = None) -> torch.Tensor:
    """F.linear(x, weight, bias) in BF16 through the library's split-K matrix-core GEMM (nwc_gemm_xbf16): x [..., K],
    weight [N, K] (a row-strided view such as dequant()'s is fine), bias [N] or None; fp32 accumulation, one RNE
    rounding of the sum + bias.  The partial sums are added in a fixed order: equal inputs give equal bits."""
    _need_gpu(weight)
    for name, t in (("x", x), ("bias", bias)):
        if t is not None and t.device != weight.device:
            raise RuntimeError(f"gemm_xbf16: {name} is on {t.device}, the weight on {weight.device}")
    N, K = weight.shape
    xs = x.reshape(-1, K)
    if xs.stride(-1) != 1 or xs.stride(0) % 8 or xs.data_ptr() % 16:
        xs = xs.contiguous()
    T = xs.shape[0]
    y = torch.empty(T, N, dtype=torch.bfloat16, device=weight.device)
    if T == 0:
        return y.view(*x.shape[:-1], N)
    need = int(lib.nwc_gemm_workspace(T, N, K))
    ws = None
    if need:
        key = weight.device.index
        ws = _GEMM_WS.get(key)
        if ws is None or ws.numel() < need:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("gemm_xbf16: run this shape once outside graph capture first (workspace)")
            if ws is not None:
                _GEMM_WS_RETIRED.append(ws)
            ws = _GEMM_WS[key] = torch.zeros(need, dtype=torch.uint8, device=weight.device)
    b = None if bias is None else bias.to(torch.bfloat16).contiguous()
    call("nwc_gemm_xbf16", stream(), ptr(xs), xs.stride(0), ptr(weight), weight.stride(0), ptr(b), ptr(y), T, N, K,
         ptr(ws), 0 if ws is None else ws.numel())
    return y.view(*x.shape[:-1], N)


def fits(out_features, in_features):
    """Whether the format can hold a matrix of this shape: any size, padded to whole blocks."""
    return out_features >= 1 and in_features >= 1


def choose_block(n):
    """Weights per block: fixed at 4096 (8 x 512) by the format."""
    return FIXED_BLOCK


# ---------------------------------------------------------------------------------------------------------------
# host-side encoding and validation of the compressed tensors

class _Geometry(NamedTuple):
    blocks: int           # 8 x 512 (layout 0) or 16 x 512 (layouts 1/2) blocks
    raw_bytes: int        # bytes of the raw plane `low`, without its slack
    scratch_floats: int   # Mp * CB, the reference's partial-sum scratch
    K16: int              # in_features rounded up to 16


def _geometry(rows, cols, code) -> _Geometry:
    out = torch.empty(4, dtype=torch.int64)
    if lib.nwc_layout(rows, cols, code, ptr(out)):
        raise RuntimeError(f"nwc_layout refused a {rows} x {cols} matrix")
    return _Geometry(*out.tolist())


def _encoder_capacities(n, blocks):
    """data buffers to try: about 4 bits per weight first (streams of real or Gaussian weights need under 3), then
    the worst case of 24 bits per weight (every weight an escape or an exception)."""
    slack = 64 * blocks + 4096
    return (n // 2 + slack, 3 * n + slack)


def _encode(src, rows, cols, code):
    """Run the host encoder on row-major source bits (int16 BF16 or uint8 fp8, CPU).  Returns the five stored
    tensors on the CPU: data (the encoder's bytes + DATA_SLACK zero bytes), bases, hdr, lut, low (+ RAW_SLACK)."""
    geo = _geometry(rows, cols, code)
    n = rows * cols
    freq = torch.empty(NPAIR, dtype=torch.int16)
    psym = torch.empty(NPAIR, dtype=torch.int16)
    bases = torch.empty(geo.blocks, dtype=torch.int32)
    hdr = torch.empty(geo.blocks * HDR_BLOCK, dtype=torch.uint8)
    low = torch.zeros(geo.raw_bytes + RAW_SLACK, dtype=torch.uint8)
    length, buf = -1, None
    for cap in _encoder_capacities(n, geo.blocks):
        buf = torch.empty(cap, dtype=torch.uint8)
        length = lib.nwc_encode(ptr(src), n, cols, code, ptr(freq), ptr(psym), ptr(bases), ptr(hdr), ptr(buf), cap,
                                ptr(low))
        if length != -1:
            break
    if length == -2:
        raise ValueError("fp8 weights contain NaN")
    if length == -3:
        raise ValueError("layout 2 cannot code this matrix (a lane stream has more than 255 exceptions); "
                         "use layout 0 or 1")
    if length < 0:
        raise RuntimeError(f"nwc_encode failed ({length})")
    lut = torch.empty(TAB_WORDS, dtype=torch.int32)
    lib.nwc_build_tab(ptr(freq), ptr(psym), code, ptr(lut))
    data = torch.zeros(length + DATA_SLACK, dtype=torch.uint8)
    data[:length] = buf[:length]
    return {"data": data, "bases": bases, "hdr": hdr, "lut": lut, "low": low}, length, geo


def _validate_streams(bases, hdr, data_len, layout, elem):
    """Structural check of stored tensors before any kernel reads them.  Block bases are 8-byte aligned byte
    offsets; every block's lane streams (layouts 0/1: 4 bytes per header word) or exception entries (layout 2: 3
    bytes, fp8 2) end at or before the next block's base, and the last block's end leaves the decoder's read-ahead
    slack inside `data`.  A tensor set that breaks this (a corrupt or foreign checkpoint) would make the kernels
    read outside their buffers, so it is refused with ValueError."""
    if bases.numel() == 0:
        return
    start = bases.to(torch.int64) & 0xFFFFFFFF
    words = hdr.to(torch.int64).view(-1, LANES).sum(1)
    unit = 4 if layout != 2 else (2 if elem == ELEM_FP8 else 3)
    end = start + words * unit
    tail = DATA_SLACK if layout != 2 else 0
    if bool((start % 8 != 0).any()):
        raise ValueError("block bases are not 8-byte aligned: corrupt checkpoint")
    if bool((start[1:] < end[:-1]).any()):
        raise ValueError("block streams overlap or go backwards: corrupt checkpoint")
    if int(end[-1]) + tail > data_len:
        raise ValueError("compressed streams run past the data tensor: corrupt checkpoint")


def _block_spans(bases, hdr):
    """int64 byte offset and byte length of every block's lane streams (layouts 0/1: four bytes per header word)."""
    start = bases.to(torch.int64) & 0xFFFFFFFF
    return start, hdr.view(-1, LANES).to(torch.int64).sum(1) * 4


def _copy_spans(src, dst, src_start, dst_start, size, chunk=2048):
    """dst[dst_start[b] + j] = src[src_start[b] + j] for every block b and j < size[b], a chunk of blocks at a time."""
    j = torch.arange(int(size.max()), device=src.device)
    for b0 in range(0, size.numel(), chunk):
        part = slice(b0, b0 + chunk)
        keep = j[None, :] < size[part, None]
        dst[(dst_start[part, None] + j[None, :])[keep]] = src[(src_start[part, None] + j[None, :])[keep]]


# ---------------------------------------------------------------------------------------------------------------

class NWCWeight:
    """An [out, in] matrix held compressed on the GPU.
    elem "bf16": the BF16 weights, lossless.  elem "fp8": weight-only fp8 e4m3 with an fp32 scale per output row
    (quantized here from a BF16 matrix, or given as a float8 tensor plus `scale`); the fp8 codes are stored lossless.
    The stored tensors are the format's (data, bases, hdr, lut, low, and scale for fp8); the row index and the
    13-bit decode table are derived from them on first use and are not part of the format."""

    def __init__(self, w: torch.Tensor, device="cuda", block=None, elem="bf16", scale=None, layout=None):
        assert w.dim() == 2, "a 2-D weight matrix is expected"
        rows, cols = w.shape
        assert fits(rows, cols), f"shape {tuple(w.shape)} not supported"
        kind = ELEMS[elem]
        layout = LAYOUT_DEFAULT[kind] if layout is None else int(layout)
        _check_layout(layout)
        src, scale = self._source(w, kind, scale)
        self._shape(rows, cols, block, kind, layout)
        stored, length, geo = _encode(src, rows, cols, self.code)
        self._place(stored, scale, device, geo)
        self.bytes = self._stored_bytes(length)
        self._derive()

    @staticmethod
    def _source(w, kind, scale):
        """Row-major source bits on the CPU and the fp32 row scale (fp8 only)."""
        if kind == ELEM_BF16:
            assert w.dtype == torch.bfloat16, "BF16 expected (elem='fp8' for fp8 weights)"
            return w.detach().contiguous().cpu().view(torch.int16), None
        if w.dtype == torch.float8_e4m3fn:
            if scale is None:
                raise ValueError("fp8 weights need their per-row scale")
            codes = w
        else:
            codes, scale = quantize_fp8(w)
        return codes.detach().contiguous().cpu().view(torch.uint8), scale.detach().float().contiguous()

    def _shape(self, rows, cols, block, kind, layout):
        self.out_features, self.in_features = rows, cols
        self.n = rows * cols
        self.block = block or choose_block(self.n)
        self.elem, self.layout = kind, layout
        self._slot, self._packed = 0, None

    def _place(self, stored, scale, device, geo):
        for name in ("data", "bases", "hdr", "lut", "low"):
            setattr(self, name, stored[name].to(device))
        self.scale = None if scale is None else scale.float().to(device)
        self.K16 = geo.K16
        self._raw_bytes, self._n_scratch = geo.raw_bytes, geo.scratch_floats
        self._scratch = self._row_index = self._seq_table = None
        self.bytes_bf16 = 2 * self.n
        self.bytes_native = self.n + 4 * self.out_features if self.elem == ELEM_FP8 else 2 * self.n
        self._packed_len = self.data.numel()
        # (not inside HIP-graph capture: the move ends in a host read of two sums)
        if (self.layout <= 1 and FIXED_SLOTS and self.data.device.type == "cuda" and self.bases.numel()
                and not torch.cuda.is_current_stream_capturing()):
            self._to_slots()

    def _to_slots(self):
        """Move the block streams of layouts 0/1 into slots of one stride (the largest block's bytes, rounded up to
        16): block b at byte b * stride, so bases[b] = b * stride, which is still a valid tensor set of the format.
        Kept packed when the slots would hold more than SLOT_OVERHEAD times the bytes, when the stride passes the
        layout's SLOT_MAX, or when `data` holds non-zero bytes outside the blocks' streams (tensors() could not restore
        it exactly)."""
        start, size = _block_spans(self.bases, self.hdr)
        nb = size.numel()
        stride = -(-int(size.max()) // 16) * 16
        if not 0 < stride <= SLOT_MAX[self.layout] or nb * stride > SLOT_OVERHEAD * self._packed_len \
                or nb * stride + SLOT_TAIL >= 1 << 31:
            return
        slots = torch.zeros(nb * stride + SLOT_TAIL, dtype=torch.uint8, device=self.data.device)
        first = torch.arange(nb, device=self.data.device, dtype=torch.int64) * stride
        _copy_spans(self.data, slots, start, first, size)
        # the copy holds every stream byte, so equal sums mean every byte outside the streams is zero
        if int(slots.sum(dtype=torch.int64)) != int(self.data.sum(dtype=torch.int64)):
            return
        self._packed = self.bases
        self.data, self.bases, self._slot = slots, first.to(torch.int32), stride

    def _stored_bytes(self, stream_bytes):
        """Compressed size: streams + bases + header + table + raw plane (+ fp8 scale), the reference's `bytes`."""
        scale = 4 * self.scale.numel() if self.scale is not None else 0
        return stream_bytes + 4 * self.bases.numel() + self.hdr.numel() + 4 * self.lut.numel() + self._raw_bytes + scale

    @classmethod
    def from_tensors(cls, out_f, in_f, block, data, bases, hdr, lut, low, device="cuda", elem="bf16", scale=None,
                     layout=0):
        """Rebuild from stored tensors (a checkpoint), without the original weights.  Tensors that do not match the
        shape, or whose streams are malformed, raise ValueError before anything reaches the GPU."""
        self = cls.__new__(cls)
        kind, layout = ELEMS[elem], int(layout)
        _check_layout(layout)
        self._shape(out_f, in_f, block, kind, layout)
        geo = _geometry(out_f, in_f, self.code)
        for name, t, dtype in (("data", data, torch.uint8), ("bases", bases, torch.int32), ("hdr", hdr, torch.uint8),
                               ("lut", lut, torch.int32), ("low", low, torch.uint8)):
            if t.dtype != dtype:
                # the kernels read these bytes as u8 / u32 words: another dtype would move every offset and length
                raise ValueError(f"checkpoint tensor {name} is {t.dtype}, expected {dtype}")
        if kind == ELEM_FP8 and (scale is None or not scale.dtype.is_floating_point or scale.numel() != out_f):
            raise ValueError("fp8 checkpoint needs a floating-point scale with one value per output row")
        data, bases, hdr, lut, low = (t.reshape(-1).contiguous() for t in (data, bases, hdr, lut, low))
        if (bases.numel() != geo.blocks or hdr.numel() != geo.blocks * HDR_BLOCK or lut.numel() != TAB_WORDS
                or low.numel() not in (geo.raw_bytes, geo.raw_bytes + RAW_SLACK)):
            raise ValueError("checkpoint does not match this library version")
        _validate_streams(bases.cpu(), hdr.cpu(), data.numel(), layout, kind)
        if low.numel() == geo.raw_bytes:
            low = F.pad(low, (0, RAW_SLACK))
        self._place({"data": data, "bases": bases, "hdr": hdr, "lut": lut, "low": low}, scale, device, geo)
        self.bytes = self._stored_bytes(self._packed_len)
        self._derive()
        return self

    def tensors(self):
        """The stored tensors (what a checkpoint keeps); streams in fixed slots are packed back to the bytes they
        were placed from."""
        out = {name: getattr(self, name) for name in ("data", "bases", "hdr", "lut", "low")}
        if self._slot:
            start, size = _block_spans(self._packed, self.hdr)
            data = torch.zeros(self._packed_len, dtype=torch.uint8, device=self.data.device)
            _copy_spans(self.data, data, self.bases.to(torch.int64), start, size)
            out["data"], out["bases"] = data, self._packed
        if self.scale is not None:
            out["scale"] = self.scale
        return out

    @property
    def code(self):
        """The library's `elem` argument: element type in bits 0-3, layout in bits 4-7, the fixed-slot stride / 16
        in bits 8-15 (0: blocks at bases[])."""
        return self.elem | (self.layout << 4) | (self._slot // 16) << 8

    @property
    def scratch(self):
        """fp32 [Mp * CB] scratch of the reference ABI.  The gfx950 kernels reduce the column-block partial sums
        inside a workgroup and never touch it, so it is allocated only when asked for."""
        if self._scratch is None:
            self._scratch = torch.empty(self._n_scratch, dtype=torch.float32, device=self.data.device)
        return self._scratch

    def _streams(self):
        return ptr(self.data), ptr(self.bases), ptr(self.hdr), ptr(self.lut), ptr(self.low)

    # ---- derived structures (built once per matrix) ----
    def _derive(self):
        """Build the row index and the 13-bit table when the matrix is placed on a GPU, so that no later call, for
        instance inside HIP-graph capture, has to build them."""
        if self.data.device.type == "cuda" and not torch.cuda.is_current_stream_capturing():
            self.row_index()
            self.seq_table()

    @staticmethod
    def _not_capturing(what):
        # a build recorded into a graph would not run before the graph is replayed, and the 13-bit table's host copy
        # is not capturable: refuse rather than cache a tensor that was never written
        if torch.cuda.is_available() and torch.cuda.is_current_stream_capturing():
            raise RuntimeError(f"NWCWeight.{what}() is built on first use and cannot be built during HIP-graph capture; "
                               f"call it once before capturing")

    def row_index(self):
        """uint16 [blocks x 3 x 32]: each lane's bit position at rows 2, 4, 6 (layout 0) or super-chunks 4, 8, 12
        (layout 1), built on the GPU on first use, so the token kernels can split a block over two or four
        half-waves.  None for layout 2, for layout-1 shapes the index kernel has no plan for, or with
        NWC_ROW_INDEX=0."""
        if self.layout > 1 or not ROW_INDEX:
            return None
        if self._row_index is None:
            _need_gpu(self.data)
            self._not_capturing("row_index")
            index = torch.empty(self.bases.numel() * 3 * LANES, dtype=torch.int16, device=self.data.device)
            rc = lib.nwc_row_index(stream(), *self._streams(), ptr(index), self.n, self.in_features, self.code)
            if rc == -1 and self.layout == 1:
                index = False                                  # no plan for this shape: decode without an index
            elif rc:
                raise RuntimeError(f"nwc_row_index error {rc}")
            self._row_index = index
        return self._row_index if self._row_index is not False else None

    def seq_table(self):
        """int32 [8196] 13-bit decode table of layouts 0/1 on the device, built on the host from the stored LUT on
        first use.  None for layout 2 or with NWC_SEQ_TABLE=0."""
        if self.layout > 1 or not SEQ_TABLE:
            return None
        if self._seq_table is None:
            self._not_capturing("seq_table")
            table = torch.empty(SEQ_TABLE_WORDS, dtype=torch.int32)
            lut = self.lut.cpu().contiguous()
            if lib.nwc_seq_table(ptr(lut), self.code, ptr(table)):
                raise RuntimeError("nwc_seq_table failed")
            self._seq_table = table.to(self.data.device)
        return self._seq_table

    def token_bytes(self):
        """Bytes one token-path call reads: the compressed matrix, the row-index entries its plan uses (64 per block
        at two half-waves per block, 192 at four) and the 13-bit table."""
        flags = int(self.row_index() is not None) | int(self.seq_table() is not None) << 1
        split = lib.nwc_token_split(self.n, self.in_features, self.code, flags)
        table = 4 * SEQ_TABLE_WORDS if self.seq_table() is not None else 0
        return self.bytes + self.bases.numel() * LANES * 2 * (split - 1) + table

    # ---- compute ----
    def _padded(self, x):
        """x zero-extended to the kernels' width: K16 (layout 0) or in_features rounded up to 32 (layouts 1/2)."""
        width = -(-self.in_features // 32) * 32 if self.layout else self.K16
        extra = width - self.in_features
        x = (F.pad(x, (0, extra)) if extra else x).contiguous()
        return x if x.data_ptr() % 16 == 0 else x.clone()          # the kernels read x in 16-byte pieces

    def matvec(self, x_f32: torch.Tensor) -> torch.Tensor:
        """fp32 test path: y = W x in fp32 (times the row scale for fp8)."""
        _need_gpu(self.data)
        y = torch.empty(self.out_features, dtype=torch.float32, device=x_f32.device)
        xin = self._padded(x_f32.float())
        call("nwc_matvec", stream(), *self._streams(), ptr(xin), ptr(y), self.n, self.block, self.in_features,
             self.code)
        return y if self.scale is None else y * self.scale

    def linear_bf16(self, x: torch.Tensor, bias) -> torch.Tensor:
        """Token path: BF16 y = scale * (W x) + bias for one activation vector (BF16 or fp32)."""
        _need_gpu(self.data)
        y = torch.empty(self.out_features, dtype=torch.bfloat16, device=x.device)
        if x.dtype == torch.bfloat16 or self.layout:
            # BF16 activations (layouts 1/2 always take them): the extended entry point with the derived structures
            xin = self._padded(x.to(torch.bfloat16))
            call("nwc_linear_xbf16", stream(), *self._streams(), ptr(self.row_index()), ptr(self.seq_table()),
                 ptr(xin), ptr(bias), ptr(self.scale), ptr(y), self.n, self.in_features, self.code)
        else:
            # layout 0 with fp32 activations: the reference's entry point
            xin = self._padded(x.float())
            call("nwc_linear_bf16", stream(), *self._streams(), ptr(xin), ptr(bias), ptr(self.scale), None, ptr(y),
                 self.n, self.block, self.in_features, self.code)
        return y

    def linear_batch(self, x: torch.Tensor, bias) -> torch.Tensor:
        """Token path for a few BF16 vectors at once, layout 0: x [T, in_features] -> y BF16 [T, out_features], the
        matrix decoded once per four vectors (y[t] equals linear_bf16(x[t]) bit for bit)."""
        _need_gpu(self.data)
        if self.layout != 0:
            raise ValueError("linear_batch: layout 0 only")
        T = x.shape[0]
        xin = torch.zeros(T, self.K16, dtype=torch.bfloat16, device=x.device)
        xin[:, :self.in_features] = x
        y = torch.empty(T, self.out_features, dtype=torch.bfloat16, device=x.device)
        for t0 in range(0, T, BATCH_LAUNCH):
            nt = min(BATCH_LAUNCH, T - t0)
            call("nwc_linear_xbf16_batch", stream(), *self._streams(), ptr(self.seq_table()), ptr(xin[t0]), ptr(bias),
                 ptr(self.scale), ptr(y[t0]), self.n, self.in_features, self.code, nt)
        return y

    def prefill(self, x: torch.Tensor, bias) -> torch.Tensor:
        """Several BF16 tokens at once, layout 0, without a temporary BF16 matrix: x [T, in_features] -> y BF16
        [T, out_features] = x W^T (fp8: times the row scales) + bias, accumulated in fp32 on the matrix cores
        (nwc_prefill_xbf16; equal to F.linear on the decompressed matrix up to fp32 summation order)."""
        _need_gpu(self.data)
        if self.layout != 0:
            raise ValueError("prefill: layout 0 only")
        T = x.shape[0]
        if (self.K16 == self.in_features and x.dtype == torch.bfloat16 and x.is_contiguous()
                and x.data_ptr() % 16 == 0):         # the kernel reads x in 16-byte pieces
            xin = x
        else:
            xin = torch.zeros(T, self.K16, dtype=torch.bfloat16, device=x.device)
            xin[:, :self.in_features] = x
        y = torch.empty(T, self.out_features, dtype=torch.bfloat16, device=x.device)
        call("nwc_prefill_xbf16", stream(), *self._streams(), ptr(self.row_index()), ptr(self.seq_table()), ptr(xin),
             ptr(bias), ptr(self.scale), ptr(y), self.n, self.in_features, self.code, T)
        return y

    def gather(self, ids: torch.Tensor) -> torch.Tensor:
        """Rows `ids` as BF16 [..., in_features], decoded straight from the compressed matrix (embedding lookup)."""
        _need_gpu(self.data)
        flat = ids.reshape(-1).to(device=self.data.device, dtype=torch.int64).contiguous()
        rows = torch.empty(flat.numel(), self.K16, dtype=torch.bfloat16, device=self.data.device)
        index = self.row_index()
        if index is not None:      # layouts 0/1: decode from the row index's starts (same rows, bit for bit)
            call("nwc_gather_xindex", stream(), *self._streams(), ptr(index), ptr(self.seq_table()), ptr(flat),
                 flat.numel(), ptr(rows), self.n, self.in_features, self.code)
        else:
            call("nwc_gather", stream(), *self._streams(), ptr(flat), flat.numel(), ptr(rows), self.n, self.block,
                 self.in_features, self.code)
        if self.K16 != self.in_features:
            rows = rows[:, :self.in_features].contiguous()
        return rows.view(*ids.shape, self.in_features)

    def dequant(self, out: torch.Tensor = None) -> torch.Tensor:
        """The matrix decompressed to BF16, row-major; a view with row stride K16 when K is not a multiple of 16.
        fp8: the unscaled fp8 values (exact in BF16).  `out` may supply a BF16 [out_features, K16] buffer."""
        _need_gpu(self.data)
        if out is None:
            out = torch.empty((self.out_features, self.K16), dtype=torch.bfloat16, device=self.data.device)
        table = self.seq_table()
        if table is not None:
            call("nwc_dequant_seq", stream(), *self._streams(), ptr(self.row_index()), ptr(table), ptr(out), self.n,
                 self.in_features, self.code)
        else:
            call("nwc_dequant", stream(), *self._streams(), ptr(out), self.n, self.block, self.in_features, self.code)
        return out if self.K16 == self.in_features else out[:, :self.in_features]

    def dequant_fp8(self):
        """fp8 matrices: (float8_e4m3fn [out, in], fp32 scale[out]), bit-exact with what was encoded."""
        if self.elem != ELEM_FP8:
            raise ValueError("not an fp8 matrix")
        return self.dequant().to(torch.float8_e4m3fn), self.scale


# ---------------------------------------------------------------------------------------------------------------
# modules

def _bf16_bias(bias, device):
    if bias is None:
        return None
    return nn.Parameter(bias.detach().to(device=device, dtype=torch.bfloat16), requires_grad=False)


class NWCLinear(nn.Module):
    """nn.Linear over a compressed matrix (elem "bf16" lossless, or "fp8" weight-only).  One BF16 token goes through
    the fused decode-matvec kernel, up to NWC_BATCH_MAX (8) BF16 tokens of a layout-0 matrix through the batched one
    (the matrix decoded once per four tokens); anything else through a temporary BF16 matrix and linear_dequantized
    (hipBLASLt, or the library's split-K GEMM where that is faster), or, with NWC_PREFILL=fused, BF16 tokens of a
    layout-0 matrix through the fused prefill kernel (NWCWeight.prefill)."""

    def __init__(self, linear: nn.Linear = None, device="cuda", block=None, w: "NWCWeight" = None, bias=None,
                 elem="bf16"):
        super().__init__()
        self.w = NWCWeight(linear.weight.data, device, block, elem=elem) if w is None else w
        self.in_features, self.out_features = self.w.in_features, self.w.out_features
        if linear is not None and linear.bias is not None:
            bias = linear.bias.data
        self.bias = _bf16_bias(bias, device)

    def _bias_data(self):
        return None if self.bias is None else self.bias.data

    def forward(self, x):
        if x.dtype == torch.bfloat16 and x.numel() == self.in_features:
            y = self.w.linear_bf16(x.contiguous().view(-1), self._bias_data())
            return y.view(*x.shape[:-1], self.out_features)
        tokens = x.numel() // self.in_features
        if x.dtype == torch.bfloat16 and self.w.layout == 0 and 1 < tokens <= BATCH_MAX and self.w.K16 <= 16384:
            y = self.w.linear_batch(x.reshape(tokens, self.in_features), self._bias_data())
            return y.view(*x.shape[:-1], self.out_features)
        if (PREFILL == "fused" and x.dtype == torch.bfloat16 and self.w.layout == 0 and self.w.row_index() is not None
                and self.w.seq_table() is not None):
            y = self.w.prefill(x.reshape(tokens, self.in_features), self._bias_data())
            return y.view(*x.shape[:-1], self.out_features)
        weight = self.w.dequant()
        if self.w.scale is None:
            return linear_dequantized(x, weight, self._bias_data())
        # fp8: the product of the unscaled codes, then the row scale and the bias in fp32
        y = linear_dequantized(x, weight).float() * self.w.scale
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype)

    def extra_repr(self):
        kind = "fp8" if self.w.elem == ELEM_FP8 else "bf16"
        return (f"in={self.in_features}, out={self.out_features}, elem={kind}, layout={self.w.layout}, "
                f"{self.w.bytes / 1e6:.1f} MB compressed of {self.w.bytes_bf16 / 1e6:.1f} MB BF16")


class NWCEmbedding(nn.Module):
    """nn.Embedding over a compressed matrix (shared with a tied output projection); rows are decoded by the
    gather kernel, fp8 rows then scaled."""

    def __init__(self, emb: nn.Embedding = None, w: NWCWeight = None, padding_idx=None):
        super().__init__()
        self.w = w
        self.num_embeddings, self.embedding_dim = w.out_features, w.in_features
        self.padding_idx = padding_idx if emb is None else emb.padding_idx

    def forward(self, ids):
        rows = self.w.gather(ids)
        if self.w.scale is None:
            return rows
        row_scale = self.w.scale[ids.to(self.w.scale.device)].unsqueeze(-1)
        return (rows.float() * row_scale).to(torch.bfloat16)

    def extra_repr(self):
        return (f"{self.num_embeddings}, {self.embedding_dim}, {self.w.bytes / 1e6:.1f} MB compressed of "
                f"{self.w.bytes_bf16 / 1e6:.1f} MB BF16")


class _FusedGroup:
    """Sibling projections that read the same input, concatenated into one compressed matrix.  The first slice
    computes the whole product; later slices called with the same input tensor reuse it."""

    def __init__(self, lin: NWCLinear, names, sizes):
        self.lin, self.names, self.sizes = lin, list(names), list(sizes)
        self.starts = [sum(self.sizes[:i]) for i in range(len(self.sizes))]
        self._input = self._output = None

    def output(self, index, x):
        if index == 0 or self._input is not x or self._output is None:
            self._output = self.lin(x)
            self._input = x
        a = self.starts[index]
        return self._output[..., a:a + self.sizes[index]]


class _FusedSlice(nn.Module):
    """Stands in for one projection of a fused group: its rows of the group's output."""

    def __init__(self, group: _FusedGroup, index):
        super().__init__()
        self.group, self.index = group, index
        self.in_features, self.out_features = group.lin.in_features, group.sizes[index]

    def forward(self, x):
        return self.group.output(self.index, x)

    def extra_repr(self):
        return f"slice {self.index} of fused {'+'.join(self.group.names)}, out={self.out_features}"


def _children(model, kind):
    """(parent, attribute name, child) for every direct child of type `kind` anywhere in the model."""
    for parent in list(model.modules()):
        for name, child in list(parent.named_children()):
            if isinstance(child, kind):
                yield parent, name, child


def _release(*params):
    """Drop the host copies of converted weights."""
    for p in params:
        p.data = torch.empty(0)


def _concat_bias(linears, dtype):
    """Biases of fused projections: None if none has one, otherwise concatenated with zeros for the missing."""
    if all(l.bias is None for l in linears):
        return None
    parts = [l.bias.data if l.bias is not None else torch.zeros(l.out_features, dtype=dtype) for l in linears]
    return torch.cat(parts, 0)


def fuse(model: nn.Module, groups=(("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj")), device="cuda",
         elem="bf16"):
    """Concatenate sibling nn.Linear layers with the same input into one compressed matrix each (fewer, larger
    kernel launches).  Call before `convert`.  Returns the number of fused groups."""
    count = 0
    for parent in list(model.modules()):
        for names in groups:
            linears = [getattr(parent, nm, None) for nm in names]
            if not all(isinstance(l, nn.Linear) and l.weight.dtype == torch.bfloat16 for l in linears):
                continue
            if len({l.in_features for l in linears}) != 1:
                continue
            weight = torch.cat([l.weight.data for l in linears], 0)
            if not fits(*weight.shape):
                continue
            lin = NWCLinear(w=NWCWeight(weight, device, elem=elem), bias=_concat_bias(linears, weight.dtype),
                            device=device)
            group = _FusedGroup(lin, names, [l.out_features for l in linears])
            for index, (nm, l) in enumerate(zip(names, linears)):
                setattr(parent, nm, _FusedSlice(group, index))
                _release(l.weight)
            count += 1
    print(f"nwc_amd.fuse: {count} projection groups now share one compressed matrix each")
    return count


class _Tally:
    def __init__(self):
        self.nwc = self.bf16 = self.modules = 0
        self.skipped = []

    def add(self, w):
        self.nwc += w.bytes
        self.bf16 += w.bytes_bf16
        self.modules += 1


def _same_storage(a, b):
    return a is b or (a.numel() > 0 and a.data_ptr() == b.data_ptr())


def convert(model: nn.Module, device="cuda", verbose=True, tied=True, elem="bf16", embeddings=True):
    """Replace the model's BF16 nn.Linear layers by NWCLinear (and embeddings by NWCEmbedding), then move the
    model to `device`.  elem "bf16" is lossless; "fp8" stores weight-only fp8 e4m3 codes (per-row scale) losslessly.
    tied: an output projection that shares its weight with an embedding becomes one compressed matrix serving
    both (gather for the lookup, matvec for the logits).  embeddings: compress the other embedding tables too
    (always lossless BF16).  Returns (bytes_nwc, bytes_bf16) of the compressed matrices."""
    tally = _Tally()
    tables = [e for _, _, e in _children(model, nn.Embedding)]
    tied_tables, tied_linears = set(), set()

    # 1. output projections tied to an embedding table
    for parent, name, lin in list(_children(model, nn.Linear)):
        table = next((e for e in tables if _same_storage(e.weight, lin.weight)), None)
        if table is None:
            continue
        tied_tables.add(id(table))
        tied_linears.add(id(lin))
        if not (tied and table.weight.dtype == torch.bfloat16 and fits(*table.weight.shape)):
            tally.skipped.append(f"{name} {tuple(lin.weight.shape)} [tied]")
            continue
        w = NWCWeight(table.weight.data, device, elem=elem)
        setattr(parent, name, NWCLinear(lin, device, w=w))
        for p2, n2, e2 in list(_children(model, nn.Embedding)):
            if e2 is table:
                setattr(p2, n2, NWCEmbedding(table, w))
        tally.add(w)
        _release(table.weight, lin.weight)

    # 2. the other embedding tables (a table still tied to a BF16 projection stays as it is)
    if embeddings:
        for parent, name, table in list(_children(model, nn.Embedding)):
            if id(table) in tied_tables or table.weight.dtype != torch.bfloat16 or table.weight.numel() == 0 \
                    or not fits(*table.weight.shape):
                continue
            w = NWCWeight(table.weight.data, device, elem="bf16")
            setattr(parent, name, NWCEmbedding(table, w))
            tally.add(w)
            _release(table.weight)

    # 3. groups fused earlier
    seen = set()
    for module in model.modules():
        if isinstance(module, _FusedSlice) and id(module.group) not in seen:
            seen.add(id(module.group))
            tally.add(module.group.lin.w)

    # 4. every other BF16 linear layer
    for parent, name, lin in list(_children(model, nn.Linear)):
        if id(lin) in tied_linears:
            continue                                           # tied to a table that stays BF16 (listed above)
        if lin.weight.dtype == torch.bfloat16 and lin.weight.numel() and fits(lin.out_features, lin.in_features):
            new = NWCLinear(lin, device, elem=elem)
            setattr(parent, name, new)
            tally.add(new.w)
            _release(lin.weight)
        else:
            tally.skipped.append(f"{name} {tuple(lin.weight.shape)} [{lin.weight.dtype}]")

    model.to(device)
    if verbose:
        ratio = tally.nwc / max(tally.bf16, 1)
        print(f"nwc_amd.convert ({elem}): {tally.modules} matrices compressed, {tally.bf16 / 1e9:.2f} GB of BF16 held "
              f"in {tally.nwc / 1e9:.2f} GB ({ratio:.4f})")
        if tally.skipped:
            print("  left as they were:", ", ".join(tally.skipped[:6]) + (" ..." if len(tally.skipped) > 6 else ""))
    return tally.nwc, tally.bf16


# ---------------------------------------------------------------------------------------------------------------
# the uncompressed fp8 baseline

class RefFP8Linear(nn.Module):
    """Comparison only: weight-only fp8 without compression (same quantization as NWCWeight(elem="fp8")).  One
    BF16 token goes through the library's uncompressed fp8 matvec; anything else through a BF16 copy and
    F.linear."""

    def __init__(self, linear: nn.Linear, device="cuda"):
        super().__init__()
        codes, scale = quantize_fp8(linear.weight.data)
        self.w8, self.scale = codes.contiguous().to(device), scale.to(device)
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self.bias = _bf16_bias(None if linear.bias is None else linear.bias.data, device)

    def forward(self, x):
        if x.dtype == torch.bfloat16 and x.numel() == self.in_features:
            y = ref_fp8_matvec(self.w8, self.scale, x.reshape(-1).float())
            if self.bias is not None:
                y = y + self.bias
            return y.view(*x.shape[:-1], self.out_features)
        y = F.linear(x, self.w8.to(torch.bfloat16)).float() * self.scale
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype)


def convert_ref_fp8(model: nn.Module, device="cuda", verbose=True):
    """Replace every BF16 nn.Linear by RefFP8Linear; a projection tied to an embedding stays BF16.  Returns the
    number of replaced layers."""
    tables = [e.weight for _, _, e in _children(model, nn.Embedding)]
    count = 0
    for parent, name, lin in list(_children(model, nn.Linear)):
        if lin.weight.dtype != torch.bfloat16 or any(_same_storage(t, lin.weight) for t in tables):
            continue
        setattr(parent, name, RefFP8Linear(lin, device))
        _release(lin.weight)
        count += 1
    model.to(device)
    if verbose:
        print(f"nwc_amd.convert_ref_fp8: {count} linear layers as uncompressed fp8")
    return count
