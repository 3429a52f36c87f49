"""NWC for PyTorch on AMD Instinct MI355X: NWCLinear keeps BF16 (or weight-only fp8) weights losslessly compressed in
HBM.

    batch 1 (token generation) -> fused decode-matvec kernel (decoded in registers, nwc_linear_xbf16)
    otherwise (prefill)        -> decompression into a temporary BF16 buffer + F.linear (hipBLASLt)

Mirror of the reference bridge parda21/NWC nwc/nwc_torch.py: same classes, functions, arguments, buffer contracts and
errors, over the gfx950 C-ABI library nwc_amd/lib/nwc_ops.so (include/nwc_ops.h).  There is no CPU fallback: the
compute entry points need the HIP library and a GPU, the host encoder needs only the library.
"""
import ctypes
import os

import torch
import torch.nn as nn
import torch.nn.functional as F

LANES = 32
NPAIR = 1024                      # size of the freq/psym buffers of the ABI
RAW_SLACK = 512                   # bytes appended to the raw plane (nwc_torch.py:43)


def _find_library():
    """Search order as in the reference (nwc_torch.py:14-22): NWC_DLL, then the package's lib/ directory."""
    here = os.path.dirname(os.path.abspath(__file__))
    candidates = [os.environ.get("NWC_DLL"), os.path.join(here, "lib", "nwc_ops.so")]
    for c in candidates:
        if c and os.path.exists(c):
            return c
    raise ImportError("NWC library not found: run `python -m nwc_amd.build` (needs hipcc, builds for gfx950); looked for "
                      + ", ".join(c for c in candidates if c))


_LIB_PATH = _find_library()
_lib = ctypes.CDLL(_LIB_PATH)
P = ctypes.c_void_p
U64, U32, I32 = ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
_lib.nwc_info.restype = I32; _lib.nwc_info.argtypes = [I32]
VERSION, NSTATE, TAB_WORDS, HDR_BLOCK = (_lib.nwc_info(i) for i in range(4))
FIXED_BLOCK = _lib.nwc_info(4)
ELEM = _lib.nwc_info(5) == 1
LAYOUT1 = _lib.nwc_info(6) == 1
LAYOUT2 = _lib.nwc_info(7) == 1
V9 = VERSION >= 9
X_FP32 = True                     # the reference ABI's layout-0 token path takes x as fp32
ELEM_BF16, ELEM_FP8 = 0, 1
ELEMS = {"bf16": ELEM_BF16, "fp8": ELEM_FP8}
LAYOUTS = {0, 1, 2}
LAYOUT_DEFAULT = {ELEM_BF16: 0, ELEM_FP8: 0}
if "NWC_LAYOUT" in os.environ:
    LAYOUT_DEFAULT = {k: int(os.environ["NWC_LAYOUT"]) for k in LAYOUT_DEFAULT}

_lib.nwc_layout.restype = I32; _lib.nwc_layout.argtypes = [U64, U32, I32, P]
_lib.nwc_encode.restype = ctypes.c_int64; _lib.nwc_encode.argtypes = [P, U64, U32, I32, P, P, P, P, P, U64, P]
_lib.nwc_build_tab.restype = None; _lib.nwc_build_tab.argtypes = [P, P, I32, P]
_lib.nwc_matvec.restype = I32; _lib.nwc_matvec.argtypes = [P, P, P, P, P, P, P, P, U64, U32, U32, I32]
_lib.nwc_dequant.restype = I32; _lib.nwc_dequant.argtypes = [P, P, P, P, P, P, P, U64, U32, U32, I32]
_lib.nwc_linear_bf16.restype = I32
_lib.nwc_linear_bf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, U64, U32, U32, I32]
_lib.nwc_linear_xbf16.restype = I32
_lib.nwc_linear_xbf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, P, U64, U32, I32]
_lib.nwc_dequant_seq.restype = I32
_lib.nwc_dequant_seq.argtypes = [P, P, P, P, P, P, P, P, P, U64, U32, I32]
_lib.nwc_seq_table.restype = I32
_lib.nwc_seq_table.argtypes = [P, I32, P]
_lib.nwc_row_index.restype = I32; _lib.nwc_row_index.argtypes = [P, P, P, P, P, P, P, U64, U32, I32]
_lib.nwc_token_split.restype = I32; _lib.nwc_token_split.argtypes = [U64, U32, I32, I32]
SEQ_TABLE = os.environ.get("NWC_SEQ_TABLE", "1") != "0"     # layout 0: the 13-bit token-path decode table
SEQ_TABLE_WORDS = 8196
ROW_INDEX = os.environ.get("NWC_ROW_INDEX", "1") != "0"   # layouts 0/1: build the row index for the token path
_lib.nwc_gather.restype = I32; _lib.nwc_gather.argtypes = [P, P, P, P, P, P, P, U32, P, U64, U32, U32, I32]
_lib.nwc_ref_fp8.restype = I32; _lib.nwc_ref_fp8.argtypes = [P, P, P, P, P, U64, U32]
_lib.nwc_setup.restype = I32; _lib.nwc_setup.argtypes = []


def _check_layout(layout):
    if layout not in LAYOUTS:
        raise ValueError(f"unknown layout {layout}")


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _need_gpu(t):
    if t.device.type != "cuda":
        raise RuntimeError("NWC kernels run on the GPU: move the NWCWeight to a cuda device")


FP8_MAX = 448.0


def quantize_fp8(w: torch.Tensor):
    """BF16/float [out, in] -> (fp8 e4m3fn tensor, fp32 scale[out]): symmetric absmax scale per output channel
    (nwc_torch.py:88-94)."""
    wf = w.detach().float()
    scale = wf.abs().amax(dim=1).clamp_min(1e-12) / FP8_MAX
    q = (wf / scale[:, None]).clamp(-FP8_MAX, FP8_MAX).to(torch.float8_e4m3fn)
    return q, scale


def ref_fp8_matvec(w8: torch.Tensor, scale: torch.Tensor, x_f32: torch.Tensor) -> torch.Tensor:
    """Uncompressed fp8 weight-only matvec in the library (the bandwidth baseline): y = scale * (W8 x), y BF16."""
    _need_gpu(w8)
    M, K = w8.shape
    y = torch.empty(M, dtype=torch.bfloat16, device=w8.device)
    xin = (x_f32 if x_f32.numel() % 16 == 0 else F.pad(x_f32, (0, 16 - x_f32.numel() % 16))).contiguous()
    err = _lib.nwc_ref_fp8(_stream(), _ptr(w8.view(torch.uint8)), _ptr(scale), _ptr(xin), _ptr(y), M, K)
    if err:
        raise RuntimeError(f"nwc_ref_fp8 HIP error {err}")
    return y


def fits(out_features, in_features):
    """Whether a matrix of this shape can be compressed (format v9+ pads any shape to its blocks)."""
    return in_features >= 1 and out_features >= 1


def choose_block(n):
    """The format's fixed block of 4096 weights."""
    return FIXED_BLOCK


def _layout_info(out_f, in_f, code):
    lay = torch.empty(4, dtype=torch.int64)
    if _lib.nwc_layout(out_f, in_f, code, _ptr(lay)):
        raise RuntimeError("nwc_layout")
    return lay.tolist()


def _check_streams(bases, hdr, data_len, layout, elem):
    """Structural check of stored tensors before the kernels read them: every block's lane streams (or exception
    lists) end inside `data` with the decoder's read-ahead slack."""
    if bases.numel() == 0:
        return
    h = hdr.to(torch.int64).view(-1, LANES).sum(1)
    esz = 4 if layout != 2 else (2 if elem == ELEM_FP8 else 3)
    end = bases.to(torch.int64) + h * esz + (64 if layout != 2 else 0)
    if int(bases.to(torch.int64).min()) < 0 or int(end.max()) > data_len:
        raise ValueError("compressed streams run past the data tensor: corrupt checkpoint")


class NWCWeight:
    """Compressed representation of an [out, in] matrix on the GPU.
    elem "bf16": the BF16 weights, lossless.  elem "fp8": weight-only fp8 e4m3 with a per-output-channel fp32 scale
    (from a BF16 matrix via quantize_fp8, or a float8 tensor plus `scale`), the fp8 values stored lossless."""

    def __init__(self, w: torch.Tensor, device="cuda", block=None, elem="bf16", scale=None, layout=None):
        assert w.dim() == 2
        out_f, in_f = w.shape
        assert fits(out_f, in_f), f"shape {tuple(w.shape)} not supported"
        self.elem = ELEMS[elem]
        self.layout = LAYOUT_DEFAULT[self.elem] if layout is None else int(layout)
        _check_layout(self.layout)
        if self.elem == ELEM_FP8:
            if w.dtype == torch.float8_e4m3fn:
                if scale is None:
                    raise ValueError("fp8 weights need their per-row scale")
                q = w
            else:
                q, scale = quantize_fp8(w)
            src = q.detach().contiguous().cpu().view(torch.uint8)
            self.scale = scale.detach().float().contiguous().to(device)
        else:
            assert w.dtype == torch.bfloat16, "BF16 expected (elem='fp8' for fp8 weights)"
            src = w.detach().contiguous().cpu().view(torch.int16)
            self.scale = None
        n = out_f * in_f
        block = block or choose_block(n)
        nb, n_low, n_scratch, self.K16 = _layout_info(out_f, in_f, self.code)
        freq = torch.empty(NPAIR, dtype=torch.int16)
        psym = torch.empty(NPAIR, dtype=torch.int16)
        bases = torch.empty(nb, dtype=torch.int32)
        hdr = torch.empty(nb * HDR_BLOCK, dtype=torch.uint8)
        low = torch.zeros(n_low + RAW_SLACK, dtype=torch.uint8)
        dl = -1
        for cap in (n + n // 2 + nb * 64 + 4096, 3 * n + nb * 64 + 4096):   # same capacity ladder as nwc_torch.py:163
            data = torch.empty(cap, dtype=torch.uint8)
            dl = _lib.nwc_encode(_ptr(src), n, in_f, self.code, _ptr(freq), _ptr(psym), _ptr(bases), _ptr(hdr),
                                 _ptr(data), cap, _ptr(low))
            if dl >= 0 or dl in (-2, -3):
                break
        if dl == -2:
            raise ValueError("fp8 weights contain NaN")
        if dl == -3:
            raise ValueError("layout 2 cannot code this matrix (a lane stream has more than 255 exceptions); use layout 0 or 1")
        if dl < 0:
            raise RuntimeError("nwc_encode failed")
        lut = torch.empty(TAB_WORDS, dtype=torch.int32)
        _lib.nwc_build_tab(_ptr(freq), _ptr(psym), self.code, _ptr(lut))
        self.out_features, self.in_features, self.n, self.block = out_f, in_f, n, block
        stored = torch.zeros(dl + 64, dtype=torch.uint8)            # the encoder writes data[0 .. dl); the rest is slack
        stored[:dl] = data[:dl]
        self.data = stored.to(device)
        self.bases = bases.to(device)
        self.hdr = hdr.to(device)
        self.lut = lut.to(device)
        self.low = low.to(device)
        self._finish(dl, n_low, n_scratch)

    @property
    def code(self):
        """elem parameter of the library: element type in bits 0..3, layout in bits 4..7."""
        return self.elem | (self.layout << 4)

    def _finish(self, dl, n_low, n_scratch):
        n = self.n
        self.bytes = (dl + self.bases.numel() * 4 + self.hdr.numel() + self.lut.numel() * 4 + n_low
                      + (self.scale.numel() * 4 if self.scale is not None else 0))
        self.bytes_bf16 = 2 * n
        self.bytes_native = n + self.out_features * 4 if self.elem == ELEM_FP8 else 2 * n
        self._n_scratch = n_scratch
        self._scratch = None

    @property
    def scratch(self):
        """fp32 [Mp * CB] scratch of the reference ABI; the gfx950 kernels reduce inside the workgroup and do not use
        it, so it is only allocated when asked for."""
        if self._scratch is None:
            self._scratch = torch.empty(self._n_scratch, dtype=torch.float32, device=self.data.device)
        return self._scratch

    @classmethod
    def from_tensors(cls, out_f, in_f, block, data, bases, hdr, lut, low, device="cuda", elem="bf16", scale=None, layout=0):
        """Compressed representation from stored tensors (nwc_amd.checkpoint), without the originals."""
        self = cls.__new__(cls)
        self.elem = ELEMS[elem]
        self.layout = int(layout)
        _check_layout(self.layout)
        n = out_f * in_f
        nb, n_low, n_scratch, self.K16 = _layout_info(out_f, in_f, self.code)
        if bases.numel() != nb or low.numel() not in (n_low, n_low + RAW_SLACK) or hdr.numel() != nb * HDR_BLOCK \
                or lut.numel() != TAB_WORDS:
            raise ValueError("checkpoint does not match this library version")
        _check_streams(bases.cpu(), hdr.cpu(), data.numel(), self.layout, self.elem)
        self.out_features, self.in_features, self.n, self.block = out_f, in_f, n, block
        if low.numel() == n_low:
            low = F.pad(low, (0, RAW_SLACK))
        self.data, self.bases, self.hdr, self.lut, self.low = (t.to(device) for t in (data, bases, hdr, lut, low))
        self.scale = None if scale is None else scale.float().to(device)
        self._finish(self.data.numel() - 64, n_low, n_scratch)
        self.bytes = (self.data.numel() + self.bases.numel() * 4 + self.hdr.numel() + self.lut.numel() * 4 + n_low
                      + (self.scale.numel() * 4 if self.scale is not None else 0))
        return self

    def tensors(self):
        """The tensors that fully describe the compressed state (for nwc_amd.checkpoint)."""
        t = {"data": self.data, "bases": self.bases, "hdr": self.hdr, "lut": self.lut, "low": self.low}
        if self.scale is not None:
            t["scale"] = self.scale
        return t

    def _x16(self, x):
        """Extend x to K16 (layout 0) or K rounded up to 32 (layouts 1/2) with zeros."""
        kp = (self.in_features + 31) // 32 * 32 if self.layout else self.K16
        return x if kp == self.in_features else F.pad(x, (0, kp - self.in_features))

    def matvec(self, x_f32: torch.Tensor) -> torch.Tensor:
        """fp32 test path: y = W x with fp32 output (times scale for fp8)."""
        _need_gpu(self.data)
        y = torch.empty(self.out_features, dtype=torch.float32, device=x_f32.device)
        xin = self._x16(x_f32.contiguous().float())
        err = _lib.nwc_matvec(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                              _ptr(self.low), _ptr(xin), _ptr(y), self.n, self.block, self.in_features, self.code)
        if err:
            raise RuntimeError(f"nwc_matvec HIP error {err}")
        return y if self.scale is None else y * self.scale

    def row_index(self):
        """Row index (uint16 [blocks x 3 x 32], built on the GPU on first use; not part of the format): each lane's bit
        position at rows 2, 4, 6 (layout 0) or super-chunks 4, 8, 12 (layout 1), so the token kernel can split a block
        over two or four half-waves.  None for layout 2, for layout-1 shapes whose index kernel has no single-round
        plan (K > 16384), or with NWC_ROW_INDEX=0."""
        if self.layout > 1 or not ROW_INDEX:
            return None
        ri = getattr(self, "_row_index", None)
        if ri is None:
            _need_gpu(self.data)
            ri = torch.empty(self.bases.numel() * 3 * LANES, dtype=torch.int16, device=self.data.device)
            err = _lib.nwc_row_index(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                                     _ptr(self.low), _ptr(ri), self.n, self.in_features, self.code)
            if err == -1 and self.layout == 1:
                ri = False                                         # no plan for this shape: decode without an index
            elif err:
                raise RuntimeError(f"nwc_row_index error {err}")
            self._row_index = ri
        return ri if ri is not False else None

    def seq_table(self):
        """The 13-bit token-path decode table of layouts 0/1 (int32 [8196] on the device, built on the host from the
        stored LUT on first use; not part of the format), or None for layout 2 or with NWC_SEQ_TABLE=0."""
        if self.layout > 1 or not SEQ_TABLE:
            return None
        st = getattr(self, "_seq_table", None)
        if st is None:
            host = torch.empty(SEQ_TABLE_WORDS, dtype=torch.int32)
            lut = self.lut.cpu().contiguous()                      # held: the library reads it through a raw pointer
            if _lib.nwc_seq_table(_ptr(lut), self.code, _ptr(host)):
                raise RuntimeError("nwc_seq_table failed")
            st = self._seq_table = host.to(self.data.device)
        return st

    def token_bytes(self):
        """Algorithmic bytes one token-path call reads: the compressed matrix, plus the row-index entries the kernel
        uses (64 bytes per block when it splits blocks over two half-waves, 192 over four) and the 13-bit table."""
        split = _lib.nwc_token_split(self.n, self.in_features, self.code, int(self.row_index() is not None))
        table = 4 * SEQ_TABLE_WORDS if self.seq_table() is not None else 0
        return self.bytes + self.bases.numel() * LANES * 2 * (split - 1) + table

    def linear_bf16(self, x: torch.Tensor, bias) -> torch.Tensor:
        """Token path: y = scale * (W x) + bias, x BF16 or fp32, y BF16."""
        _need_gpu(self.data)
        y = torch.empty(self.out_features, dtype=torch.bfloat16, device=x.device)
        bp = _ptr(bias) if bias is not None else None
        sp = _ptr(self.scale) if self.scale is not None else None
        if x.dtype == torch.bfloat16 or self.layout:
            xin = self._x16(x if x.dtype == torch.bfloat16 else x.to(torch.bfloat16)).contiguous()
            ri, st = self.row_index(), self.seq_table()
            err = _lib.nwc_linear_xbf16(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                                        _ptr(self.low), _ptr(ri) if ri is not None else None,
                                        _ptr(st) if st is not None else None, _ptr(xin), bp, sp, _ptr(y),
                                        self.n, self.in_features, self.code)
        else:                                                      # layout 0 with fp32 activations: the reference ABI
            xin = self._x16(x.float()).contiguous()
            err = _lib.nwc_linear_bf16(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                                       _ptr(self.low), _ptr(xin), bp, sp, None, _ptr(y), self.n, self.block,
                                       self.in_features, self.code)
        if err:
            raise RuntimeError(f"nwc_linear_bf16 HIP error {err}")
        return y

    def gather(self, ids: torch.Tensor) -> torch.Tensor:
        """Rows ids -> BF16[..., in_features] (embedding lookup straight from the compressed state)."""
        _need_gpu(self.data)
        flat = ids.reshape(-1).to(device=self.data.device, dtype=torch.int64).contiguous()
        out = torch.empty(flat.numel(), self.K16, dtype=torch.bfloat16, device=self.data.device)
        err = _lib.nwc_gather(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                              _ptr(self.low), _ptr(flat), flat.numel(), _ptr(out), self.n, self.block, self.in_features,
                              self.code)
        if err:
            raise RuntimeError(f"nwc_gather HIP error {err}")
        if self.K16 != self.in_features:
            out = out[:, :self.in_features].contiguous()
        return out.view(*ids.shape, self.in_features)

    def dequant(self, out: torch.Tensor = None) -> torch.Tensor:
        """The full matrix as BF16 (row-major); a view with row stride K16 if K is not a multiple of 16.
        fp8: the unscaled fp8 values (exact in BF16); multiply rows by `scale` for the weights.
        `out` may supply a preallocated BF16 [out_features, K16] buffer (prefill keeps one per shape)."""
        _need_gpu(self.data)
        w = out if out is not None else torch.empty((self.out_features, self.K16), dtype=torch.bfloat16, device=self.data.device)
        st = self.seq_table() if self.layout <= 1 else None
        if st is not None:
            ri = self.row_index() if self.layout <= 1 else None
            err = _lib.nwc_dequant_seq(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                                       _ptr(self.low), _ptr(ri) if ri is not None else None, _ptr(st), _ptr(w), self.n,
                                       self.in_features, self.code)
        else:
            err = _lib.nwc_dequant(_stream(), _ptr(self.data), _ptr(self.bases), _ptr(self.hdr), _ptr(self.lut),
                                   _ptr(self.low), _ptr(w), self.n, self.block, self.in_features, self.code)
        if err:
            raise RuntimeError(f"nwc_dequant HIP error {err}")
        return w if self.K16 == self.in_features else w[:, :self.in_features]

    def dequant_fp8(self):
        """fp8 weights: (float8_e4m3fn tensor [out, in], fp32 scale[out]), bit-exact with what was encoded."""
        if self.elem != ELEM_FP8:
            raise ValueError("not an fp8 matrix")
        return self.dequant().to(torch.float8_e4m3fn), self.scale


class RefFP8Linear(nn.Module):
    """Comparison only: weight-only fp8 without compression, served by the library's uncompressed fp8 matvec at batch 1
    and by dequantization + hipBLASLt otherwise (nwc_torch.py:272-290)."""

    def __init__(self, linear: nn.Linear, device="cuda"):
        super().__init__()
        q, scale = quantize_fp8(linear.weight.data)
        self.w8 = q.contiguous().to(device)
        self.scale = scale.to(device)
        self.in_features, self.out_features = linear.in_features, linear.out_features
        self.bias = None if linear.bias is None else nn.Parameter(
            linear.bias.data.to(device=device, dtype=torch.bfloat16), requires_grad=False)

    def forward(self, x):
        if x.numel() == self.in_features and x.dtype == torch.bfloat16:
            y = ref_fp8_matvec(self.w8, self.scale, x.reshape(-1).float())
            if self.bias is not None:
                y = y + self.bias
            return y.view(*x.shape[:-1], self.out_features)
        y = F.linear(x, self.w8.to(torch.bfloat16)).float() * self.scale
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype)


def convert_ref_fp8(model: nn.Module, device="cuda", verbose=True):
    """Replace every nn.Linear by RefFP8Linear (the uncompressed fp8 baseline); a tied lm_head stays BF16."""
    shared = {m.weight.data_ptr() for m in model.modules() if isinstance(m, nn.Embedding)}
    n = 0
    for name, mod in list(model.named_modules()):
        for child, cm in list(mod.named_children()):
            if isinstance(cm, nn.Linear) and cm.weight.dtype == torch.bfloat16 and cm.weight.data_ptr() not in shared:
                setattr(mod, child, RefFP8Linear(cm, device))
                cm.weight.data = torch.empty(0)
                n += 1
    model.to(device)
    if verbose:
        print(f"reference fp8: {n} linear layers replaced (uncompressed fp8, reference matvec)")
    return n


class NWCLinear(nn.Module):
    """Drop-in replacement for nn.Linear on a compressed matrix (elem "bf16" lossless, or "fp8" weight-only)."""

    def __init__(self, linear: nn.Linear = None, device="cuda", block=None, w: "NWCWeight" = None, bias=None, elem="bf16"):
        super().__init__()
        self.w = w if w is not None else NWCWeight(linear.weight.data, device, block, elem=elem)
        self.in_features, self.out_features = self.w.in_features, self.w.out_features
        if linear is not None and linear.bias is not None:
            bias = linear.bias.data
        self.bias = None if bias is None else nn.Parameter(bias.to(device=device, dtype=torch.bfloat16), requires_grad=False)

    def forward(self, x):
        if x.numel() == self.in_features and x.dtype == torch.bfloat16:   # one token -> fused kernel
            xf = x if x.is_contiguous() else x.contiguous()
            y = self.w.linear_bf16(xf.view(-1), None if self.bias is None else self.bias.data)
            return y.view(*x.shape[:-1], self.out_features)
        if self.w.scale is None:
            return F.linear(x, self.w.dequant(), self.bias)          # prefill -> temporary decompression + hipBLASLt
        y = F.linear(x, self.w.dequant()).float() * self.w.scale      # fp8: unscaled product, then the row scale
        if self.bias is not None:
            y = y + self.bias.float()
        return y.to(x.dtype)

    def extra_repr(self):
        return (f"in={self.in_features}, out={self.out_features}, elem={'fp8' if self.w.elem else 'bf16'}, layout={self.w.layout}, "
                f"{self.w.bytes/1e6:.1f} MB (BF16: {self.w.bytes_bf16/1e6:.1f} MB)")


class NWCEmbedding(nn.Module):
    """nn.Embedding replacement on a compressed matrix (shares the weight with a tied lm_head)."""

    def __init__(self, emb: nn.Embedding = None, w: NWCWeight = None, padding_idx=None):
        super().__init__()
        self.w = w
        self.num_embeddings, self.embedding_dim = w.out_features, w.in_features
        self.padding_idx = emb.padding_idx if emb is not None else padding_idx

    def forward(self, ids):
        rows = self.w.gather(ids)
        if self.w.scale is None:
            return rows
        return (rows.float() * self.w.scale[ids.to(self.w.scale.device)][..., None]).to(torch.bfloat16)

    def extra_repr(self):
        return f"{self.num_embeddings}, {self.embedding_dim}, {self.w.bytes/1e6:.1f} MB (BF16: {self.w.bytes_bf16/1e6:.1f} MB)"


class _FusedHead(nn.Module):
    """One output slice of a fused projection: head 0 computes the whole fused matvec, the others pick up their slice
    (nwc_torch.py:347-357)."""

    def __init__(self, shared, index, start, end):
        super().__init__()
        self.g, self.index, self.start, self.end = shared, index, start, end
        self.in_features, self.out_features = shared["lin"].in_features, end - start

    def forward(self, x):
        g = self.g
        if self.index == 0 or g["x_id"] != id(x) or g["y"] is None:
            g["y"] = g["lin"](x)
            g["x_id"] = id(x)
        return g["y"][..., self.start:self.end]


def fuse(model: nn.Module, groups=(("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj")), device="cuda", elem="bf16"):
    """Concatenate sibling nn.Linear layers with the same input into one NWC matrix (fewer, larger kernel launches).
    Call before `convert`; the fused layers are NWC afterwards.  Returns the number of fused groups."""
    n_fused = 0
    for mod in list(model.modules()):
        for names in groups:
            lins = [getattr(mod, nm, None) for nm in names]
            if not all(isinstance(l, nn.Linear) for l in lins):
                continue
            if len({l.in_features for l in lins}) != 1 or any(l.weight.dtype != torch.bfloat16 for l in lins):
                continue
            W = torch.cat([l.weight.data for l in lins], 0)
            if not fits(W.shape[0], W.shape[1]):
                continue
            b = None
            if all(l.bias is not None for l in lins):
                b = torch.cat([l.bias.data for l in lins], 0)
            elif any(l.bias is not None for l in lins):
                b = torch.cat([l.bias.data if l.bias is not None else torch.zeros(l.out_features, dtype=W.dtype) for l in lins], 0)
            whole = nn.Linear(W.shape[1], W.shape[0], bias=b is not None, dtype=torch.bfloat16)
            whole.weight.data = W
            if b is not None:
                whole.bias.data = b
            lin = NWCLinear(whole, device, elem=elem)
            shared = {"lin": lin, "y": None, "x_id": None, "names": list(names), "sizes": [l.out_features for l in lins]}
            a = 0
            for i, (nm, l) in enumerate(zip(names, lins)):
                setattr(mod, nm, _FusedHead(shared, i, a, a + l.out_features))
                a += l.out_features
                l.weight.data = torch.empty(0)
            n_fused += 1
    print(f"NWC: {n_fused} projection groups fused")
    return n_fused


def convert(model: nn.Module, device="cuda", verbose=True, tied=True, elem="bf16", embeddings=True):
    """Replace every supported nn.Linear (and a tied embedding) by NWC modules; move the rest to `device`.
    elem "bf16": lossless; "fp8": weight-only fp8 e4m3 (per-channel scale), the fp8 values stored lossless.
    embeddings: also compress untied nn.Embedding tables (always lossless BF16, looked up with the gather kernel).
    Returns (bytes_nwc, bytes_bf16) of the compressed matrices (nwc_torch.py:389-445)."""
    total_nwc = total_bf16 = 0
    replaced, skipped = 0, []
    shared_ptrs = {m.weight.data_ptr() for m in model.modules() if isinstance(m, nn.Embedding)}
    if tied:
        embs = {m.weight.data_ptr(): m for m in model.modules() if isinstance(m, nn.Embedding)
                and m.weight.dtype == torch.bfloat16 and fits(m.num_embeddings, m.embedding_dim)}
        lins = [(name, mod, child, cm) for name, mod in list(model.named_modules()) for child, cm in list(mod.named_children())
                if isinstance(cm, nn.Linear) and cm.weight.data_ptr() in embs]
        for name, mod, child, cm in lins:
            emb = embs[cm.weight.data_ptr()]
            w = NWCWeight(emb.weight.data, device, elem=elem)
            setattr(mod, child, NWCLinear(cm, device, w=w))
            for ename, emod in list(model.named_modules()):
                for echild, ecm in list(emod.named_children()):
                    if ecm is emb:
                        setattr(emod, echild, NWCEmbedding(emb, w))
            total_nwc += w.bytes
            total_bf16 += w.bytes_bf16
            replaced += 1
            shared_ptrs.discard(cm.weight.data_ptr())
            emb.weight.data = torch.empty(0)
            cm.weight.data = torch.empty(0)
    if embeddings:
        for name, mod in list(model.named_modules()):
            for child, cm in list(mod.named_children()):
                if isinstance(cm, nn.Embedding) and cm.weight.dtype == torch.bfloat16 and cm.weight.numel() \
                        and fits(cm.num_embeddings, cm.embedding_dim):
                    w = NWCWeight(cm.weight.data, device, elem="bf16")
                    setattr(mod, child, NWCEmbedding(cm, w))
                    total_nwc += w.bytes
                    total_bf16 += w.bytes_bf16
                    replaced += 1
                    cm.weight.data = torch.empty(0)
    for m in model.modules():
        if isinstance(m, _FusedHead) and m.index == 0:
            w = m.g["lin"].w
            total_nwc += w.bytes
            total_bf16 += w.bytes_bf16
            replaced += 1
    for name, mod in list(model.named_modules()):
        for child, cm in list(mod.named_children()):
            if isinstance(cm, nn.Linear) and cm.weight.dtype == torch.bfloat16 \
                    and fits(cm.out_features, cm.in_features) and cm.weight.data_ptr() not in shared_ptrs:
                new = NWCLinear(cm, device, elem=elem)
                setattr(mod, child, new)
                total_nwc += new.w.bytes
                total_bf16 += new.w.bytes_bf16
                replaced += 1
                cm.weight.data = torch.empty(0)
            elif isinstance(cm, nn.Linear):
                reason = "tied" if cm.weight.data_ptr() in shared_ptrs else "shape"
                skipped.append(f"{name}.{child} {tuple(cm.weight.shape)} [{reason}]")
    model.to(device)
    if verbose:
        print(f"NWC ({elem}): {replaced} linear layers replaced, {total_bf16/1e9:.2f} GB BF16 -> {total_nwc/1e9:.2f} GB "
              f"(ratio {total_nwc/max(total_bf16,1):.4f}" + (f", vs fp8 {total_nwc/max(total_bf16/2,1):.3f}" if elem == "fp8" else "") + ")")
        if skipped:
            print("  skipped:", ", ".join(skipped[:6]), "..." if len(skipped) > 6 else "")
    return total_nwc, total_bf16
