"""TEST INFRASTRUCTURE ONLY: numpy/ctypes front end of the C oracle (nwc_oracle.c).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module, and only as the
checker.  The product package (nwc_amd) never imports it.

Buffers follow the reference's Python bridge (nwc/nwc_torch.py:154-177): the same capacity ladder, the stored
`data` keeps dl + 64 bytes, `low` carries 512 bytes of slack.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")

LANES = 32
NPAIR = 1024
TAB_WORDS = 4096
RAW_SLACK = 512
ELEM_BF16, ELEM_FP8 = 0, 1


def build(quiet=True):
    """Compile liboracle.so with the Makefile beside this file."""
    out = subprocess.run(["make", "-C", HERE, "-s"], capture_output=True, text=True)
    if out.returncode:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout, end="")


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P, U64, U32, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
        L.or_layout.restype = I; L.or_layout.argtypes = [U64, U32, I, P]
        L.or_encode.restype = ctypes.c_int64; L.or_encode.argtypes = [P, U64, U32, I, P, P, P, P, P, U64, P]
        L.or_build_tab.restype = None; L.or_build_tab.argtypes = [P, I, P]
        L.or_decode.restype = I; L.or_decode.argtypes = [P, U64, P, P, P, P, U64, U32, I, P, I]
        L.or_matvec_f32.restype = None; L.or_matvec_f32.argtypes = [P, U64, U32, P, P, I]
        L.or_linear.restype = I; L.or_linear.argtypes = [P, U64, P, P, P, P, U64, U32, I, P, P, P, I]
        L.or_f32_to_e4m3.restype = ctypes.c_uint8; L.or_f32_to_e4m3.argtypes = [ctypes.c_float]
        L.or_e4m3_to_f32.restype = ctypes.c_float; L.or_e4m3_to_f32.argtypes = [ctypes.c_uint8]
        L.or_quantize_e4m3.restype = None; L.or_quantize_e4m3.argtypes = [P, U64, P, I]
        for fn in ("or_fp8_split", "or_fp8_split2"):
            getattr(L, fn).restype = I
            getattr(L, fn).argtypes = [ctypes.c_uint8, P, P]
        L.or_fp8_hb2.restype = ctypes.c_uint8; L.or_fp8_hb2.argtypes = [I]
        L.or_fp8_lb2.restype = ctypes.c_uint8; L.or_fp8_lb2.argtypes = [I]
        L.or_frag_row.restype = U32; L.or_frag_row.argtypes = [U32, U32]
        L.or_frag_col.restype = U32; L.or_frag_col.argtypes = [U32, U32]
        _lib = L
    return _lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


def code(elem, layout):
    return elem | (layout << 4)


def layout_info(M, K, elem, layout):
    out = np.zeros(4, dtype=np.uint64)
    rc = lib().or_layout(M, K, code(elem, layout), _p(out))
    if rc:
        raise ValueError("bad shape")
    return [int(v) for v in out]


def encode(w, elem=ELEM_BF16, layout=0, cap=None):
    """w: np.uint16 [M, K] (BF16 bits) or np.uint8 [M, K] (fp8 bytes).  Returns a dict of numpy arrays shaped like
    the reference's NWCWeight tensors plus `dl` (the encoder's return value) and `psym`."""
    M, K = w.shape
    n = M * K
    nb, n_low, n_scratch, K16 = layout_info(M, K, elem, layout)
    src = np.ascontiguousarray(w)
    freq = np.zeros(NPAIR, np.uint16)
    psym = np.zeros(NPAIR, np.uint16)
    bases = np.zeros(nb, np.uint32)
    hdr = np.zeros(nb * LANES, np.uint8)
    low = np.zeros(n_low + RAW_SLACK, np.uint8)
    caps = [cap] if cap else [n + n // 2 + nb * 64 + 4096, 3 * n + nb * 64 + 4096]
    dl = -1
    for c in caps:
        data = np.zeros(c, np.uint8)
        dl = lib().or_encode(_p(src), n, K, code(elem, layout), _p(freq), _p(psym), _p(bases), _p(hdr), _p(data), c, _p(low))
        if dl >= 0 or dl in (-2, -3):
            break
    if dl < 0:
        return {"dl": dl}
    lut = np.zeros(TAB_WORDS, np.uint32)
    lib().or_build_tab(_p(psym), code(elem, layout), _p(lut))
    stored = np.zeros(dl + 64, np.uint8)                          # data[0 .. dl) is written; the rest is slack
    stored[:dl] = data[:dl]
    return {"dl": dl, "data": stored, "bases": bases, "hdr": hdr, "lut": lut, "low": low, "psym": psym,
            "M": M, "K": K, "K16": K16, "nb": nb, "n_low": n_low, "n_scratch": n_scratch, "elem": elem, "layout": layout}


def decode(enc, threads=0):
    """BF16 bits [M, K] (fp8: the unscaled fp8 values as BF16); threads > 0 sets the OpenMP thread count."""
    M, K = enc["M"], enc["K"]
    out = np.zeros((M, K), np.uint16)
    rc = lib().or_decode(_p(enc["data"]), enc["data"].size, _p(enc["bases"]), _p(enc["hdr"]), _p(enc["lut"]),
                         _p(enc["low"]), M, K, code(enc["elem"], enc["layout"]), _p(out), threads)
    if rc:
        raise ValueError(f"oracle decode: malformed stream ({rc})")
    return out


def linear(enc, x, scale=None, threads=0):
    """End-to-end CPU decode + fp32 matvec (the CPU baseline)."""
    M, K = enc["M"], enc["K"]
    x = np.ascontiguousarray(x, np.float32)
    y = np.zeros(M, np.float32)
    sc = None if scale is None else np.ascontiguousarray(scale, np.float32)
    rc = lib().or_linear(_p(enc["data"]), enc["data"].size, _p(enc["bases"]), _p(enc["hdr"]), _p(enc["lut"]),
                         _p(enc["low"]), M, K, code(enc["elem"], enc["layout"]), _p(x), _p(sc), _p(y), threads)
    if rc:
        raise ValueError(f"oracle linear: malformed stream ({rc})")
    return y


def matvec_f32(w_bits, x, threads=0):
    M, K = w_bits.shape
    y = np.zeros(M, np.float32)
    lib().or_matvec_f32(_p(np.ascontiguousarray(w_bits)), M, K, _p(np.ascontiguousarray(x, np.float32)), _p(y), threads)
    return y


def bf16_to_f64(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def quantize_fp8(w_f32):
    """nwc_torch.py:88-94 restated: per-row scale = max(absmax, 1e-12) / 448 in fp32, then each weight
    q = RNE_e4m3(clamp(w / scale, -448, 448)) through or_f32_to_e4m3 (nearest of the 127 finite codes, ties to
    the even code).  Returns (uint8 codes [M, K], float32 scale [M])."""
    w = np.ascontiguousarray(w_f32, np.float32)
    scale = (np.maximum(np.abs(w).max(axis=1), np.float32(1e-12)) / np.float32(448.0)).astype(np.float32)
    v = np.ascontiguousarray(np.clip(w / scale[:, None], np.float32(-448.0), np.float32(448.0)), np.float32)
    q = np.zeros(v.shape, np.uint8)
    lib().or_quantize_e4m3(_p(v), v.size, _p(q), 0)
    return q, scale


def e4m3_to_f32(b):
    f = lib().or_e4m3_to_f32
    return np.array([f(int(t)) for t in np.asarray(b).ravel()], np.float32).reshape(np.asarray(b).shape)
