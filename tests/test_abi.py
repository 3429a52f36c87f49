"""The C-ABI library (nwc_amd/lib/nwc_ops.so) loads and exports every symbol include/nwc_ops.h declares, and its
host entry points answer as the reference's do (nwc_ops.cu:100-126).  No device entry point is called here (CPU
suite); the GPU tests call them through the same ABI."""
import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nwc_ops.h")
REFERENCE_EXPORTS = {"nwc_info", "nwc_layout", "nwc_encode", "nwc_build_tab", "nwc_matvec", "nwc_dequant",
                     "nwc_linear_bf16", "nwc_gather", "nwc_ref_fp8", "nwc_setup"}      # nwc_ops.cu:27-39


def _declarations():
    """name -> number of parameters, for every function include/nwc_ops.h declares"""
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    out = {}
    for name, params in re.findall(r"^\s*(?:int|int64_t|uint64_t|void)\s+(nwc_\w+)\s*\(([^)]*)\)", text, flags=re.M):
        params = params.strip()
        out[name] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def _declared():
    return set(_declarations())


def _lib():
    from nwc_amd.nwc_torch import _LIB_PATH
    return ctypes.CDLL(_LIB_PATH)


def test_header_declares_the_reference_exports():
    d = _declared()
    assert REFERENCE_EXPORTS <= d
    assert d - REFERENCE_EXPORTS == {"nwc_linear_xbf16", "nwc_linear_xbf16_batch", "nwc_row_index", "nwc_token_split",
                                     "nwc_seq_table", "nwc_dequant_seq", "nwc_prefill_xbf16",
                                     "nwc_gather_xindex", "nwc_ref_bf16", "nwc_stream_read", "nwc_gemm_workspace",
                                     "nwc_gemm_xbf16", "nwc_gemm_xbf16_noalloc"}              # this build's additions


def test_binding_signatures_match_the_header():
    """The ctypes table (nwc_amd/_abi.py) declares every header function with the header's number of arguments."""
    from nwc_amd._abi import SIGNATURES
    decl = _declarations()
    assert set(SIGNATURES) == set(decl)
    for name, (_, args) in SIGNATURES.items():
        assert len(args) == decl[name], name


def test_library_exports_every_declared_symbol():
    lib = _lib()
    for name in sorted(_declared()):
        assert hasattr(lib, name), f"{name} missing from the library"


def test_info():
    lib = _lib()
    lib.nwc_info.restype = ctypes.c_int
    lib.nwc_info.argtypes = [ctypes.c_int]
    assert [lib.nwc_info(i) for i in range(8)] == [11, 1, 4096, 32, 4096, 1, 1, 1]
    assert lib.nwc_info(8) == -1 and lib.nwc_info(-1) == -1


@pytest.mark.parametrize("M,K,elem,expect", [
    (19456, 2560, 0x00, (12160, 19456 * 2560, 19456 * 5, 2560)),      # Qwen3-4B gate_up: nb, raw bytes, scratch, K16
    (2560, 9728, 0x00, (6080, 2560 * 9728, 2560 * 19, 9728)),
    (13, 40, 0x00, (2, 13 * 48, 16, 48)),                              # M * K16 raw bytes, Mp * CB
])
def test_layout_values(M, K, elem, expect):
    lib = _lib()
    lib.nwc_layout.restype = ctypes.c_int
    lib.nwc_layout.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
    out = np.zeros(4, np.uint64)
    assert lib.nwc_layout(M, K, elem, out.ctypes.data) == 0
    assert tuple(int(v) for v in out) == expect


def test_layout_matches_oracle():
    from oracle import oracle as O
    lib = _lib()
    lib.nwc_layout.restype = ctypes.c_int
    lib.nwc_layout.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
    out = np.zeros(4, np.uint64)
    for M, K in [(1, 1), (7, 513), (19456, 2560), (4608, 3584), (152064, 3584)]:
        for elem in (0, 1):
            for layout in (0, 1, 2):
                assert lib.nwc_layout(M, K, elem | layout << 4, out.ctypes.data) == 0
                assert tuple(int(v) for v in out) == tuple(O.layout_info(M, K, elem, layout))


def test_layout_rejects():
    lib = _lib()
    lib.nwc_layout.restype = ctypes.c_int
    lib.nwc_layout.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_void_p]
    out = np.zeros(4, np.uint64)
    assert lib.nwc_layout(0, 16, 0, out.ctypes.data) == -1
    assert lib.nwc_layout(16, 0, 0, out.ctypes.data) == -1
    assert lib.nwc_layout(1 << 32, 16, 0, out.ctypes.data) == -1


def _device_entry(lib):
    P, U64, U32, I = ctypes.c_void_p, ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int
    lib.nwc_linear_bf16.restype = I
    lib.nwc_linear_bf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, U64, U32, U32, I]
    lib.nwc_matvec.restype = I
    lib.nwc_matvec.argtypes = [P, P, P, P, P, P, P, P, U64, U32, U32, I]
    lib.nwc_linear_xbf16.restype = I
    lib.nwc_linear_xbf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, P, U64, U32, I]
    lib.nwc_linear_xbf16_batch.restype = I
    lib.nwc_linear_xbf16_batch.argtypes = [P, P, P, P, P, P, P, P, P, P, P, U64, U32, I, U32]
    lib.nwc_prefill_xbf16.restype = I
    lib.nwc_prefill_xbf16.argtypes = [P, P, P, P, P, P, P, P, P, P, P, P, U64, U32, I, U32]
    lib.nwc_gather_xindex.restype = I
    lib.nwc_gather_xindex.argtypes = [P, P, P, P, P, P, P, P, P, U32, P, U64, U32, I]
    return lib


@pytest.mark.parametrize("elem,ntok", [(0x10, 2), (0x20, 2), (0x00, 0), (0x00, 5), (0x01, 9)])
def test_batch_entry_point_refusals(elem, ntok):
    """nwc_linear_xbf16_batch takes layout 0 and 1..4 vectors; anything else gets -1 before any device call."""
    lib = _device_entry(_lib())
    assert lib.nwc_linear_xbf16_batch(None, *([None] * 10), 2560 * 4096, 4096, elem, ntok) == -1


@pytest.mark.parametrize("elem,index,table,ntok,want", [
    (0x10, 1, 1, 512, -1),      # layout 1
    (0x20, 1, 1, 512, -1),      # layout 2
    (0x00, 0, 1, 512, -1),      # no row index
    (0x00, 1, 0, 512, -1),      # no 13-bit table
    (0x00, 1, 1, 0, 0),         # no tokens: nothing to do
    (0x01, 1, 1, 65535 * 64 + 1, -1),
])
def test_prefill_entry_point_refusals(elem, index, table, ntok, want):
    """nwc_prefill_xbf16 answers these before any device call (dummy non-null pointers are never dereferenced)."""
    lib = _device_entry(_lib())
    dummy = ctypes.c_void_p(8)
    args = [None] * 6 + [dummy if index else None, dummy if table else None] + [None] * 4
    assert lib.nwc_prefill_xbf16(*args, 2560 * 4096, 4096, elem, ntok) == want


@pytest.mark.parametrize("elem,index,n_ids,want", [
    (0x10, 0, 4, -1),           # layout 1 without the row index
    (0x20, 1, 4, -1),           # layout 2
    (0x00, 0, 4, -1),           # no row index
    (0x00, 1, 0, 0),            # no ids: nothing to do
])
def test_gather_xindex_refusals(elem, index, n_ids, want):
    """nwc_gather_xindex answers these before any device call (a dummy non-null row index is never dereferenced)."""
    lib = _device_entry(_lib())
    args = [None] * 6 + [ctypes.c_void_p(8) if index else None, None, None]
    assert lib.nwc_gather_xindex(*args, n_ids, None, 2560 * 4096, 4096, elem) == want


@pytest.mark.parametrize("M,K,elem,ok", [
    ((1 << 20) - 1, 4096, 0x10, False),   # layout 1: M * K16 = 2^32 - 4096, but the plane padded to 16 rows is 2^32 B
    ((1 << 20) - 1, 4096, 0x20, False),   # layout 2: nibble + raw planes beyond 2^32 bytes
    ((1 << 20) - 1, 4096, 0x00, False),   # layout 0: rows padded to 8 reach 2^32 weights
    ((1 << 28), 16, 0x00, False),         # M * K16 = 2^32
    ((1 << 20) - 1, 4096, 0x11, True),    # layout 1 fp8: 8 bytes per lane and super-chunk, 2^31 bytes
    ((1 << 20) - 8, 4096, 0x00, True),    # layout 0 just below the bound
])
def test_device_entry_points_refuse_unaddressable_planes(M, K, elem, ok):
    """Shapes whose raw plane the kernels cannot address with 32-bit offsets get -1 from every device entry point
    before any device call (null pointers; no GPU needed).  Accepted shapes are probed only through nwc_token_split,
    which launches nothing."""
    from oracle import oracle as O
    lib = _device_entry(_lib())
    lib.nwc_token_split.restype = ctypes.c_int
    lib.nwc_token_split.argtypes = [ctypes.c_uint64, ctypes.c_uint32, ctypes.c_int, ctypes.c_int]
    n = M * K
    _, n_low, _, K16 = O.layout_info(M, K, elem & 15, elem >> 4)
    if elem >> 4:
        assert (n_low + 512 < (1 << 32)) == ok
    if ok:
        assert lib.nwc_token_split(n, K, elem, 0) != -1
        return
    assert lib.nwc_token_split(n, K, elem, 0) == -1
    assert lib.nwc_linear_bf16(None, *([None] * 10), n, 4096, K, elem) == -1
    assert lib.nwc_matvec(None, *([None] * 7), n, 4096, K, elem) == -1
    assert lib.nwc_linear_xbf16(None, *([None] * 11), n, K, elem) == -1
    assert lib.nwc_linear_xbf16_batch(None, *([None] * 10), n, K, elem, 2) == -1
    assert lib.nwc_prefill_xbf16(None, *([None] * 11), n, K, elem, 512) == -1
    assert lib.nwc_gather_xindex(None, *([None] * 8), 4, None, n, K, elem) == -1
