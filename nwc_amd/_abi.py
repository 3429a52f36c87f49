"""ctypes binding of the C-ABI library nwc_amd/lib/nwc_ops.so (declared in include/nwc_ops.h).

The library is located the way the reference bridge locates its own (parda21/NWC nwc/nwc_torch.py:14-22): the
NWC_DLL environment variable first, then the package's lib/ directory.  Signatures are declared from one table;
`call` runs an entry point and turns a non-zero return code into an exception.  Importing this module without the
built library raises ImportError: there is no CPU fallback for any compute entry point.
"""
import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))

# one letter per C type: p pointer, Q uint64_t, I uint32_t, i int, q int64_t, - void
_CTYPES = {"p": ctypes.c_void_p, "Q": ctypes.c_uint64, "I": ctypes.c_uint32, "i": ctypes.c_int,
           "q": ctypes.c_int64, "-": None}
# name: (return type, argument types), in include/nwc_ops.h order
SIGNATURES = {
    "nwc_info": ("i", "i"),
    "nwc_layout": ("i", "QIip"),
    "nwc_encode": ("q", "pQIipppppQp"),
    "nwc_build_tab": ("-", "ppip"),
    "nwc_matvec": ("i", "ppppppppQIIi"),
    "nwc_dequant": ("i", "pppppppQIIi"),
    "nwc_dequant_seq": ("i", "pppppppppQIi"),
    "nwc_linear_bf16": ("i", "pppppppppppQIIi"),
    "nwc_linear_xbf16": ("i", "ppppppppppppQIi"),
    "nwc_linear_xbf16_batch": ("i", "pppppppppppQIiI"),
    "nwc_prefill_xbf16": ("i", "ppppppppppppQIiI"),
    "nwc_gather_xindex": ("i", "pppppppppIpQIi"),
    "nwc_seq_table": ("i", "pip"),
    "nwc_row_index": ("i", "pppppppQIi"),
    "nwc_token_split": ("i", "QIii"),
    "nwc_gather": ("i", "pppppppIpQIIi"),
    "nwc_ref_fp8": ("i", "pppppQI"),
    "nwc_ref_bf16": ("i", "ppppQI"),
    "nwc_gemm_workspace": ("Q", "III"),
    "nwc_gemm_xbf16": ("i", "ppIpIppIIIpQ"),
    "nwc_gemm_xbf16_noalloc": ("i", "ppIpIppIII"),
    "nwc_stream_read": ("i", "ppQpI"),
    "nwc_setup": ("i", ""),
}


def library_path():
    env = os.environ.get("NWC_DLL")
    packaged = os.path.join(_HERE, "lib", "nwc_ops.so")
    for candidate in (env, packaged):
        if candidate and os.path.exists(candidate):
            return candidate
    tried = ", ".join(c for c in (env, packaged) if c)
    raise ImportError(f"NWC library not found ({tried}); build it with `python -m nwc_amd.build` (hipcc, gfx950)")


def _bind(path):
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = _CTYPES[res]
        fn.argtypes = [_CTYPES[a] for a in args]
    return lib


LIB_PATH = library_path()
lib = _bind(LIB_PATH)

# capabilities (nwc_info codes 0..7)
VERSION, NSTATE, TAB_WORDS, HDR_BLOCK, FIXED_BLOCK = (lib.nwc_info(i) for i in range(5))
HAS_ELEM, HAS_LAYOUT1, HAS_LAYOUT2 = (lib.nwc_info(i) == 1 for i in range(5, 8))


def ptr(t):
    """Device or host address of a tensor (None passes a null pointer)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream():
    """torch's current HIP stream as the ABI's void* stream argument."""
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def call(name, *args):
    """Run a device entry point; 0 is success, -1 a shape the library refuses, anything else a HIP error code.
    Both failures raise RuntimeError, as the reference bridge does for any non-zero return."""
    rc = getattr(lib, name)(*args)
    if rc == -1:
        raise RuntimeError(f"{name}: shape or element type not supported by the library")
    if rc:
        raise RuntimeError(f"{name}: HIP error {rc}")
    return rc
