"""ctypes binding of libulm_fm.so, the HIP/CDNA4 fast-memory library.

The library is built in place by ``build.py`` (hipcc, gfx950). There is no
fallback: if the library is missing, loading raises, and every operator
requires its tensors on a ROCm device.
"""
import ctypes
import os

import torch

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libulm_fm.so")

ULM_OK, ULM_ERR_INVALID, ULM_ERR_UNSUPPORTED, ULM_ERR_LAUNCH = 0, 1, 2, 3
ULM_F32, ULM_BF16, ULM_F16 = 0, 1, 2
DTYPE_CODE = {torch.float32: ULM_F32, torch.bfloat16: ULM_BF16, torch.float16: ULM_F16}

P, I, SZ, F = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_float

# name -> (restype, argtypes); must match include/ulm_fm.h
SIGNATURES = {
    "ulm_abi_version": (I, []),
    "ulm_last_error": (ctypes.c_char_p, []),
    "ulm_fm_path": (I, [I, I, I, I]),
    "ulm_fm_saved_bytes": (SZ, [I, I, I, I, I]),
    "ulm_fm_saved_path": (I, [SZ, I, I, I, I, I]),
    "ulm_fm_fwd_workspace_bytes": (SZ, [I, I, I, I, I]),
    "ulm_fm_fwd": (I, [P, P, I, P, P, P, P, I, P, SZ, P, SZ, I, I, I, I, P]),
    "ulm_fm_prefill_path": (I, [I, I, I, I]),
    "ulm_fm_prefill_workspace_bytes": (SZ, [I, I, I, I, I, I]),
    "ulm_fm_prefill": (I, [P, P, I, P, P, P, P, I, P, P, P, SZ, I, I, I, I, P]),
    "ulm_fm_bwd_workspace_bytes": (SZ, [I, I, I, I, I, SZ, I]),
    "ulm_fm_bwd": (I, [P, P, P, P, SZ, I, P, I, P, P, P, I, P, P, P, SZ, I, I, I, I, P]),
    "ulm_la_workspace_bytes": (SZ, [I, I, I, I]),
    "ulm_la": (I, [P, P, P, P, P, I, I, I, I, I, I, P, SZ, P]),
    "ulm_addr_fwd": (I, [P, I, P, P, P, P, I, I, P]),
    "ulm_addr_bwd_workspace_bytes": (SZ, [I, I]),
    "ulm_addr_bwd": (I, [P, I, P, P, P, P, P, P, P, P, P, SZ, I, I, P]),
    "ulm_addr_bwd_noalloc": (I, [P, I, P, P, P, P, P, P, P, P, I, I, P]),
    "ulm_norm_conv_fwd": (I, [P, I, P, P, I, F, P, I, P, I, P, I, I, I, P]),
    "ulm_norm_conv_bwd_workspace_bytes": (SZ, [I, I, I, I]),
    "ulm_norm_conv_bwd": (I, [P, I, P, P, P, I, P, I, P, I, P, P, P, P, P, SZ, I, I, I, P]),
    "ulm_block_fm_fwd_workspace_bytes": (SZ, [I, I, I, I]),
    "ulm_block_fm_fwd": (I, [P, I, P, P, P, I, P, P, P, I, P, P, P, SZ, P, SZ, I, I, I, I, P]),
    "ulm_block_fm_bwd": (I, [P, I, P, P, P, P, P, SZ, I, P, I, P, I, P, P, I, P, P, P, SZ, I, I, I, I, P]),
    "ulm_cast": (I, [P, I, P, I, SZ, P]),
    "ulm_block_params": (I, [P, P, F, F, I, P, P, P]),
    "ulm_block_params_bwd": (I, [P, P, F, F, P, P, I, P, P, P]),
    "ulm_block_fm_prefill_workspace_bytes": (SZ, [I, I, I, I, I]),
    "ulm_block_fm_prefill": (I, [P, I, P, P, P, I, P, P, P, I, P, P, P, P, P, SZ, I, I, I, I, P]),
    "ulm_wgrad_workspace_bytes": (SZ, [I, I, I]),
    "ulm_wgrad": (I, [P, P, P, I, I, I, P, SZ, P]),
    "ulm_decode_pre": (I, [P, P, P, P, P, P, I, I, I, F, P]),
    "ulm_decode_addr": (I, [P, P, P, P, P, P, P, P, P, P, I, I, P]),
    "ulm_decode_state": (I, [P, P, P, P, P, P, P, P, I, I, I, P]),
    "ulm_decode_max_pending": (I, []),
    "ulm_decode_addr_deferred": (I, [P, P, P, P, P, P, P, P, P, P, P, I, P, I, I, P]),
    "ulm_decode_dots": (I, [P, P, P, I, I, I, P]),
    "ulm_decode_read": (I, [P, P, P, I, P, P, P, P, P, I, I, I, P]),
    "ulm_decode_flush": (I, [P, P, P, I, P, P, P, P, P, I, I, I, P]),
    "ulm_la_timer_start": (I, [I]),
    "ulm_la_timer_stop": (I, [ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]),
    "ulm_la_timer_product": (I, [I, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_int)]),
}

# the launch timer's block-pair product tags (ULM_PRODUCT_* of ulm_fm.h)
PRODUCTS = {"scores": 1, "apply": 2, "dscores": 3, "dv": 4, "dq_f": 5, "dk_f": 6, "state": 7}


class LaTimer:
    """Context manager: HIP-event time of every chunked-kernel launch inside it.
    After exit, ``total_ms`` and ``launches`` hold the sums, and ``products``
    maps each block-pair product that ran (PRODUCTS) to its (ms, launches)."""

    def __init__(self, max_launches=4096):
        self.max_launches = max_launches
        self.total_ms, self.launches = 0.0, 0
        self.products = {}

    def __enter__(self):
        call("ulm_la_timer_start", self.max_launches)
        return self

    def __exit__(self, *exc):
        ms, n = ctypes.c_double(), ctypes.c_int()
        call("ulm_la_timer_stop", ctypes.byref(ms), ctypes.byref(n))
        self.total_ms, self.launches = ms.value, n.value
        for name, tag in PRODUCTS.items():
            call("ulm_la_timer_product", tag, ctypes.byref(ms), ctypes.byref(n))
            if n.value:
                self.products[name] = (ms.value, n.value)
        return False

_lib = None


def lib():
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is missing: build it with `python unifiedlm.c_amd/build.py` "
                               "(the fast-memory operators have no CPU or PyTorch fallback)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def call(name, *args):
    """Calls an entry point and raises RuntimeError on a nonzero status."""
    status = getattr(lib(), name)(*args)
    if status != ULM_OK:
        msg = lib().ulm_last_error().decode(errors="replace")
        raise RuntimeError(f"{name} failed with status {status}: {msg}")


def ptr(t):
    """Device pointer of a tensor, or NULL for None."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(t):
    """The current stream of t's device, as the hipStream_t the entry points take
    (read without building a Python stream object where torch offers that)."""
    if _raw_stream is not None:
        return ctypes.c_void_p(_raw_stream(t.get_device()))
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_device(*tensors):
    """All tensors on one ROCm device; raises otherwise (no CPU fallback)."""
    dev = None
    for t in tensors:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise RuntimeError("the fast-memory operators run only on a ROCm GPU; got a tensor on "
                               f"{t.device}")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise RuntimeError(f"tensors on different devices: {dev} and {t.device}")
    return dev


def dtype_code(dtype):
    if dtype not in DTYPE_CODE:
        raise TypeError(f"unsupported dtype {dtype}; expected float32, bfloat16 or float16")
    return DTYPE_CODE[dtype]
