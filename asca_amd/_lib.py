"""ctypes binding of libasca_hip.so (the C ABI declared in include/asca_hip.h).

This is the Python-side counterpart of the reference's FFI module
rust/src/cuda/sys.rs: one declaration per exported symbol, and a status check
that turns a non-zero return into an exception carrying asca_last_error()
(rust/src/cuda/sys.rs:68-70 does the same with CUresult).

The library is loaded from the package directory only; when it is missing the
import of any GPU entry point fails loudly (there is no CPU fallback here).
"""
from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libasca_hip.so")

_i = C.c_int
_sz = C.c_size_t
_p = C.c_void_p
_fp = C.POINTER(C.c_float)
_u64p = C.POINTER(C.c_uint64)
_l = C.c_long
_f = C.c_float

# name -> (restype, argtypes).  Float tensors travel as void* device pointers.
SIGNATURES: dict[str, tuple] = {
    "asca_last_error": (C.c_char_p, []),
    "asca_init": (_i, [_i]),
    "asca_device_count": (_i, [C.POINTER(_i)]),
    "asca_describe": (_i, [C.c_char_p, _i]),
    "asca_alloc": (_i, [C.POINTER(_p), _sz]),
    "asca_free": (_i, [_p]),
    "asca_pool_release": (_i, []),
    "asca_h2d": (_i, [_p, _p, _sz]),
    "asca_d2h": (_i, [_p, _p, _sz]),
    "asca_d2d": (_i, [_p, _p, _sz, _p]),
    "asca_memset32": (_i, [_p, C.c_uint32, _sz, _p]),
    "asca_sync": (_i, []),
    "asca_stream_sync": (_i, [_p]),
    "asca_stats": (_i, [_u64p, _u64p, _u64p]),
    "asca_reset_stats": (_i, []),
    "asca_fail_after": (_i, [C.c_int64]),
    "asca_stream_create": (_i, [C.POINTER(_p)]),
    "asca_stream_destroy": (_i, [_p]),
    "asca_event_create": (_i, [C.POINTER(_p)]),
    "asca_event_destroy": (_i, [_p]),
    "asca_event_record": (_i, [_p, _p]),
    "asca_event_elapsed_ms": (_i, [C.POINTER(C.c_float), _p, _p]),
    "asca_selftest_wave": (_i, [_p]),
    "asca_copy_f32": (_i, [_p, _p, _sz, _p]),
    "asca_rng_seed": (None, [C.c_uint64, _u64p]),
    "asca_rng_u64": (None, [_u64p, _u64p, _sz]),
    "asca_rng_normal": (None, [_u64p, _p, _sz, C.c_float, C.c_float]),
    "asca_delta_ws_bytes": (_i, [_i, _i, _i, _i, C.POINTER(_sz)]),
    "asca_delta_fwd": (_i, [_p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "asca_delta_bwd_raw": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "asca_delta_bwd_fused": (_i, [_p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "asca_delta_states": (_i, [_p, _p, _p, _p, _p, _p, _i, _i, _i, _i, _p]),
    "asca_delta_decode_step": (_i, [_p, _p, _p, _p, _i, _i, _i, _p]),
    "asca_rmsnorm": (_i, [_p, _p, _p, _l, _i, _f, _p]),
    "asca_rmsnorm_bwd": (_i, [_p, _p, _p, _l, _i, _f, _p]),
    "asca_cross_entropy": (_i, [_p, _p, _l, _i, _p, _p, _p]),
    "asca_gather_rows": (_i, [_p, _p, _l, _i, _p, _p]),
    "asca_scatter_rows": (_i, [_p, _p, _l, _i, _p, _p]),
    "asca_colsum": (_i, [_p, _l, _i, _p, _i, _p]),
    "asca_colsum_ws_bytes": (_i, [_l, _i, C.POINTER(_sz)]),
    "asca_colsum_ws": (_i, [_p, _l, _i, _p, _i, _p, _sz, _p]),
    "asca_adamw_scalars": (_i, [_f, _f, _f, _f, _f, C.c_uint32, _fp]),
    "asca_adamw": (_i, [_p, _p, _p, _p, _l, _f, _f, _f, _f, _f, _p]),
    "asca_hash_route_ws_bytes": (_i, [_i, _i, C.POINTER(_sz)]),
    "asca_hash_route": (_i, [_p, _i, _i, _p, _p, _p, _p, _p]),
    "asca_bucket_keys": (_i, [_p, _i, _i, _p, _p, _p, _p, _p]),
    "asca_gemm": (_i, [_i, _i, _i, _i, _i, _f, _p, _l, _p, _l, _f, _p, _l, _p, _p]),
    "asca_gemm_ws_bytes": (_i, [_i, _i, _i, _i, _i, C.POINTER(_sz)]),
    "asca_gemm_noalloc": (_i, [_i, _i, _i, _i, _i, _f, _p, _l, _p, _l, _f, _p, _l, _p, _p]),
    "asca_gemm_ws": (_i, [_i, _i, _i, _i, _i, _f, _p, _l, _p, _l, _f, _p, _l, _p, _p, _sz, _p]),
    "asca_moe_fwd": (_i, [_p] * 7 + [_i] * 4 + [_p] * 4),
    "asca_moe_bwd": (_i, [_p] * 8 + [_i] * 4 + [_p] * 6 + [_i, _p]),
    "asca_chunk_ws_bytes": (_i, [_i, _i, _i, _i, _i, C.POINTER(_sz)]),
    "asca_chunk_fwd": (_i, [_p] * 7 + [_i] * 5 + [_p]),
    "asca_chunk_bwd": (_i, [_p] * 10 + [_i] * 5 + [_p]),
    "asca_chunk_ws_bytes_f32": (_i, [_i, _i, _i, _i, _i, C.POINTER(_sz)]),
    "asca_chunk_fwd_f32": (_i, [_p] * 7 + [_i] * 5 + [_p]),
    "asca_chunk_bwd_f32": (_i, [_p] * 7 + [_i] * 5 + [_p]),
    "asca_model_create": (_i, [_i] * 6 + [C.POINTER(_p)]),
    "asca_model_destroy": (_i, [_p]),
    "asca_model_num_tensors": (_i, [_p, C.POINTER(_i)]),
    "asca_model_tensor_info": (_i, [_p, _i, C.c_char_p, _i, C.POINTER(_sz), C.POINTER(_i), C.POINTER(_i)]),
    "asca_model_buffers": (_i, [_p, C.POINTER(_sz), C.POINTER(_p), C.POINTER(_p), C.POINTER(_p), C.POINTER(_p)]),
    "asca_model_set_adamw": (_i, [_p, _f, _f, _f, _f, _f, C.c_uint32]),
    "asca_model_adamw_step_count": (_i, [_p, C.POINTER(C.c_uint32)]),
    "asca_model_forward_backward": (_i, [_p, _p, _p, _i, _i, _p, _p]),
    "asca_model_adamw": (_i, [_p, _p]),
    "asca_model_train_step": (_i, [_p, _p, _p, _i, _i, _p, _p]),
    "asca_model_decode_state_floats": (_i, [_p, C.POINTER(_sz)]),
    "asca_model_decode_step": (_i, [_p, _p, _i, _p, _p, _p]),
}

ERRORS = {
    1: "invalid argument",
    2: "HIP error",
    3: "unsupported",
    4: "not initialised",
    5: "injected failure",
    6: "out of device memory",
    7: "no device",
    8: "optimiser step partially applied",
}


class AscaError(RuntimeError):
    """A libasca_hip entry point returned a non-zero status."""

    def __init__(self, code: int, func: str, msg: str):
        super().__init__(f"{func}: {ERRORS.get(code, 'error')} ({code}): {msg}")
        self.code = code
        self.func = func


_lock = threading.Lock()
_lib: C.CDLL | None = None


def load() -> C.CDLL:
    """Load libasca_hip.so from the package directory and declare its symbols."""
    global _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"{LIB_PATH} is missing: build it with `python -m asca_amd.build` "
                    "(no CPU fallback exists for the HIP path)"
                )
            lib = C.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
        return _lib


def call(name: str, *args) -> None:
    """Call an int-returning entry point and raise AscaError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.asca_last_error().decode(errors="replace")
        raise AscaError(rc, name, msg)
