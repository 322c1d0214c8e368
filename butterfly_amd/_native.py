"""ctypes binding of ``libbutterfly_amd.so`` (the C ABI in ``include/*.h``).

The library is built in-tree by ``butterfly_amd.build``.  There is no fallback:
if the library is missing every product entry point raises.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# BFLY_LIB names another build of the same library (a variant under test); the default is the
# in-tree build that butterfly_amd.build writes.
LIB_PATH = Path(os.environ.get("BFLY_LIB") or Path(__file__).resolve().parent / "_lib" / "libbutterfly_amd.so")

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3
ERR_CAPACITY = -4

DTYPE_F32 = 0
DTYPE_BF16 = 1

RULES = {
    "xor": 0,
    "bit_reversal": 1,
    "benes": 2,
    "causal_shift": 3,
    "fixed_stride": 4,
    "random": 5,
}

_i32, _i64, _f32, _vp = C.c_int32, C.c_int64, C.c_float, C.c_void_p

MAX_PARTNERS = 16


class Topology(C.Structure):
    """bfly_topology_t (include/butterfly_amd.h)."""

    _fields_ = [("rule", C.c_int32), ("width", C.c_int32), ("stage_idx", C.c_int32), ("stage_count", C.c_int32),
                ("local_window_blocks", C.c_int32), ("sink_count", C.c_int32), ("partner_count", C.c_int32),
                ("partner_bits", C.c_int32 * MAX_PARTNERS)]
_int = C.c_int
_pi32 = C.POINTER(C.c_int32)

# name -> (restype, argtypes); mirrors include/butterfly_amd.h
SIGNATURES = {
    "bfly_last_error": (C.c_char_p, []),
    "bfly_abi_version": (_int, []),
    "bfly_stage_meta": (_int, [_i64, _i64, _int, _pi32, _pi32, _pi32]),
    "bfly_partner_bits": (_int, [_int, _int, _int, _int, _int, _pi32]),
    "bfly_block_neighbors": (_int, [_i64, _i64, _int, _int, _int, _int, _vp, _int, _vp, _vp]),
    "bfly_prefill_tables": (_int, [_vp, _i64, _int, _int, _i64, _int, _vp, _vp, _vp, _vp, _vp]),
    "bfly_active_tables": (_int, [_vp, _i64, _int, _int, _i64, _int, _vp, _i64, _i64, _i64, _i64,
                                  _vp, _vp, _vp, _vp, _vp]),
    "bfly_block_mean": (_int, [_vp, _vp, _vp, _vp, _int, _i64, _i64, _int, _int, _i64, _vp]),
    "bfly_prefill": (_int, [_vp, _vp, _vp, _vp, _vp, _int, _i64, _int, _int, _i64, _int, _vp, _i64,
                            _int, _int, _int, _f32, _vp, _vp]),
    "bfly_swa_stream": (_int, [_vp, _vp, _vp, _int, _i64, _int, _int, _i64, _int, _int, _f32, _vp, _vp, _vp, _vp]),
    "bfly_compressed_stream": (_int, [_vp, _vp, _vp, _int, _i64, _int, _int, _i64, _int, _i64, _int, _vp, _i64,
                                      _int, _f32, _vp, _vp, _vp, _vp]),
    "bfly_softmax_merge": (_int, [_vp, _int, _vp, _vp, _vp, _int, _vp, _vp, _i64, _int, _vp, _vp]),
    "bfly_attend_cache": (_int, [_vp, _int, _i64, _int, _int, _i64, _int, _vp, _i64, _vp, _vp, _i64,
                                 _i64, _i64, _vp, _vp, _i64, _i64, _vp, _i64, _int, _int, _int, _f32,
                                 _vp, _vp]),
    "bfly_topology_init": (_int, [_i64, _i64, _int, _int, _int, _int, C.POINTER(Topology)]),
    "bfly_stream_chunks": (_int, [_i64, _vp, _vp, _vp, _vp, _vp, _int, _i64, _int, _int, _int, _vp, _vp, _i64, _vp,
                                  _vp, _i64, _vp, _int, _i64, _int, _int, _int, _int, _int, _int, _f32, _vp, _vp]),
    "bfly_decode": (_int, [_vp, _int, _i64, _int, _int, _int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp,
                           _i64, _i64, C.POINTER(Topology), _i64, _int, _int, _f32, _vp, _vp]),
    "bfly_decode_state_words": (_i64, [_i64, _int]),
    "bfly_decode_step": (_int, [_vp, _int, _i64, _int, _int, _int, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64, _vp,
                                _i64, _int, _int, _int, _int, _int, _int, _int, _f32, _vp, _vp]),
    "bfly_decode_step_qk_norm": (_int, [_vp, _int, _i64, _int, _int, _int, _vp, _vp, _vp, _vp, _i64, _vp, _vp, _i64,
                                        _vp, _i64, _int, _int, _int, _int, _int, _int, _int, _f32, _vp, _vp, _vp, _vp,
                                        _i64, _f32, _vp, _vp]),
    "bfly_decode_step_qk_norm_oproj": (_int, [_vp, _int, _i64, _int, _int, _int, _vp, _vp, _vp, _vp, _i64, _vp, _vp,
                                              _i64, _vp, _i64, _int, _int, _int, _int, _int, _int, _int, _f32, _vp,
                                              _vp, _vp, _vp, _i64, _f32, _vp, _vp, _i64, _int, _vp, _vp, _vp]),
    "bfly_cache_append": (_int, [_vp, _vp, _int, _i64, _int, _i64, _int, _vp, _vp, _i64, _i64, _vp]),
    "bfly_cache_compress": (_int, [_vp, _vp, _int, _i64, _int, _int, _i64, _i64, _i64, _int, _vp, _vp,
                                   _i64, _i64, _vp]),
    "bfly_cache_update": (_int, [_vp, _vp, _int, _i64, _int, _i64, _int, _vp, _vp, _i64, _i64, _i64, _i64, _int,
                                 _vp, _vp, _i64, _i64, _vp]),
    # include/butterfly_amd_decoder.h
    "bfly_add_rms_norm": (_int, [_vp, _vp, _vp, _i64, _int, _f32, _vp, _vp, _vp]),
    "bfly_qk_norm_rope": (_int, [_vp, _vp, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _i64, _i64, _int, _int, _int,
                                 _f32, _vp, _vp, _vp, _vp]),
    "bfly_silu_mul": (_int, [_vp, _vp, _i64, _i64, _i64, _vp, _vp]),
    "bfly_argmax_rows": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _i64, _vp, _vp]),
    "bfly_argmax_rows_noalloc": (_int, [_vp, _i64, _i64, _i64, _i64, _vp, _vp]),
    "bfly_q4_gemv": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _vp, _vp]),
    "bfly_q4_gemv_silu": (_int, [_vp, _vp, _vp, _i64, _i64, _int, _i64, _vp, _vp]),
    "bfly_add_rms_norm_q4_gemv": (_int, [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _int, _vp, _vp]),
    "bfly_add_rms_norm_q4_gemv_silu": (_int, [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _int, _i64, _vp,
                                              _vp]),
    "bfly_add_rms_norm_q4_gemv_silu_parts": (_int, [_vp, _int, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _int,
                                                    _i64, _vp, _vp]),
    "bfly_q4_argmax_workspace_bytes": (_i64, [_i64, _i64]),
    "bfly_add_rms_norm_q4_gemv_argmax": (_int, [_vp, _vp, _vp, _f32, _vp, _vp, _vp, _i64, _i64, _int, _vp, _vp,
                                                _i64, _vp]),
    "bfly_greedy_advance": (_int, [_vp, _i64, _vp, _i64, _i64, _vp, _vp, _vp, _i64, _vp, _vp]),
}

_lib = None
_fns = {}   # name -> bound foreign function, filled when the library loads


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load (once) and return the native library; raises if it is not built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} not found; build it with `python -m butterfly_amd.build`")
        handle = C.CDLL(os.fspath(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
            _fns[name] = fn
        _lib = handle
    return _lib


def check(rc: int, what: str = "") -> None:
    """Map a BFLY_ERR_* code to the reference's exception types."""
    if rc == OK:
        return
    msg = lib().bfly_last_error().decode(errors="replace")
    text = f"{what}: {msg}" if what else msg
    if rc == ERR_INVALID:
        raise ValueError(text)
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(text)
    raise RuntimeError(text)


def call(name: str, *args) -> None:
    fn = _fns.get(name)
    if fn is None:
        fn = getattr(lib(), name)
    rc = fn(*args)
    if rc:
        check(rc, name)
