"""ctypes binding of librfill.so (the C ABI declared in include/rfill.h).

The library is loaded on first use from this package directory. There is no fallback: if it is
missing or fails to load, every GPU entry point raises ImportError naming the build command.
Status codes become the exception types the reference raises for the same conditions
(ValueError for bad shapes / arguments, UnsupportedArchitecture for unimplemented model features).
"""
import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).with_name("librfill.so")

RF_OK, RF_EINVAL_SHAPE, RF_EINVAL_ARG, RF_EUNSUPPORTED, RF_EHIP = 0, -1, -2, -3, -4
SSQ_COLS = 256


class UnsupportedArchitecture(ValueError):
    """A model or model feature the kernels do not implement; refused by name, never approximated
    (code/kva/model.py:35-37)."""


class HipError(RuntimeError):
    """The HIP runtime reported an error for a kernel launch."""


_P, _I64, _I32, _F32, _F64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_double
_SZ, _PSZ = ctypes.c_size_t, ctypes.POINTER(ctypes.c_size_t)
_PP = ctypes.POINTER(ctypes.c_void_p)       # a host array of device pointers
_PI64 = ctypes.POINTER(ctypes.c_int64)      # a host array of counts

# name -> argument types (every function returns int status)
SIGNATURES = {
    "rf_map_apply": [_P, _I64, _P, _P, _P, _I64, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "rf_gemm_workspace_bytes": [_I64, _I64, _I64, _PSZ],
    "rf_rows_workspace_bytes": [_I64, _I64, _I64, _PSZ],
    "rf_map_apply_batch": [_I32, _P, _I64, _PP, _PP, _PP, _I64, _PP, _I64, _I64, _I64, _P],
    "rf_norm_kv_write_batch": [_I32, _PP, _I64, _PP, _I64, _I64, _F32, _PP, _I32, _I32, _PP, _I32, _P, _I32,
                               _PP, _PP, _I64, _I64, _I64, _I64, _P],
    "rf_row_ssq": [_P, _I64, _P, _I64, _I64, _P],
    "rf_row_scatter": [_P, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _P],
    "rf_fold_norm": [_P, _P, _I32, _P, _I64, _I64, _P],
    "rf_rope_table": [_P, _I64, _P, _I32, _P, _P],
    "rf_norm_kv_write": [_P, _I64, _P, _I64, _I64, _F32, _P, _I32, _I32, _P, _I32, _P, _I32,
                         _P, _P, _I64, _I64, _I64, _I64, _P, _SZ, _P],
    "rf_rope_kv_write": [_P, _I64, _P, _I64, _I64, _I32, _I32, _P, _I32, _P, _P, _I64, _I64, _I64, _I64, _P],
    "rf_norm_linear": [_P, _I64, _P, _I64, _I64, _F32, _P, _I64, _P, _I64, _P, _SZ, _P],
    "rf_norm_linear_batch": [_I32, _PP, _I64, _PP, _PI64, _I64, _F32, _PP, _PI64, _PP, _I64, _P],
    "rf_gdn_fill": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
    "rf_gdn_fill_batch": [_P, _I32, _I64, _I32, _I32, _I32, _I32, _P, _SZ, _P],
    "rf_gdn_workspace_bytes": [_I64, _I32, _I32, _I32, _I32, _PSZ],
    "rf_gdn_fill_noalloc": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P],
    "rf_transpose": [_P, _I64, _I64, _I64, _P, _I64, _P, _P],
    "rf_transpose_centred": [_P, _I64, _I64, _I64, _P, _P, _I64, _P, _I64, _P, _P, _P, _P],
    "rf_colsum_fold": [_P, _I64, _I64, _P, _P],
    "rf_gram_accumulate": [_P, _I64, _P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _SZ, _P],
    "rf_gram_workspace_bytes": [_I64, _I64, _I64, _I64, _PSZ],
    "rf_gram_accumulate_upper": [_P, _I64, _I64, _I64, _I64, _I64, _P, _I64, _P, _SZ, _P],
    "rf_gram_upper_workspace_bytes": [_I64, _I64, _I64, _I64, _PSZ],
    "rf_ridge_solve": [_P, _I64, _I64, _P, _I64, _I64, _P, _P, _P, _I32, _F64, _P, _I64, _I64, _P, _I64, _P, _SZ, _P],
    "rf_ridge_solve_workspace_bytes": [_I64, _I32, _PSZ],
    "rf_row_gather": [_P, _I64, _I64, _I64, _P, _I64, _P, _I64, _P, _P],
    "rf_norm_q": [_P, _I64, _P, _I64, _I64, _F32, _P, _I32, _I32, _P, _I32, _P, _I32, _P, _P, _I64, _P, _SZ, _P],
    "rf_norm_kv_rows": [_P, _I64, _P, _I64, _I64, _F32, _P, _I32, _I32, _P, _I32, _P, _I32, _P, _I64, _P, _P, _I64,
                        _I64, _P, _SZ, _P],
    "rf_mfma_ceiling": [_I32, _I32, _P, _P],
    "rf_map_apply_residual": [_P, _I64, _P, _P, _I64, _P, _I64, _P, _I64, _I64, _I64, _P, _SZ, _P],
    "rf_norm_linear_swiglu": [_P, _I64, _P, _I64, _I64, _F32, _P, _I64, _P, _I64, _P, _I64, _P, _SZ, _P],
    "rf_norm_qkv_rows": [_P, _I64, _P, _I64, _I64, _F32, _P, _I32, _I32, _I32, _P, _P, _I32, _P, _I32, _P, _I64, _P,
                         _I64, _P, _P, _I64, _I64, _P, _SZ, _P],
    "rf_attend_rows": [_P, _I64, _P, _I64, _I32, _I32, _P, _P, _I32, _I64, _I64, _I64, _F32, _P, _I64, _P, _SZ, _P],
    "rf_attend_rows_workspace_bytes": [_I64, _I32, _I32, _I32, _I64, _PSZ],
    "rf_attend_causal": [_P, _I64, _I64, _P, _I64, _I32, _I32, _P, _P, _I32, _I64, _I64, _I64, _F32, _P, _I64, _P,
                         _SZ, _P],
    "rf_attend_causal_workspace_bytes": [_I64, _I32, _I32, _I32, _I64, _PSZ],
    "rf_residual_add": [_P, _I64, _P, _I64, _P, _I64, _P, _I64, _I64, _P],
    "rf_silu_mul": [_P, _I64, _I64, _I64, _P, _I64, _P],
    "rf_gdn_forward_workspace_bytes": [_I64, _I32, _I32, _I32, _I32, _PSZ],
    "rf_gdn_forward": [_P, _I64, _I64, _I32, _I32, _I32, _I32, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _SZ, _P],
    "rf_sigmoid_mul": [_P, _I64, _P, _I64, _I64, _I64, _P, _I64, _P],
    "rf_gated_rms_norm": [_P, _I64, _P, _I64, _P, _I64, _I32, _I32, _F32, _P, _I64, _P],
    "rf_dequant_gguf_rows": [_I32, _P, _I64, _I64, _I64, _P, _I64, _P],
    "rf_dequant_i8_rows": [_P, _I64, _P, _I64, _I64, _I64, _I32, _P, _I64, _P],
    "rf_read_cosine": [_P, _I64, _P, _I64, _I64, _I32, _I32, _I32, _P, _I32, _F64, _P, _P, _SZ, _P],
    "rf_window_mass_workspace_bytes": [_I32, _I32, _I32, _I32, _I64, _PSZ],
    "rf_window_mass": [_P, _I64, _I32, _I64, _I32, _I32, _P, _I32, _I64, _I64, _F32, _P, _P, _SZ, _P],
}

_lib = None


def load():
    """The loaded library (loads it once). Raises ImportError if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is not built: run `make -C ridgefill-data_amd/csrc` "
                          f"(or __graft_entry__.build())")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.rf_last_error.restype = ctypes.c_char_p
    lib.rf_last_error.argtypes = []
    lib.rf_version.restype = ctypes.c_int
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = ctypes.c_int
        fn.argtypes = args
    _lib = lib
    return lib


def call(name, *args):
    """Call an entry point; raise the mapped exception on a non-zero status."""
    lib = load()
    status = getattr(lib, name)(*args)
    if status == RF_OK:
        return
    msg = lib.rf_last_error().decode(errors="replace")
    if status == RF_EUNSUPPORTED:
        raise UnsupportedArchitecture(msg)
    if status in (RF_EINVAL_SHAPE, RF_EINVAL_ARG):
        raise ValueError(msg)
    raise HipError(f"{msg} (status {status})")
