"""ctypes binding of libgrinnder_amd.so (the C ABI declared in include/grinnder_amd.h).

The library is loaded after torch so that it shares torch's HIP runtime.  A
missing library is a hard error: there is no Python or CPU fallback for any
entry point.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must be loaded first: provides the HIP runtime)

from grinnder_amd.build import source_hash

LIB_PATH = Path(__file__).resolve().parent / "libgrinnder_amd.so"

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_u64 = ctypes.c_uint64
_dbl = ctypes.c_double
_f32 = ctypes.c_float
_P = ctypes.c_void_p  # every pointer crosses as void*

# Activations of the LayerNorm epilogues (GR_ACT_* in include/grinnder_amd.h).
ACTIVATIONS = {"relu": 0, "elu": 1}

# name -> argument types (all return int status)
_SIGNATURES = {
    "gr_h2d_copy_async": [_P, _P, _i64, _P],
    "gr_d2h_copy_async": [_P, _P, _i64, _P],
    "gr_h2d_synchronize": [],
    "gr_d2h_synchronize": [],
    "gr_host_alloc": [_i64, _P],
    "gr_host_free": [_P],
    "gr_gather_partitions": [_i32, _i32, _P, _P, _P, _i64, _i64, _P, _P, _P],
    "gr_scatter_partitions": [_i32, _i32, _P, _i64, _i64, _P, _P, _P, _P, _P],
    "gr_build_subgraph": [_P, _P, _P, _i64, _i64, _P, _i64, _i32, _P, _P, _P, _P, _P, _P],
    "gr_partition_boundaries": [_i32, _i32, _P, _i64, _P, _i64, _P, _i64, _P, _P],
    "gr_partition_graph": [_P, _P, _i64, _i64, _i32, _dbl, _i32, _P, _P],
    "gr_csr_transpose": [_P, _P, _P, _i64, _i64, _P, _P, _P, _P],
    "gr_spmm_plan": [_P, _i64, _i32, _P, _P, _P, _P, _P],
    "gr_spmm_plan_blocked": [_P, _i64, _i32, _P, _i64, _P, _P, _P, _P, _P],
    "gr_gcn_aggregate": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _i64, _P, _i64, _i64, _P,
                         _i64, _P],
    "gr_gcn_aggregate_noalloc": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _i64, _P, _i64,
                                 _i64, _i64, _P],
    "gr_gcn_aggregate_into": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _i64, _i64, _i64,
                              _P, _i64, _P],
    "gr_gather_rows": [_P, _i64, _i64, _P, _i64, _i64, _P, _i64, _P],
    "gr_scatter_add_rows": [_P, _i64, _i64, _i64, _P, _P, _i64, _i64, _P],
    "gr_column_sum": [_P, _i64, _i64, _i64, _P, _P, _i64, _i64, _P, _P, _i64, _P],
    "gr_gcn_aggregate_ln_relu": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _P, _f32, _i64,
                                 _i64, _P, _P, _P, _P, _P, _i64, _P],
    "gr_ln_act_backward_product": [_P, _i64, _i64, _P, _P, _P, _P, _P, _P, _i32, _i64, _i64, _P,
                                   _P, _P, _P, _P, _P, _P, _i64, _P],
    "gr_ln_act_backward": [_P, _P, _P, _P, _P, _P, _i32, _i64, _i64, _P, _P, _P, _P, _P, _P,
                           _P, _i64, _P],
    "gr_bias_ln_act": [_P, _i64, _P, _P, _P, _f32, _i32, _i64, _i64, _P, _P, _P, _P, _P],
    "gr_gemm_tn_workspace": [_i64, _i64, _i64, _P, _P],
    "gr_linear_ln_act": [_P, _i64, _i64, _i64, _P, _i64, _P, _P, _P, _f32, _i32, _P, _P, _P, _P,
                         _P],
    "gr_xent_forward": [_P, _i64, _i64, _i64, _P, _P, _i32, _P, _P, _i64, _P, _P, _P, _i64, _P],
    "gr_gemm_tn": [_P, _i64, _P, _i64, _i64, _i64, _i64, _f32, _P, _P, _i64, _i64, _P],
    "gr_gemm_nt": [_P, _i64, _P, _i64, _i64, _i64, _i64, _P, _P, _i64, _P],
    "gr_gat_scores": [_P, _i64, _i64, _i64, _i64, _i64, _P, _P, _P, _P, _P],
    "gr_gat_row_dot": [_P, _i64, _P, _i64, _i64, _i64, _i64, _P, _P],
    "gr_gat_softmax_stats": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _P, _P, _i64, _P],
    "gr_gat_aggregate": [_P, _i64, _P, _i64, _P, _P, _i64, _P, _i64, _i64, _i64, _P, _P, _P,
                         _i64, _P, _i64, _P],
    "gr_gat_forward": [_P, _i64, _P, _i64, _P, _P, _i64, _P, _P, _i64, _i64, _i64, _P, _P, _P,
                       _P, _P, _P, _i64, _P, _i64, _i64, _P],
    "gr_gat_backward_src": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _P, _P, _P, _P,
                            _i64, _i64, _P, _P, _P, _P, _i64, _P],
    "gr_gat_backward_src_into": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _P, _P, _P, _P,
                                 _P, _i64, _i64, _P, _P, _P, _P, _i64, _P, _i64, _P, _P],
    "gr_gat_forward_ln": [_P, _i64, _P, _i64, _P, _P, _i64, _P, _P, _i64, _i64, _P, _P, _P,
                          _f32, _i32, _P, _P, _P, _P, _i64, _P, _P, _P, _i64,
                          _i64, _P],
    "gr_gat_dst_record": [_P, _P, _P, _P, _i64, _P, _P],
    "gr_gat_backward_src_h1": [_P, _i64, _P, _i64, _P, _P, _P, _i64, _P, _P, _P, _P, _P, _i64,
                               _P, _P, _P, _P, _i64, _P, _i64, _P, _P],
    "gr_gat_narrow_pack": [_P, _i64, _i64, _i64, _i64, _P, _P, _P, _P, _P, _P],
    "gr_gat_narrow_forward": [_P, _i64, _P, _i64, _P, _i64, _P, _P, _i64, _i64, _i64, _i64,
                              _P, _P, _P, _P, _P, _P, _P, _P, _i64, _P, _P, _P, _i64, _i64,
                              _P],
    "gr_gat_narrow_backward": [_P, _i64, _P, _i64, _P, _i64, _P, _P, _P, _i64, _i64, _i64,
                               _P, _i64, _P, _i64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _i64,
                               _i64, _P],
    "gr_gat_backward_dst": [_P, _i64, _P, _i64, _P, _P, _P, _P, _i64, _i64, _P, _P, _P, _i64,
                            _P],
    "gr_io_create": [_i32, _P],
    "gr_io_destroy": [_P],
    "gr_io_submit": [_P, _i32, ctypes.c_char_p, _P, _i64, _i64, _P],
    "gr_io_wait": [_P, _i64],
    "gr_io_wait_all": [_P],
    "gr_io_poll": [_P, _i64, _P],
    "gr_io_pending": [_P, _P],
    "gr_rmat_sample": [_u64, _i32, _dbl, _dbl, _dbl, _i64, _i64, _P, _P, _i32],
    "gr_gaussian_rows": [_u64, _P, _i64, _i64, _P, _i32],
}

EXPORTED = tuple(_SIGNATURES) + ("gr_last_error", "gr_abi_version", "gr_source_hash")

_lock = threading.Lock()
_lib = None


class GrError(RuntimeError):
    """Raised when a libgrinnder_amd entry point returns a non-zero status."""


def load():
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m grinnder_amd.build` "
                "(there is no fallback implementation)"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, args in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        lib.gr_last_error.argtypes = []
        lib.gr_last_error.restype = ctypes.c_char_p
        lib.gr_abi_version.argtypes = []
        lib.gr_abi_version.restype = ctypes.c_int
        lib.gr_source_hash.argtypes = []
        lib.gr_source_hash.restype = ctypes.c_char_p
        built = lib.gr_source_hash().decode()
        current = source_hash()
        if built != current:
            raise ImportError(
                f"{LIB_PATH} was built from other sources (hash {built[:12]}, the sources "
                f"here hash to {current[:12]}); rebuild it with `python -m grinnder_amd.build` "
                "in a fresh process")
        _lib = lib
    return _lib


def call(name: str, *args) -> None:
    """Calls entry point `name`; raises GrError with the library message on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.gr_last_error().decode(errors="replace")
        raise GrError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    """data_ptr of a tensor (None for None)."""
    if t is None:
        return None
    return t.data_ptr()


def stream_handle(stream=None) -> int | None:
    """Raw hipStream_t of a torch stream (the current stream by default)."""
    if stream is None:
        stream = torch.cuda.current_stream()
    return stream.cuda_stream


def ptr_array(values) -> ctypes.Array:
    """A C array of void* built from ints/None (kept alive by the caller)."""
    arr = (ctypes.c_void_p * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = v
    return arr


def i64_array(values) -> ctypes.Array:
    arr = (ctypes.c_int64 * max(1, len(values)))()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr
