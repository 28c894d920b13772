"""ctypes binding of the C ABI in ``include/tf_hip.h`` (``lib/libtf_hip.so``).

There is no fallback: when the shared library is missing this module raises
at import, so nothing can silently run a CPU path in place of the kernels.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_DIR = Path(__file__).resolve().parent / "lib"
# TF_HIP_LIBRARY names another build of the same library (a kernel-variant
# build made by ``python -m tensors_amd.build --variant``, for A/B
# measurements); the default is the in-tree build.
HIP_LIB_PATH = Path(os.environ["TF_HIP_LIBRARY"]) if os.environ.get("TF_HIP_LIBRARY") else LIB_DIR / "libtf_hip.so"

TF_OK, TF_ERR_INVALID, TF_ERR_HIP, TF_ERR_UNSUPPORTED, TF_ERR_OOM = range(5)
TF_F32, TF_F16, TF_BF16, TF_I32, TF_I64, TF_BOOL = range(6)
TF_COPY_H2H, TF_COPY_H2D, TF_COPY_D2H, TF_COPY_D2D = range(4)
TF_EPI_NONE, TF_EPI_BIAS, TF_EPI_BIAS_RELU, TF_EPI_RELU, TF_EPI_ROW_BIAS, TF_EPI_ROW_BIAS_RELU = range(6)
TF_CE_CHAIN, TF_CE_STRICT, TF_CE_CLAMP, TF_CE_MODULE = range(4)


class TFError(RuntimeError):
    """A tf_* call returned a non-zero tf_status."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"tf_status {status}: {msg}")
        self.status = status


_p = C.c_void_p
_i64 = C.c_int64
_i = C.c_int
_f = C.c_float
_sz = C.c_size_t

# name -> argtypes (all return tf_status, except the two string getters).
SIGNATURES: dict[str, list] = {
    "tf_hip_device_count": [C.POINTER(_i)],
    "tf_hip_init": [_i, C.POINTER(_p)],
    "tf_hip_shutdown": [_p],
    "tf_hip_stream": [_p, C.POINTER(_p)],
    "tf_hip_set_stream": [_p, _p],
    "tf_hip_sync": [_p],
    "tf_hip_alloc": [_p, _sz, C.POINTER(_p)],
    "tf_hip_free": [_p, _p],
    "tf_hip_trim": [_p, _sz],
    "tf_hip_pool_stats": [_p, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)],
    "tf_hip_memcpy": [_p, _p, _p, _sz, _i],
    "tf_hip_fill_f32": [_p, _p, _f, _i64],
    "tf_hip_zero": [_p, _p, _sz],
    "tf_hip_event_create": [_p, C.POINTER(_p)],
    "tf_hip_event_record": [_p, _p],
    "tf_hip_event_elapsed": [_p, _p, C.POINTER(_f)],
    "tf_hip_event_destroy": [_p],
    "tf_gemm": [_p, _i, _i, _i64, _i64, _i64, _f, _p, _i64, _p, _i64, _f, _p, _i64, _i, _i, _i, _p],
    "tf_hip_timing_start": [_i],
    "tf_hip_timing_stop": [_p],
    "tf_hip_timing_record": [_i, _p, _p, _p],
    "tf_gemm_noalloc": [_p, _i, _i, _i64, _i64, _i64, _f, _p, _i64, _p, _i64, _f, _p, _i64, _i, _i, _i, _p],
    "tf_gemm_strided_batched": [_p, _i, _i, _i64, _i64, _i64, _f, _p, _i64, _i64, _p, _i64, _i64,
                                _f, _p, _i64, _i64, _i64, _i, _i],
    "tf_gemm_ex": [_p, _i, _i, _i64, _i64, _i64, _f, _p, _i64, _i64, _p, _i64, _i64, _f, _p, _i64, _i64,
                   _i64, _i, _i, _i, _i, _p],
    "tf_layernorm_fwd": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _f],
    "tf_layernorm_bwd": [_p, _p, _p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i],
    "tf_im2col": [_p, _p, _p] + [_i64] * 12 + [_i],
    "tf_conv2d_fwd": [_p, _p, _p, _p, _p] + [_i64] * 13 + [_i],
    "tf_conv2d_bwd_weight": [_p, _p, _p, _p, _p] + [_i64] * 13,
    "tf_conv2d_bwd_data": [_p, _p, _p, _p] + [_i64] * 13,
    "tf_conv2d_bwd_weight_relu": [_p, _p, _p, _p, _p, _p, _p] + [_i64] * 13,
    "tf_decode_u8": [_p, _p, _p, _i64, _i64, _i, _p],
    "tf_col2im": [_p, _p, _p] + [_i64] * 14 + [_i],
    "tf_add": [_p, _p, _p, _p, _i64, _i],
    "tf_sub": [_p, _p, _p, _p, _i64, _i],
    "tf_sum_dim": [_p, _p, _p, _i64, _i64, _i64],
    "tf_expand_dim": [_p, _p, _p, _i64, _i64, _i64],
    "tf_transpose2d": [_p, _p, _p, _i64, _i64, _i64, _i],
    "tf_mul": [_p, _p, _p, _p, _i64, _i],
    "tf_scale_by": [_p, _p, _p, _p, _i64, _i],
    "tf_relu_fwd": [_p, _p, _p, _i64, _i],
    "tf_sigmoid_fwd": [_p, _p, _p, _i64, _i],
    "tf_tanh_fwd": [_p, _p, _p, _i64, _i],
    "tf_relu_bwd": [_p, _p, _p, _p, _i64, _i],
    "tf_sigmoid_bwd": [_p, _p, _p, _p, _i64, _i],
    "tf_tanh_bwd": [_p, _p, _p, _p, _i64, _i],
    "tf_ce_fwd": [_p, _p, _p, _p, _p, _i64, _i64, _i],
    "tf_ce_bwd": [_p, _p, _p, _p, _p, _p, _i64, _i64],
    "tf_ce_fwd_bwd": [_p, _p, _p, _p, _p, _i64, _i64, _i],
    "tf_ce_fwd_bwd_bf16": [_p, _p, _p, _p, _p, _i64, _i64, _i],
    "tf_log_softmax_fwd": [_p, _p, _p, _i64, _i64],
    "tf_softmax_fwd": [_p, _p, _p, _i64, _i64],
    "tf_argmax_rows": [_p, _p, _p, _p, _p, _i64, _i64],
    "tf_leaky_relu_fwd": [_p, _p, _p, _i64, _f, _i],
    "tf_log_softmax_bwd": [_p, _p, _p, _p, _i64, _i64],
    "tf_softmax_bwd": [_p, _p, _p, _p, _i64, _i64],
    "tf_colsum": [_p, _p, _p, _i64, _i64],
    "tf_colsum_bf16": [_p, _p, _p, _i64, _i64],
    "tf_relu_bwd_colsum": [_p, _p, _p, _p, _p, _i64, _i64, _i],
    "tf_linear_bwd_narrow": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64],
    "tf_gemm_relu_masked": [_p, _i, _i, _i64, _i64, _i64, _p, _i64, _p, _p, _i64, _p, _i64],
    "tf_linear_bwd_small": [_p, _p, _p, _p, _p, _p, _p, _i64, _i64, _i64],
    "tf_chansum_nchw": [_p, _p, _p, _i64, _i64, _i64],
    "tf_sgd_momentum": [_p, _p, _p, _p, _p, _i64, _f, _f],
    "tf_sgd_momentum_multi": [_p, _i, _p, _p, _p, _p, _p, _f, _f],
    "tf_cast_f32_bf16": [_p, _p, _p, _i64],
    "tf_graph_begin": [_p],
    "tf_graph_end": [_p, _p],
    "tf_graph_launch": [_p, _p],
    "tf_graph_destroy": [_p],
    "tf_gather_indexed": [_p, _p, _p, _i64, _p, _i64],
    "tf_record_step": [_p, _p, _p, _i64, _p],
    "tf_cast_bf16_f32": [_p, _p, _p, _i64],
}


def _load() -> C.CDLL:
    if not HIP_LIB_PATH.exists():
        raise ImportError(
            f"{HIP_LIB_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(the HIP path has no CPU fallback)")
    lib = C.CDLL(str(HIP_LIB_PATH), mode=os.RTLD_NOW | os.RTLD_GLOBAL)
    lib.tf_last_error.restype = C.c_char_p
    lib.tf_last_error.argtypes = []
    lib.tf_version.restype = C.c_char_p
    lib.tf_version.argtypes = []
    for name, args in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = C.c_int
    return lib


lib = _load()


def check(status: int) -> None:
    if status != TF_OK:
        raise TFError(status, lib.tf_last_error().decode(errors="replace"))


def call(name: str, *args) -> None:
    """Call tf_<name> and raise TFError on a non-zero status."""
    check(getattr(lib, name)(*args))


def device_count() -> int:
    n = C.c_int(0)
    check(lib.tf_hip_device_count(C.byref(n)))
    return n.value
