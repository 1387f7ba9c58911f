"""ctypes binding of libdecide_hip.so (the C ABI in include/decide_hip.h).

The library is required: importing this module raises if it has not been
built (``python -c "import __graft_entry__ as g; g.build()"``). There is no
CPU fallback in this package; a caller that wants one does what the
reference's openDevice does (internal/train/engine.go:42-61) on NoGPUError.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
# DECIDE_HIP_LIBRARY names another build of the same library (the host-code
# sanitizer build the CPU tests load); the default is the in-tree build.
LIB_PATH = os.environ.get("DECIDE_HIP_LIBRARY") or os.path.join(HERE, "libdecide_hip.so")

DN_OK, DN_NO_GPU, DN_INVALID_ARG, DN_OUT_OF_MEMORY, DN_DEVICE_ERROR, DN_UNSUPPORTED = range(6)
DN_PRECISION_FP32, DN_PRECISION_BF16, DN_PRECISION_FP16 = 0, 1, 2
PRECISIONS = {"fp32": DN_PRECISION_FP32, "bf16": DN_PRECISION_BF16, "fp16": DN_PRECISION_FP16}
DN_STATE_WEIGHT, DN_STATE_GRAD, DN_STATE_M, DN_STATE_V = range(4)


class DecideError(RuntimeError):
    """A non-zero status from the library: (status, message)."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} [status {status}]")
        self.status = status
        self.message = message


class NoGPUError(DecideError):
    """DN_NO_GPU: the counterpart of the reference's cuda.ErrNoGPU (internal/cuda/driver.go:19)."""


class InvalidArgument(DecideError, ValueError):
    pass


class Unsupported(DecideError):
    pass


if not os.path.exists(LIB_PATH):
    raise ImportError(f"decide_amd: {LIB_PATH} is missing; build it with __graft_entry__.build()")

_c = ctypes
lib = _c.CDLL(LIB_PATH, mode=getattr(os, "RTLD_NOW", 2) | getattr(os, "RTLD_GLOBAL", 0x100))

_vp, _i, _i32p, _f32p, _f64p = _c.c_void_p, _c.c_int, _c.c_void_p, _c.c_void_p, _c.c_void_p

_SIGS = {
    "dn_abi_version": ([], _i),
    "dn_status_string": ([_i], _c.c_char_p),
    "dn_open": ([_i, _c.POINTER(_vp)], _i),
    "dn_close": ([_vp], None),
    "dn_last_error": ([_vp], _c.c_char_p),
    "dn_set_stream": ([_vp, _vp], _i),
    "dn_set_config": ([_vp, _i, _i, _i, _i, _i, _c.c_float, _i, _c.c_double, _c.c_double, _vp, _i], _i),
    "dn_upload_tensor": ([_vp, _c.c_char_p, _f32p, _c.c_int64], _i),
    "dn_upload_tensor_bf16": ([_vp, _c.c_char_p, _vp, _c.c_int64], _i),
    "dn_weights_ready": ([_vp], _i),
    "dn_forward": ([_vp, _i, _i32p, _i32p, _i32p, _i32p, _i32p, _i32p, _f32p, _i], _i),
    "dn_forward_device": ([_vp, _i, _i32p, _vp, _vp, _vp, _i, _vp, _vp], _i),
    "dn_forward_device_noalloc": ([_vp, _i, _i32p, _vp, _vp, _vp, _i, _vp, _vp], _i),
    "dn_check_device_errors": ([_vp], _i),
    "dn_gemm_f32": ([_vp, _i, _i, _i, _i, _i, _f32p, _i, _f32p, _i, _f32p, _i, _i], _i),
    "dn_gemm_device": ([_vp, _i, _i, _i, _i, _vp, _vp, _vp, _i], _i),
    "dn_gemm_device_store": ([_vp, _i, _i, _i, _i, _vp, _vp, _vp], _i),
    "dn_synchronize": ([_vp], _i),
    "dn_set_stream_split": ([_vp, _i], _i),
    "dn_set_row_tail": ([_vp, _i], _i),
    "dn_set_ln_fold": ([_vp, _i], _i),
    "dn_set_certify": ([_vp, _c.c_float], _i),
    "dn_set_small_m_loads": ([_vp, _i], _i),
    "dn_read_certify": ([_vp, _c.POINTER(_c.c_int64), _c.POINTER(_c.c_int64)], _i),
    "dn_set_probe": ([_vp, _i], _i),
    "dn_read_probe": ([_vp, _f64p, _c.POINTER(_i)], _i),
    "dn_read_probe_backward": ([_vp, _f64p, _c.POINTER(_i)], _i),
    "dn_mfma_calibrate": ([_vp, _i, _c.POINTER(_c.c_double)], _i),
    "dn_build_sequence": ([_i32p, _i, _c.c_int32, _i, _i32p, _i32p, _i32p, _c.POINTER(_i)], _i),
    "dn_answer": ([_f64p, _i, _c.c_double, _f64p, _c.POINTER(_i), _c.POINTER(_c.c_double)], _i),
    "dn_round": ([_c.c_double, _i], _c.c_double),
    "dn_evaluate": ([_vp, _i, _vp, _vp, _vp, _vp, _f64p, _c.c_int32, _i, _f64p, _vp, _f64p, _f64p], _i),
    "dn_enable_training": ([_vp], _i),
    "dn_set_trainable": ([_vp, _i, _i], _i),
    "dn_forward_train": ([_vp, _i, _i32p, _i32p, _i32p, _i32p, _i32p, _i32p, _f32p, _i], _i),
    "dn_backward": ([_vp, _f32p, _i], _i),
    "dn_zero_grad": ([_vp], _i),
    "dn_grad_sumsq": ([_vp, _c.POINTER(_c.c_double)], _i),
    "dn_adamw_step": ([_vp, _c.c_float, _c.c_float, _c.c_float, _c.c_float], _i),
    "dn_download_tensor": ([_vp, _c.c_char_p, _i, _f32p, _c.c_int64], _i),
    "dn_upload_state": ([_vp, _c.c_char_p, _i, _f32p, _c.c_int64], _i),
    "dn_set_adam_step": ([_vp, _i], _i),
    "dn_tokenizer_parse": ([_vp, _c.c_int64, _c.POINTER(_vp)], _i),
    "dn_tokenizer_free": ([_vp], None),
    "dn_tokenizer_special_ids": ([_vp, _vp, _vp, _vp, _vp], _i),
    "dn_tokenize": ([_vp, _vp, _c.c_int64, _i, _vp, _c.c_int64, _c.POINTER(_c.c_int64)], _i),
    "dn_pretokenize": ([_vp, _c.c_int64, _vp, _c.c_int64, _c.POINTER(_c.c_int64)], _i),
    "dn_nfc": ([_vp, _c.c_int64, _vp, _c.c_int64, _c.POINTER(_c.c_int64)], _i),
}
for _name, (_args, _res) in _SIGS.items():
    _fn = getattr(lib, _name)
    _fn.argtypes = _args
    _fn.restype = _res


def exported_symbols():
    return sorted(_SIGS)


def check(status: int, ctx=None) -> None:
    if status == DN_OK:
        return
    msg = lib.dn_last_error(ctx).decode(errors="replace")
    cls = {DN_NO_GPU: NoGPUError, DN_INVALID_ARG: InvalidArgument, DN_UNSUPPORTED: Unsupported}.get(status,
                                                                                                   DecideError)
    raise cls(status, msg)
