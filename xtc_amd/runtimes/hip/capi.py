# SPDX-License-Identifier: BSD-3-Clause
"""ctypes binding of libxtc_hip.so (declared in include/xtc_hip.h).

This is the only place the Python side touches the native library.  Loading
fails loudly when the library has not been built: there is no CPU fallback
for any operator.
"""

from __future__ import annotations

import ctypes
import os
import threading
from pathlib import Path
from typing import Any

__all__ = [
    "LIB_PATH",
    "HipError",
    "XTC_HIP_F32",
    "XTC_HIP_BF16",
    "XTC_HIP_F64",
    "Tile",
    "MatmulDesc",
    "Conv2dDesc",
    "GemmInstance",
    "lib",
    "check",
    "library_available",
]

LIB_PATH = Path(__file__).resolve().parents[2] / "lib" / "libxtc_hip.so"
INCLUDE_PATH = Path(__file__).resolve().parents[3] / "include"

XTC_HIP_F32 = 0
XTC_HIP_BF16 = 1
XTC_HIP_F64 = 2


class HipError(RuntimeError):
    """A libxtc_hip call returned a non-zero status."""


class Tile(ctypes.Structure):
    _fields_ = [
        ("bm", ctypes.c_int),
        ("bn", ctypes.c_int),
        ("bk", ctypes.c_int),
        ("wgm", ctypes.c_int),
        ("wgn", ctypes.c_int),
    ]

    def as_tuple(self) -> tuple[int, int, int, int, int]:
        return (self.bm, self.bn, self.bk, self.wgm, self.wgn)


class MatmulDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("M", ctypes.c_int),
        ("N", ctypes.c_int),
        ("K", ctypes.c_int),
        ("lda", ctypes.c_int),
        ("ldb", ctypes.c_int),
        ("ldc", ctypes.c_int),
        ("tile", Tile),
        ("split_k", ctypes.c_int),
        ("group_m", ctypes.c_int),
        ("xcd_remap", ctypes.c_int),
        ("relu", ctypes.c_int),
        ("relu_threshold", ctypes.c_float),
        ("stream", ctypes.c_void_p),
        ("trans_a", ctypes.c_int),
        ("trans_b", ctypes.c_int),
        ("stages", ctypes.c_int),
        ("relu_threshold_f64", ctypes.c_double),
    ]


class Conv2dDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("N", ctypes.c_int),
        ("H", ctypes.c_int),
        ("W", ctypes.c_int),
        ("C", ctypes.c_int),
        ("F", ctypes.c_int),
        ("R", ctypes.c_int),
        ("S", ctypes.c_int),
        ("stride_h", ctypes.c_int),
        ("stride_w", ctypes.c_int),
        ("pad_top", ctypes.c_int),
        ("pad_bottom", ctypes.c_int),
        ("pad_left", ctypes.c_int),
        ("pad_right", ctypes.c_int),
        ("pad_value", ctypes.c_float),
        ("tile", Tile),
        ("split_k", ctypes.c_int),
        ("group_m", ctypes.c_int),
        ("xcd_remap", ctypes.c_int),
        ("relu", ctypes.c_int),
        ("relu_threshold", ctypes.c_float),
        ("stream", ctypes.c_void_p),
        ("relu_threshold_f64", ctypes.c_double),
        ("pad_value_f64", ctypes.c_double),
    ]


class GemmInstance(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int),
        ("conv", ctypes.c_int),
        ("tile", Tile),
        ("lds_bytes", ctypes.c_int),
        ("threads", ctypes.c_int),
    ]


_vp = ctypes.c_void_p
_i = ctypes.c_int
_u64 = ctypes.c_uint64
_f = ctypes.c_float

# name -> (restype, argtypes); exactly the declarations of include/xtc_hip.h
SIGNATURES: dict[str, tuple[Any, list[Any]]] = {
    "xtc_hip_last_error": (ctypes.c_char_p, []),
    "xtc_hip_device_count": (_i, []),
    "xtc_hip_init": (_i, [_i]),
    "xtc_hip_device_arch": (_i, [ctypes.c_char_p, _i]),
    "xtc_hip_device_name": (_i, [ctypes.c_char_p, _i]),
    "xtc_hip_stream": (_vp, []),
    "xtc_hip_synchronize": (_i, []),
    "xtc_hip_stream_create": (_vp, []),
    "xtc_hip_stream_synchronize": (_i, [_vp]),
    "xtc_hip_stream_destroy": (_i, [_vp]),
    "xtc_hip_stream_release": (_i, [_vp]),
    "xtc_hip_malloc": (_vp, [_u64]),
    "xtc_hip_free": (_i, [_vp]),
    "xtc_hip_memcpy_h2d": (_i, [_vp, _vp, _u64]),
    "xtc_hip_memcpy_d2h": (_i, [_vp, _vp, _u64]),
    "xtc_hip_memcpy_d2d": (_i, [_vp, _vp, _u64]),
    "xtc_hip_memset_zero": (_i, [_vp, _u64]),
    "xtc_hip_event_create": (_vp, []),
    "xtc_hip_event_record": (_i, [_vp, _vp]),
    "xtc_hip_event_elapsed_ms": (_i, [_vp, _vp, ctypes.POINTER(_f)]),
    "xtc_hip_event_destroy": (_i, [_vp]),
    "xtc_hip_matmul": (_i, [ctypes.POINTER(MatmulDesc), _vp, _vp, _vp, _vp]),
    "xtc_hip_matmul_noalloc": (_i, [ctypes.POINTER(MatmulDesc), _vp, _vp, _vp, _vp]),
    "xtc_hip_conv2d": (_i, [ctypes.POINTER(Conv2dDesc), _vp, _vp, _vp, _vp]),
    "xtc_hip_relu": (_i, [_vp, _vp, _u64, _f, _vp]),
    "xtc_hip_pad": (
        _i,
        [
            _vp,
            _vp,
            _i,
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            _f,
            _vp,
        ],
    ),
    "xtc_hip_relu_f64": (_i, [_vp, _vp, _u64, ctypes.c_double, _vp]),
    "xtc_hip_pad_f64": (
        _i,
        [
            _vp,
            _vp,
            _i,
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            ctypes.c_double,
            _vp,
        ],
    ),
    "xtc_hip_unpad": (
        _i,
        [
            _vp,
            _vp,
            _i,
            _i,
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            ctypes.POINTER(ctypes.c_int64),
            _vp,
        ],
    ),
    "xtc_hip_cast_f32_to_bf16": (_i, [_vp, _vp, _u64, _vp]),
    "xtc_hip_cast_bf16_to_f32": (_i, [_vp, _vp, _u64, _vp]),
    "xtc_hip_matmul_desc_size": (_i, []),
    "xtc_hip_conv2d_desc_size": (_i, []),
    "xtc_hip_gemm_instance_count": (_i, []),
    "xtc_hip_gemm_instance_get": (_i, [_i, ctypes.POINTER(GemmInstance)]),
    "xtc_hip_default_tile": (
        _i,
        [_i, _i, _i, _i, _i, ctypes.POINTER(Tile), ctypes.POINTER(_i)],
    ),
    "xtc_hip_conv2d_default_tile": (_i, [ctypes.POINTER(Conv2dDesc), ctypes.POINTER(Tile), ctypes.POINTER(_i)]),
    "xtc_hip_matmul_pipeline_depths": (_i, [ctypes.POINTER(MatmulDesc), ctypes.POINTER(_i), _i]),
    "xtc_hip_conv2d_pipeline_depths": (_i, [ctypes.POINTER(Conv2dDesc), ctypes.POINTER(_i), _i]),
    "xtc_hip_evaluate_perf": (
        None,
        [
            ctypes.POINTER(ctypes.c_double),
            _i,
            ctypes.POINTER(ctypes.c_char_p),
            _i,
            _i,
            _i,
            _vp,
            ctypes.POINTER(_vp),
            _i,
        ],
    ),
    "xtc_hip_evaluate": (
        None,
        [ctypes.POINTER(ctypes.c_double), _i, _i, _i, _vp, ctypes.POINTER(_vp), _i],
    ),
    "xtc_hip_evaluate_status": (_i, []),
    "xtc_hip_evaluate_flops": (ctypes.c_double, [ctypes.c_char_p]),
    "xtc_hip_evaluate_flops_operands": (ctypes.c_double, [ctypes.c_char_p, _i]),
    "xtc_hip_datasheet_flops": (ctypes.c_double, [ctypes.c_char_p]),
}

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def library_available() -> bool:
    return LIB_PATH.exists()


def lib() -> ctypes.CDLL:
    """The loaded libxtc_hip.so with typed entry points."""
    global _lib
    if _lib is None and os.environ.get("XTC_HIP_PMU") == "1":
        from . import pmu  # GPU counters: the tool must register before the runtime starts

        pmu.enable()
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise HipError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m xtc_amd.csrc.build` (or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            for struct, size_fn in ((MatmulDesc, handle.xtc_hip_matmul_desc_size),
                                    (Conv2dDesc, handle.xtc_hip_conv2d_desc_size)):
                if ctypes.sizeof(struct) != size_fn():
                    raise HipError(f"{struct.__name__} is {ctypes.sizeof(struct)} bytes here but "
                                   f"{size_fn()} in {LIB_PATH.name}: the binding and include/xtc_hip.h differ")
            _lib = handle
    return _lib


def last_error() -> str:
    msg = lib().xtc_hip_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str = "") -> None:
    """Raises HipError with the library's message on a non-zero status."""
    if status != 0:
        raise HipError(f"{what + ': ' if what else ''}{last_error()}")


def gemm_instances() -> list[dict[str, Any]]:
    L = lib()
    out = []
    inst = GemmInstance()
    for i in range(L.xtc_hip_gemm_instance_count()):
        check(L.xtc_hip_gemm_instance_get(i, ctypes.byref(inst)), "gemm_instance_get")
        out.append(
            {
                "dtype": DTYPE_NAMES[inst.dtype],
                "conv": bool(inst.conv),
                "tile": inst.tile.as_tuple(),
                "lds_bytes": inst.lds_bytes,
                "threads": inst.threads,
            }
        )
    return out


_DTYPE_IDS = {"float32": XTC_HIP_F32, "bfloat16": XTC_HIP_BF16, "float64": XTC_HIP_F64}
DTYPE_IDS = _DTYPE_IDS
DTYPE_NAMES = {v: k for k, v in _DTYPE_IDS.items()}


def default_tile(dtype: str, conv: bool, M: int, N: int, K: int) -> tuple[tuple[int, int, int, int, int], int]:
    """(tile, split_k) the library picks for a shape when none is given."""
    t = Tile()
    sk = ctypes.c_int(1)
    check(lib().xtc_hip_default_tile(_DTYPE_IDS[dtype], int(conv), M, N, K, ctypes.byref(t), ctypes.byref(sk)), "default_tile")
    return t.as_tuple(), int(sk.value)


def matmul_pipeline_depths(desc: MatmulDesc) -> list[int]:
    """Pipeline depths of the kernel that runs `desc`, the default first."""
    out = (ctypes.c_int * 16)()
    n = lib().xtc_hip_matmul_pipeline_depths(ctypes.byref(desc), out, 16)
    if n < 0:
        raise HipError(f"matmul_pipeline_depths: {last_error()}")
    return list(out[: min(n, 16)])


def conv2d_pipeline_depths(desc: Conv2dDesc) -> list[int]:
    """Pipeline depths of the kernel that runs `desc`, the default first."""
    out = (ctypes.c_int * 16)()
    n = lib().xtc_hip_conv2d_pipeline_depths(ctypes.byref(desc), out, 16)
    if n < 0:
        raise HipError(f"conv2d_pipeline_depths: {last_error()}")
    return list(out[: min(n, 16)])


def conv2d_default_tile(desc: Conv2dDesc) -> tuple[tuple[int, int, int, int, int], int]:
    """(tile, split_k) a conv2d descriptor gets when it leaves the tile zeroed."""
    t = Tile()
    sk = ctypes.c_int(1)
    check(lib().xtc_hip_conv2d_default_tile(ctypes.byref(desc), ctypes.byref(t), ctypes.byref(sk)), "conv2d_default_tile")
    return t.as_tuple(), int(sk.value)
