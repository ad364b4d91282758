"""ctypes view of the C ABI in include/axis_hip.h (libaxis_hip.so).

This is the thin binding a reference-side FFI would generate: every call goes straight to the
HIP library, raises ``AxisError`` with ``axis_last_error()`` on a nonzero status, and never
falls back to anything else.  ``load()`` fails loudly when the library has not been built.
"""
from __future__ import annotations

import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libaxis_hip.so")
HEADER = os.path.join(os.path.dirname(HERE), "include", "axis_hip.h")

_lib = None


class AxisError(RuntimeError):
    """A nonzero status from the C ABI, carrying axis_last_error()."""


class UnfoldSpec(ctypes.Structure):
    """axis_unfold_spec (the reference's UnfoldSpec, runtime/backend.rs:1481-1501)."""

    _fields_ = [
        ("spatial_rank", ctypes.c_int32),
        ("input_len", ctypes.c_int64),
        ("output_len", ctypes.c_int64),
        ("input_rank", ctypes.c_int32),
        ("output_rank", ctypes.c_int32),
        ("forward_metadata", ctypes.c_int32 * 32),
        ("backward_metadata", ctypes.c_int32 * 32),
        ("channels_per_group", ctypes.c_int32),
        ("fill", ctypes.c_float),
        ("kernel", ctypes.c_int32 * 3),
        ("stride", ctypes.c_int32 * 3),
        ("padding", ctypes.c_int32 * 3),
        ("input_spatial", ctypes.c_int32 * 3),
        ("output_spatial", ctypes.c_int32 * 3),
        ("input_special_strides", ctypes.c_int32 * 4),
        ("output_special_strides", ctypes.c_int32 * 5),
    ]


class AdamTensor(ctypes.Structure):
    _fields_ = [("value", ctypes.c_void_p), ("gradient", ctypes.c_void_p),
                ("first", ctypes.c_void_p), ("second", ctypes.c_void_p),
                ("learning_rates", ctypes.c_void_p), ("len", ctypes.c_int64)]


def header_functions() -> list[str]:
    """Every function the public header declares."""
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(axis_\w+)\s*\(", text, re.M)))


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise AxisError(f"{LIB_PATH} is missing: run `python -m axis_amd.build` first")
        lib = ctypes.CDLL(LIB_PATH)
        lib.axis_last_error.restype = ctypes.c_char_p
        lib.axis_version.restype = ctypes.c_char_p
        _lib = lib
    return _lib


def check(status: int, what: str = "axis call") -> None:
    if status != 0:
        raise AxisError(f"{what}: {load().axis_last_error().decode()} (status {status})")


I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
VP = ctypes.c_void_p


class Buffer:
    """Device memory from the handle's caching allocator; released when collected."""

    def __init__(self, device: "Device", nbytes: int):
        self.device = device
        self.nbytes = int(nbytes)
        ptr = ctypes.c_void_p()
        check(load().axis_alloc(device.handle, ctypes.c_size_t(max(self.nbytes, 1)),
                                ctypes.byref(ptr)), "axis_alloc")
        self.ptr = ptr.value

    def __del__(self):
        try:
            if self.ptr and self.device.handle:
                load().axis_free(self.device.handle, VP(self.ptr))
        except Exception:
            pass

    @property
    def vp(self):
        return VP(self.ptr)


class Device:
    """One GPU, one stream, one caching allocator (axis_device)."""

    def __init__(self, ordinal: int = 0, bf16_matmul: bool = False):
        h = ctypes.c_void_p()
        create = "axis_device_create_bf16" if bf16_matmul else "axis_device_create"
        check(getattr(load(), create)(ordinal, ctypes.byref(h)), create)
        self.handle = h

    def call(self, name: str, *args):
        check(getattr(load(), name)(self.handle, *args), name)

    def empty(self, count: int, dtype=np.float32) -> Buffer:
        return Buffer(self, count * np.dtype(dtype).itemsize)

    def upload(self, array) -> Buffer:
        a = np.ascontiguousarray(array)
        buf = Buffer(self, a.nbytes)
        self.call("axis_upload", buf.vp, a.ctypes.data_as(VP), ctypes.c_size_t(a.nbytes))
        return buf

    def read(self, buf: Buffer, count: int, dtype=np.float32) -> np.ndarray:
        out = np.empty(count, dtype)
        self.call("axis_read", out.ctypes.data_as(VP), buf.vp, ctypes.c_size_t(out.nbytes))
        return out

    def synchronize(self):
        self.call("axis_device_synchronize")

    def stream(self) -> int:
        s = ctypes.c_void_p()
        self.call("axis_device_stream", ctypes.byref(s))
        return s.value or 0
