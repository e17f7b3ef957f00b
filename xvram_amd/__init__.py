"""xvram_amd — MI355X-native out-of-core FP32 SGEMM behind the xVRAM v1 C ABI.

The product is the native library ``lib/libxvram.so`` (C++20 host runtime +
gfx950 FP32-MFMA kernel). It exports exactly one symbol, ``xvram_get_api``: the
reference's v1 and v2 tables, and (under the private version number
``abi.EXT_ABI_VERSION_1``) this build's extension table: GEMM plans with a
fused bias/ReLU epilogue and a device query. This module is a thin Python client of that C ABI
(ctypes), used by the tests and the bench the same way a C caller uses the
function tables. There is no Python or CPU fallback: if the native library is
missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import numpy as np

from . import abi

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(HERE, "lib")
PRODUCT_LIB = os.path.join(LIB_DIR, "libxvram.so")
HOSTSIM_LIB = os.path.join(LIB_DIR, "libxvram_hostsim.so")

__all__ = ["Library", "Session", "Allocation", "GemmPlan", "Operation", "XvramError", "abi",
           "TransactionView", "access", "epilogue", "matrix", "load", "PRODUCT_LIB",
           "HOSTSIM_LIB"]


class XvramError(RuntimeError):
    def __init__(self, status: int, where: str, info: Optional[abi.ErrorInfo] = None):
        self.status = status
        self.status_name = abi.STATUS.get(status, "unknown")
        self.where = where
        self.info = info
        detail = ""
        if info is not None:
            detail = (f" [{info.stage.decode()}/{info.operation.decode()}"
                      f" native={info.native_name.decode()}:{info.native_code}]"
                      f" {info.message.decode()}")
        super().__init__(f"{where}: {self.status_name} ({status}){detail}")


class Library:
    """The xvram_get_api function table of one native library."""

    def __init__(self, path: str = PRODUCT_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(
                f"{path} is not built; run `python -m xvram_amd.build` (no fallback exists)")
        self.path = path
        self.dll = ctypes.CDLL(path)
        get_api = self.dll.xvram_get_api
        get_api.argtypes = [ctypes.c_uint32, ctypes.c_uint32, ctypes.c_void_p]
        get_api.restype = ctypes.c_uint32
        self.get_api = get_api
        self.api = abi.ApiV1()
        status = get_api(abi.ABI_VERSION_1, ctypes.sizeof(self.api), ctypes.byref(self.api))
        if status != abi.SUCCESS:
            raise XvramError(status, "xvram_get_api")
        self.ext = abi.ExtV1()
        status = get_api(abi.EXT_ABI_VERSION_1, ctypes.sizeof(self.ext), ctypes.byref(self.ext))
        if status != abi.SUCCESS:
            raise XvramError(status, "xvram_get_api(extension table)")

    def status_name(self, status: int) -> str:
        return self.api.status_name(status).decode()


_loaded = {}


def load(hostsim: bool = False) -> Library:
    path = HOSTSIM_LIB if hostsim else PRODUCT_LIB
    if path not in _loaded:
        _loaded[path] = Library(path)
    return _loaded[path]


class Session:
    def __init__(self, lib: Library, **config):
        self.lib = lib
        self.api = lib.api
        cfg = abi.session_config_init()
        for key, value in config.items():
            setattr(cfg, key, value)
        handle = ctypes.c_void_p()
        status = self.api.session_create(ctypes.byref(cfg), ctypes.byref(handle))
        if status != abi.SUCCESS:
            raise XvramError(status, "session_create")
        self.handle = handle
        self.config = cfg

    def error(self) -> abi.ErrorInfo:
        info = abi.error_info_init()
        self.api.session_get_error(self.handle, ctypes.byref(info))
        return info

    def check(self, status: int, where: str) -> None:
        if status != abi.SUCCESS:
            raise XvramError(status, where, self.error())

    def telemetry(self) -> abi.SessionTelemetry:
        t = abi.telemetry_init()
        self.check(self.api.session_get_telemetry(self.handle, ctypes.byref(t)), "telemetry")
        return t

    def allocation(self, size: int, alignment: int = 0, flags: int = 0) -> "Allocation":
        return Allocation(self, size, alignment, flags)

    def drain(self, timeout_ms: int = abi.TIMEOUT_INFINITE) -> None:
        self.check(self.api.session_drain(self.handle, timeout_ms), "session_drain")

    def prefetch(self, ranges, deadline_ms: int = 0) -> "Operation":
        """prefetch_submit over ``ranges`` (a list of :func:`access` records)."""
        arr = (abi.AccessRange * len(ranges))(*ranges)
        desc = abi.PrefetchDesc()
        desc.struct_size = ctypes.sizeof(desc)
        desc.ranges = ctypes.cast(arr, ctypes.POINTER(abi.AccessRange)) if ranges else None
        desc.range_count = len(ranges)
        desc.deadline_ms = deadline_ms
        handle = ctypes.c_void_p()
        self.check(self.api.prefetch_submit(self.handle, ctypes.byref(desc), ctypes.byref(handle)),
                   "prefetch_submit")
        return Operation(self, handle)

    def _transaction_desc(self, ranges, callback, workspace_bytes, deadline_ms):
        def trampoline(ctx_ptr, _user, err_ptr):
            try:
                result = callback(TransactionView(ctx_ptr.contents))
                return abi.SUCCESS if result is None else int(result)
            except Exception as exc:  # reported through the callback error record
                msg = f"{type(exc).__name__}: {exc}".encode()[:255]
                err_ptr.contents.message = msg
                return abi.CALLBACK_FAILED
        cb = abi.TransactionCallback(trampoline)
        arr = (abi.AccessRange * len(ranges))(*ranges)
        desc = abi.TransactionDesc()
        desc.struct_size = ctypes.sizeof(desc)
        desc.ranges = ctypes.cast(arr, ctypes.POINTER(abi.AccessRange)) if ranges else None
        desc.range_count = len(ranges)
        desc.workspace_bytes = workspace_bytes
        desc.deadline_ms = deadline_ms
        desc.callback = cb
        return desc, (cb, arr)

    def transaction(self, ranges, callback, workspace_bytes: int = 0,
                    deadline_ms: int = 0) -> "Operation":
        """transaction_submit: ``callback(view)`` runs on the session worker with
        the working set resident; it returns None (success) or a status."""
        desc, keep = self._transaction_desc(ranges, callback, workspace_bytes, deadline_ms)
        handle = ctypes.c_void_p()
        self.check(self.api.transaction_submit(self.handle, ctypes.byref(desc),
                                               ctypes.byref(handle)), "transaction_submit")
        op = Operation(self, handle)
        op._keep = keep  # the callback must outlive the queued operation
        return op

    def execute_transaction(self, ranges, callback, workspace_bytes: int = 0,
                            deadline_ms: int = 0, timeout_ms: int = abi.TIMEOUT_INFINITE) -> None:
        desc, keep = self._transaction_desc(ranges, callback, workspace_bytes, deadline_ms)
        status = self.api.transaction_execute(self.handle, ctypes.byref(desc), timeout_ms)
        del keep
        self.check(status, "transaction_execute")

    def close(self, timeout_ms: int = abi.TIMEOUT_INFINITE) -> None:
        if self.handle:
            self.check(self.api.session_close(self.handle, timeout_ms), "session_close")

    def release(self) -> None:
        if self.handle:
            self.api.session_release(self.handle)
            self.handle = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        try:
            self.close()
        finally:
            self.release()


class Allocation:
    def __init__(self, session: Session, size: int, alignment: int = 0, flags: int = 0):
        self.session = session
        desc = abi.allocation_desc_init(size)
        desc.alignment_bytes = alignment
        desc.flags = flags
        handle = ctypes.c_void_p()
        session.check(session.api.allocation_create(session.handle, ctypes.byref(desc),
                                                    ctypes.byref(handle)), "allocation_create")
        self.handle = handle
        self.size = size

    def info(self) -> abi.AllocationInfo:
        out = abi.AllocationInfo()
        out.struct_size = ctypes.sizeof(out)
        self.session.check(self.session.api.allocation_get_info(self.handle, ctypes.byref(out)),
                           "allocation_get_info")
        return out

    def write(self, data, offset: int = 0) -> None:
        arr = np.ascontiguousarray(data)
        self.session.check(self.session.api.allocation_write(
            self.handle, offset, arr.ctypes.data_as(ctypes.c_void_p), arr.nbytes),
            "allocation_write")

    def read_into(self, out: np.ndarray, offset: int = 0) -> np.ndarray:
        assert out.flags.c_contiguous
        self.session.check(self.session.api.allocation_read(
            self.handle, offset, out.ctypes.data_as(ctypes.c_void_p), out.nbytes),
            "allocation_read")
        return out

    def read(self, nbytes: Optional[int] = None, offset: int = 0, dtype=np.uint8) -> np.ndarray:
        nbytes = self.size - offset if nbytes is None else nbytes
        out = np.empty(nbytes // np.dtype(dtype).itemsize, dtype=dtype)
        return self.read_into(out, offset)

    def release(self) -> None:
        if self.handle:
            self.session.check(self.session.api.allocation_release(self.handle),
                               "allocation_release")
            self.handle = None


def access(allocation: Allocation, offset: int, length: int,
           mode: int = abi.ACCESS_READ) -> abi.AccessRange:
    r = abi.AccessRange()
    r.allocation = allocation.handle.value if allocation is not None else None
    r.offset_bytes, r.length_bytes, r.mode = offset, length, mode
    return r


class TransactionView:
    """What a transaction callback sees: the resolved ranges (allocation id,
    offset, length, device address, mode), the workspace and the stream."""

    def __init__(self, ctx: abi.TransactionContext):
        self.operation_id = ctx.operation_id
        self.transaction_id = ctx.transaction_id
        self.ranges = [(r.allocation_id, r.offset_bytes, r.length_bytes, r.device_address, r.mode)
                       for r in (ctx.ranges[i] for i in range(ctx.range_count))]
        self.workspace_address = ctx.workspace_device_address
        self.workspace_bytes = ctx.workspace_bytes
        self.stream = ctx.native_stream


def matrix(allocation: Allocation, rows: int, columns: int, ld: int,
           layout: int = abi.COLUMN_MAJOR, offset: int = 0,
           data_type: int = abi.DATA_FP32) -> abi.Matrix:
    m = abi.matrix_init()
    m.allocation = allocation.handle.value if allocation is not None else None
    m.rows, m.columns, m.leading_dimension = rows, columns, ld
    m.layout = layout
    m.offset_bytes = offset
    m.data_type = data_type
    return m


class Operation:
    def __init__(self, session: Session, handle: ctypes.c_void_p):
        self.session = session
        self.handle = handle

    def poll(self) -> abi.OperationInfo:
        info = abi.operation_info_init()
        self.session.check(self.session.api.operation_poll(self.handle, ctypes.byref(info)),
                           "operation_poll")
        return info

    def wait(self, timeout_ms: int = abi.TIMEOUT_INFINITE):
        info = abi.operation_info_init()
        status = self.session.api.operation_wait(self.handle, timeout_ms, ctypes.byref(info))
        return status, info

    def cancel(self) -> int:
        return self.session.api.operation_cancel(self.handle)

    def error(self) -> abi.ErrorInfo:
        info = abi.error_info_init()
        self.session.api.operation_get_error(self.handle, ctypes.byref(info))
        return info

    def release(self) -> None:
        if self.handle:
            self.session.api.operation_release(self.handle)
            self.handle = None


def epilogue(bias: Optional[Allocation] = None, axis: int = abi.BIAS_NONE, offset: int = 0,
             relu: bool = False) -> abi.EpilogueV1:
    """A fused-epilogue record for GemmPlan(..., epilogue=...)."""
    e = abi.epilogue_init()
    e.bias = bias.handle.value if bias is not None else None
    e.bias_offset_bytes = offset
    e.bias_axis = axis
    e.activation = abi.ACTIVATION_RELU if relu else abi.ACTIVATION_NONE
    return e


class GemmPlan:
    def __init__(self, session: Session, a: abi.Matrix, b: abi.Matrix, c: abi.Matrix,
                 op_a: int = abi.OP_N, op_b: int = abi.OP_N, alpha: float = 1.0,
                 beta: float = 0.0, compute_mode: int = abi.COMPUTE_AUTO,
                 tile_hints=(0, 0, 0), deadline_ms: int = 0,
                 epilogue: Optional[abi.EpilogueV1] = None):
        self.session = session
        desc = abi.gemm_desc_init()
        desc.a, desc.b, desc.c = a, b, c
        desc.operation_a, desc.operation_b = op_a, op_b
        desc.alpha, desc.beta = alpha, beta
        desc.compute_mode = compute_mode
        desc.tile_m_hint, desc.tile_n_hint, desc.tile_k_hint = tile_hints
        desc.deadline_ms = deadline_ms
        self.desc = desc
        handle = ctypes.c_void_p()
        if epilogue is None:
            status = session.api.gemm_plan_create(session.handle, ctypes.byref(desc),
                                                  ctypes.byref(handle))
        else:
            status = session.lib.ext.gemm_plan_create_epilogue(
                session.handle, ctypes.byref(desc), ctypes.byref(epilogue), ctypes.byref(handle))
        session.check(status, "gemm_plan_create")
        self.handle = handle

    def info(self) -> abi.GemmPlanInfo:
        out = abi.plan_info_init()
        self.session.check(self.session.api.gemm_plan_get_info(self.handle, ctypes.byref(out)),
                           "gemm_plan_get_info")
        return out

    def execute(self, timeout_ms: int = abi.TIMEOUT_INFINITE) -> None:
        self.session.check(self.session.api.gemm_execute(self.handle, timeout_ms), "gemm_execute")

    def submit(self) -> Operation:
        handle = ctypes.c_void_p()
        self.session.check(self.session.api.gemm_submit(self.handle, ctypes.byref(handle)),
                           "gemm_submit")
        return Operation(self.session, handle)

    def release(self) -> None:
        if self.handle:
            self.session.api.gemm_plan_release(self.handle)
            self.handle = None
