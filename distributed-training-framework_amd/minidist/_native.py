"""ctypes binding of libmdx.so (the C ABI in include/mdx.h).

This is the only module that touches the native library.  Every kernel call
goes through :func:`lib`, which raises when ``libmdx.so`` has not been built:
there is no Python or CPU fallback for any kernel, so a missing library is a
loud error, never a silently slower path.

Span / piece tables are built as numpy structured arrays whose memory layout
is the C structs ``mdx_span`` / ``mdx_piece``; the library copies them into
each dispatch's kernel arguments, so they only have to live for the call.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import numpy as np
import torch

LIB_PATH = Path(__file__).resolve().parent / "libmdx.so"

MDX_F32 = 0
MDX_BF16 = 1
MDX_F16 = 2
MDX_MAX_WORLD = 16
ABI_VERSION = 10
# Reduction operations of mdx_allreduce_op (torch.distributed.ReduceOp's SUM, PRODUCT, MIN, MAX).
MDX_OP_SUM, MDX_OP_PRODUCT, MDX_OP_MIN, MDX_OP_MAX = 0, 1, 2, 3

# Every function declared in include/mdx.h, with (restype, argtypes).
_vp, _i32, _i64, _f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float
SIGNATURES: dict[str, tuple] = {
    "mdx_pack": (_i32, [_vp, _i32, _i32, _i32, _f32, _i32, _vp, _vp]),
    "mdx_unpack": (_i32, [_vp, _i32, _i32, _i32, _f32, _vp, _vp]),
    "mdx_unscale_found_inf": (_i32, [_vp, _i32, _i32, _f32, _vp, _vp]),
    "mdx_allreduce_sum": (_i32, [_vp, _i32, _i32, _vp, _vp, _i32, _vp, _vp]),
    "mdx_allreduce_op": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp, _i32, _vp, _vp]),
    "mdx_allreduce_unpack": (_i32, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _f32, _vp, _vp]),
    "mdx_allreduce_unpack_wide": (_i32, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _i32, _f32, _f32, _vp, _vp]),
    "mdx_reduce_scatter_share": (
        _i32,
        [_vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _vp, _i32, _i32, _f32, _vp, _vp],
    ),
    "mdx_pack_allreduce_unpack": (
        _i32, [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _f32, _f32, _vp, _vp, _vp],
    ),
    "mdx_cast_f32_bf16": (_i32, [_vp, _vp, _i64, _vp]),
    "mdx_plan_spans": (_i32, [_vp, _i32, _i32, _i32, _vp, _vp]),
    "mdx_plan_allreduce_unpack": (_i32, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _vp, _vp]),
    "mdx_plan_allreduce_unpack_wide": (
        _i32, [_vp, _i32, _i32, _vp, _i32, _vp, _i32, _i32, _f32, _vp, _vp],
    ),
    "mdx_plan_pack_allreduce_unpack": (
        _i32, [_vp, _i32, _i32, _i32, _vp, _i32, _vp, _i32, _f32, _vp, _vp],
    ),
    "mdx_pack_allreduce_unpack_planned": (_i32, [_vp, _vp, _f32, _vp, _vp, _vp]),
    "mdx_pack_planned": (_i32, [_vp, _vp, _f32, _i32, _vp, _vp]),
    "mdx_unpack_planned": (_i32, [_vp, _vp, _f32, _vp, _vp]),
    "mdx_allreduce_unpack_planned": (_i32, [_vp, _vp, _f32, _vp, _vp]),
    "mdx_pack_allreduce_unpack_planned_noalloc": (_i32, [_vp, _f32, _vp, _vp, _vp]),
    "mdx_reduce_scatter_share_multi": (
        _i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _vp, _vp],
    ),
    "mdx_plan_reduce_scatter_share_multi": (_i32, [_vp, _vp, _i32, _vp, _i32, _i32, _i32, _vp, _vp]),
    "mdx_reduce_scatter_share_multi_planned": (_i32, [_vp, _vp, _i32, _i32, _f32, _vp, _vp]),
    "mdx_host_device_address": (_i32, [_vp, _vp]),
    "mdx_ipc_export": (_i32, [_vp, _vp]),
    "mdx_ipc_open": (_i32, [_vp, _vp]),
    "mdx_ipc_close": (_i32, [_vp]),
    "mdx_strerror": (ctypes.c_char_p, [_i32]),
    "mdx_abi_version": (_i32, []),
}

SPAN_DTYPE = np.dtype([("src", "<u8"), ("dst", "<u8"), ("numel", "<i8")])
PIECE_DTYPE = np.dtype([("own", "<u8"), ("pos", "<i8"), ("numel", "<i8")])
GRAD_RUN_DTYPE = np.dtype([("offset", "<i8"), ("numel", "<i8"), ("grad", "<u8")])
PACK_RUN_DTYPE = np.dtype([("offset", "<i8"), ("numel", "<i8"), ("src", "<u8"), ("grad", "<u8")])

_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


class NativeLibraryMissing(RuntimeError):
    pass


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it was never built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is missing: build the gfx950 kernels with "
                    "`python -m minidist._build` (there is no fallback path)"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            if handle.mdx_abi_version() != ABI_VERSION:
                raise NativeLibraryMissing(
                    f"{LIB_PATH} has ABI {handle.mdx_abi_version()}, expected {ABI_VERSION}: rebuild it"
                )
            _lib = handle
    return _lib


def available() -> bool:
    return LIB_PATH.exists()


def strerror(code: int) -> str:
    return lib().mdx_strerror(code).decode()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise RuntimeError(f"{what} failed: {strerror(rc)} (status {rc})")


# ---------------------------------------------------------------------------
# torch <-> ABI plumbing
# ---------------------------------------------------------------------------


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return MDX_F32
    if dtype == torch.bfloat16:
        return MDX_BF16
    if dtype == torch.float16:
        return MDX_F16
    raise TypeError(f"minidist kernels handle float32, bfloat16 and float16, not {dtype}")


def require_device_tensor(t: torch.Tensor, what: str) -> None:
    if not t.is_cuda:
        raise RuntimeError(
            f"{what} lives on {t.device}; minidist's gradient path runs only as HIP kernels "
            "on a GPU (there is no CPU implementation)"
        )


def require_dense(t: torch.Tensor, what: str) -> None:
    if not t.is_contiguous():
        raise RuntimeError(f"{what} must be contiguous for the flat-span kernels")


_current_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    """The raw handle of ``device``'s current stream (one C call where torch exposes it)."""
    if _current_raw_stream is not None:
        return _current_raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


# (device index, raw handle) -> the Stream object torch.cuda.current_stream returned for it
_stream_objects: dict[tuple[int, int], torch.cuda.Stream] = {}


def current_stream(device: torch.device) -> torch.cuda.Stream:
    """``torch.cuda.current_stream(device)``, found by the stream's raw handle (one C call) among
    the Stream objects built before: a handle names one stream, and building the object costs
    ~2 us of host time on the path between a launch and the step's flag read."""
    if _current_raw_stream is None:
        return torch.cuda.current_stream(device)
    index = device.index if device.index is not None else torch.cuda.current_device()
    key = (index, _current_raw_stream(index))
    stream = _stream_objects.get(key)
    if stream is None:
        stream = _stream_objects[key] = torch.cuda.current_stream(device)
    return stream


def spans_array(rows: list[tuple[int, int, int]]) -> np.ndarray:
    return np.array(rows, dtype=SPAN_DTYPE)


def pieces_array(rows: list[tuple[int, int, int]]) -> np.ndarray:
    return np.array(rows, dtype=PIECE_DTYPE)


def _ptr(a: np.ndarray | None) -> int | None:
    return None if a is None or a.size == 0 else a.ctypes.data


def _ptrs(values: list[int]) -> ctypes.Array:
    return (ctypes.c_void_p * len(values))(*values)


# ---------------------------------------------------------------------------
# Entry points (thin: argument marshalling + status check)
# ---------------------------------------------------------------------------


def pack(
    spans: np.ndarray, src_dtype: int, dst_dtype: int, scale: float, divide: bool, stream: int,
    clear_flag: int | None = None,
) -> None:
    rc = lib().mdx_pack(_ptr(spans), len(spans), src_dtype, dst_dtype, scale, int(divide), clear_flag, stream)
    check(rc, "mdx_pack")


def unpack(
    spans: np.ndarray, src_dtype: int, dst_dtype: int, inv_scale: float, found_inf: int | None, stream: int
) -> None:
    rc = lib().mdx_unpack(_ptr(spans), len(spans), src_dtype, dst_dtype, inv_scale, found_inf, stream)
    check(rc, "mdx_unpack")


def unscale_found_inf(spans: np.ndarray, dtype: int, inv_scale: float, found_inf: int | None, stream: int) -> None:
    rc = lib().mdx_unscale_found_inf(_ptr(spans), len(spans), dtype, inv_scale, found_inf, stream)
    check(rc, "mdx_unscale_found_inf")


def allreduce_sum(
    replicas: list[int], dtype: int, offsets: list[int], numels: list[int], out: int, stream: int
) -> None:
    n = len(offsets)
    offs = (ctypes.c_int64 * n)(*offsets)
    nums = (ctypes.c_int64 * n)(*numels)
    rc = lib().mdx_allreduce_sum(_ptrs(replicas), len(replicas), dtype, offs, nums, n, out, stream)
    check(rc, "mdx_allreduce_sum")


def allreduce_op(
    replicas: list[int], dtype: int, op: int, offsets: list[int], numels: list[int], out: int, stream: int
) -> None:
    n = len(offsets)
    offs = (ctypes.c_int64 * n)(*offsets)
    nums = (ctypes.c_int64 * n)(*numels)
    rc = lib().mdx_allreduce_op(_ptrs(replicas), len(replicas), dtype, op, offs, nums, n, out, stream)
    check(rc, "mdx_allreduce_op")


def grad_runs_array(rows: list[tuple[int, int, int]]) -> np.ndarray:
    return np.array(rows, dtype=GRAD_RUN_DTYPE)


def allreduce_unpack(
    replicas: list[int], dtype: int, runs: np.ndarray, out: int | None, grad_dtype: int,
    inv_scale: float, found_inf: int | None, stream: int,
) -> None:
    rc = lib().mdx_allreduce_unpack(
        _ptrs(replicas), len(replicas), dtype, _ptr(runs), len(runs), out, grad_dtype, inv_scale,
        found_inf, stream,
    )
    check(rc, "mdx_allreduce_unpack")


def allreduce_unpack_wide(
    replicas: list[int], wire_dtype: int, runs: np.ndarray, out: int | None, reduce_dtype: int, grad_dtype: int,
    prescale: float, inv_scale: float, found_inf: int | None, stream: int,
) -> None:
    rc = lib().mdx_allreduce_unpack_wide(
        _ptrs(replicas), len(replicas), wire_dtype, _ptr(runs), len(runs), out, reduce_dtype, grad_dtype,
        prescale, inv_scale, found_inf, stream,
    )
    check(rc, "mdx_allreduce_unpack_wide")


def pack_runs_array(rows: list[tuple[int, int, int, int]]) -> np.ndarray:
    return np.array(rows, dtype=PACK_RUN_DTYPE)


def pack_allreduce_unpack(
    replicas: list[int], rank: int, wire_dtype: int, runs: np.ndarray, out: int | None, reduce_dtype: int,
    scale: float, inv_scale: float, found_inf: int | None, clear_flag: int | None, stream: int,
) -> None:
    rc = lib().mdx_pack_allreduce_unpack(
        _ptrs(replicas), len(replicas), rank, wire_dtype, _ptr(runs), len(runs), out, reduce_dtype, scale,
        inv_scale, found_inf, clear_flag, stream,
    )
    check(rc, "mdx_pack_allreduce_unpack")


def reduce_scatter_share(
    own: np.ndarray,
    peers: list[int],
    rank: int,
    in_dtype: int,
    reduce_dtype: int,
    divide: bool,
    shard: int,
    shard_dtype: int,
    accumulate: bool,
    inv_scale: float,
    found_inf: int | None,
    stream: int,
) -> None:
    rc = lib().mdx_reduce_scatter_share(
        _ptr(own), len(own), _ptrs(peers), len(peers), rank, in_dtype, reduce_dtype, int(divide),
        shard, shard_dtype, int(accumulate), inv_scale, found_inf, stream,
    )
    check(rc, "mdx_reduce_scatter_share")


MDX_EDTYPE = -2
MDX_EALIAS = -4
MDX_ESIZE = -5
MDX_ESCRATCH = -6
MDX_EOP = -7
NOALLOC_SCRATCH_BYTES = 256 * 1024


class Plan:
    """A device-resident work plan: host bytes (kernel arguments, grid) + device copy.

    Built once by ``mdx_plan_*``; launched any number of times while the
    addresses frozen into it stay valid.  Keeping the object alive keeps the
    device copy alive (it is released to torch's stream-ordered allocator)."""

    __slots__ = ("host", "device", "host_ptr", "device_ptr")

    def __init__(self, host: np.ndarray, device_tensor):
        self.host = host
        self.device = device_tensor
        self.host_ptr = host.ctypes.data
        self.device_ptr = device_tensor.data_ptr()


def _build_plan(call, what: str, device) -> Plan:
    size = ctypes.c_int64(0)
    rc = call(None, ctypes.byref(size))
    if rc not in (0, MDX_ESIZE):
        check(rc, what)
    host = np.zeros((size.value + 7) // 8, dtype=np.uint64)  # 8-byte aligned
    cap = ctypes.c_int64(host.nbytes)
    check(call(host.ctypes.data, ctypes.byref(cap)), what)
    # Staged through pinned memory so the upload is an asynchronous copy on the
    # current stream: rebuilding a plan never waits for the GPU to drain.
    staged = torch.empty(host.nbytes, dtype=torch.uint8, pin_memory=True)
    staged.copy_(torch.from_numpy(host.view(np.uint8)))
    dev = staged.to(device, non_blocking=True)
    return Plan(host, dev)


def plan_spans(spans: np.ndarray, src_dtype: int, dst_dtype: int, device) -> Plan:
    return _build_plan(
        lambda buf, size: lib().mdx_plan_spans(_ptr(spans), len(spans), src_dtype, dst_dtype, buf, size),
        "mdx_plan_spans", device,
    )


def plan_allreduce_unpack(
    replicas: list[int], dtype: int, runs: np.ndarray, out: int | None, grad_dtype: int, device
) -> Plan:
    reps = _ptrs(replicas)
    return _build_plan(
        lambda buf, size: lib().mdx_plan_allreduce_unpack(
            reps, len(replicas), dtype, _ptr(runs), len(runs), out, grad_dtype, buf, size
        ),
        "mdx_plan_allreduce_unpack", device,
    )


def plan_allreduce_unpack_wide(
    replicas: list[int], wire_dtype: int, runs: np.ndarray, out: int | None, reduce_dtype: int, grad_dtype: int,
    prescale: float, device,
) -> Plan:
    reps = _ptrs(replicas)
    return _build_plan(
        lambda buf, size: lib().mdx_plan_allreduce_unpack_wide(
            reps, len(replicas), wire_dtype, _ptr(runs), len(runs), out, reduce_dtype, grad_dtype, prescale,
            buf, size,
        ),
        "mdx_plan_allreduce_unpack_wide", device,
    )


def plan_pack_allreduce_unpack(
    replicas: list[int], rank: int, wire_dtype: int, runs: np.ndarray, out: int | None, reduce_dtype: int,
    scale: float, device,
) -> Plan:
    reps = _ptrs(replicas)
    return _build_plan(
        lambda buf, size: lib().mdx_plan_pack_allreduce_unpack(
            reps, len(replicas), rank, wire_dtype, _ptr(runs), len(runs), out, reduce_dtype, scale, buf, size
        ),
        "mdx_plan_pack_allreduce_unpack", device,
    )


def pack_allreduce_unpack_planned(
    plan: Plan, inv_scale: float, found_inf: int | None, clear_flag: int | None, stream: int
) -> None:
    rc = lib().mdx_pack_allreduce_unpack_planned(plan.host_ptr, plan.device_ptr, inv_scale, found_inf, clear_flag,
                                                 stream)
    check(rc, "mdx_pack_allreduce_unpack_planned")


def reduce_scatter_share_multi(
    own: np.ndarray, outs: list[int], peers: list[int], rank: int, in_dtype: int, reduce_dtype: int, divide: bool,
    shard_dtype: int, accumulate: bool, inv_scale: float, found_inf: int | None, stream: int,
) -> None:
    """Several units' reduce-scatter shares: piece k of ``own`` (absolute row positions) lands in ``outs[k]``."""
    rc = lib().mdx_reduce_scatter_share_multi(
        _ptr(own), _ptrs(outs) if outs else None, len(own), _ptrs(peers), len(peers), rank, in_dtype, reduce_dtype,
        int(divide), shard_dtype, int(accumulate), inv_scale, found_inf, stream,
    )
    check(rc, "mdx_reduce_scatter_share_multi")


def plan_reduce_scatter_share_multi(
    own: np.ndarray, outs: list[int], peers: list[int], rank: int, in_dtype: int, device
) -> Plan:
    out_ptrs = _ptrs(outs) if outs else None
    reps = _ptrs(peers)
    return _build_plan(
        lambda buf, size: lib().mdx_plan_reduce_scatter_share_multi(
            _ptr(own), out_ptrs, len(own), reps, len(peers), rank, in_dtype, buf, size
        ),
        "mdx_plan_reduce_scatter_share_multi", device,
    )


def reduce_scatter_share_multi_planned(
    plan: Plan, divide: bool, accumulate: bool, inv_scale: float, found_inf: int | None, stream: int
) -> None:
    rc = lib().mdx_reduce_scatter_share_multi_planned(
        plan.host_ptr, plan.device_ptr, int(divide), int(accumulate), inv_scale, found_inf, stream
    )
    check(rc, "mdx_reduce_scatter_share_multi_planned")


def host_device_address(host_ptr: int) -> int:
    """The address kernels use for pinned host memory at ``host_ptr``."""
    out = ctypes.c_void_p()
    check(lib().mdx_host_device_address(host_ptr, ctypes.byref(out)), "mdx_host_device_address")
    return int(out.value)


def clear_flag(flag_address: int, stream: int) -> None:
    """Set one int32 found-inf flag to 0 in stream order (a one-lane dispatch; works for device
    memory and for pinned host memory at its device address)."""
    check(lib().mdx_pack(None, 0, MDX_F32, MDX_F32, 1.0, 0, flag_address, stream), "mdx_pack (flag clear)")


IPC_HANDLE_BYTES = 64
IPC_MAX_ALLOC_BYTES = 1 << 31


class IpcHandle(ctypes.Structure):
    """``mdx_ipc_handle``: the runtime's handle of a device allocation, the exported pointer's
    offset in it, and the allocation's size."""

    _fields_ = [("bytes", ctypes.c_ubyte * IPC_HANDLE_BYTES), ("offset", ctypes.c_int64),
                ("alloc_bytes", ctypes.c_int64)]

    def to_bytes(self) -> bytes:
        return bytes(memoryview(self))

    @classmethod
    def from_bytes(cls, raw: bytes) -> IpcHandle:
        return cls.from_buffer_copy(raw)


def ipc_export(ptr: int) -> IpcHandle:
    h = IpcHandle()
    check(lib().mdx_ipc_export(ptr, ctypes.byref(h)), "mdx_ipc_export")
    return h


def ipc_open(h: IpcHandle) -> int:
    """Maps a peer's exported allocation; returns the exported pointer in this process."""
    base = ctypes.c_void_p()
    check(lib().mdx_ipc_open(ctypes.byref(h), ctypes.byref(base)), "mdx_ipc_open")
    return int(base.value) + int(h.offset)


def ipc_close_base(base: int) -> None:
    """Unmaps a peer allocation by its mapped base address (what :func:`ipc_open` returned, minus
    the handle's offset)."""
    check(lib().mdx_ipc_close(base), "mdx_ipc_close")


def pack_allreduce_unpack_planned_noalloc(
    plan: Plan, inv_scale: float, found_inf: int | None, clear_flag: int | None, stream: int
) -> None:
    """The same launch as :func:`pack_allreduce_unpack_planned` from the plan's host bytes only:
    the library uploads them into its own per-GPU buffer (no device memory is allocated)."""
    rc = lib().mdx_pack_allreduce_unpack_planned_noalloc(plan.host_ptr, inv_scale, found_inf, clear_flag, stream)
    check(rc, "mdx_pack_allreduce_unpack_planned_noalloc")


def pack_planned(plan: Plan, scale: float, divide: bool, stream: int, clear_flag: int | None = None) -> None:
    rc = lib().mdx_pack_planned(plan.host_ptr, plan.device_ptr, scale, int(divide), clear_flag, stream)
    check(rc, "mdx_pack_planned")


def unpack_planned(plan: Plan, inv_scale: float, found_inf: int | None, stream: int) -> None:
    check(lib().mdx_unpack_planned(plan.host_ptr, plan.device_ptr, inv_scale, found_inf, stream), "mdx_unpack_planned")


def allreduce_unpack_planned(plan: Plan, inv_scale: float, found_inf: int | None, stream: int) -> None:
    rc = lib().mdx_allreduce_unpack_planned(plan.host_ptr, plan.device_ptr, inv_scale, found_inf, stream)
    check(rc, "mdx_allreduce_unpack_planned")


def cast_f32_bf16(src: int, dst: int, numel: int, stream: int) -> None:
    check(lib().mdx_cast_f32_bf16(src, dst, numel, stream), "mdx_cast_f32_bf16")


def f32(x: float) -> float:
    """The fp32 value a Python float becomes when ATen uses it as a scalar."""
    return float(np.float32(x))
