"""Process-group bootstrap, instrumented collectives, and the resident replica group.

Public surface and byte accounting follow minidist/comm.py of the reference
(``CommStats`` :50-99, ``record_comm`` :105-113, bootstrap :121-202, the
collective wrappers :223-277), so callers and the accounting formulas are
unchanged.  What changes is what sits under the collective hook:

* With a real ``torch.distributed`` group the wrappers forward to
  ``dist.*`` exactly as the reference does (RCCL on ROCm devices).  A gloo
  group moves host memory: a device tensor handed to one of its collectives
  is staged through the host with synchronous copies (``dist_*`` below).
* With a :class:`ResidentGroup` -- W data-parallel replicas emulated on ONE
  GPU -- the peers' contributions are already resident in this GPU's HBM
  (symmetric buffers, one row per replica) and the reduction arithmetic runs
  as a gfx950 kernel over them, in the fixed rank order 0..W-1.  The call
  returns a Work whose ``wait()`` orders the caller's stream after the kernel;
  nothing synchronises the host.
* With an :class:`IpcGroup` -- W processes of a real group -- the rows are
  each process's own allocations, mapped into its peers over IPC, and the
  same kernels run one-shot (each rank reads all W rows) or two-shot (each
  rank reduces its share, then copies its peers' reduced shares), ordered by
  host barriers over the wrapped group.
"""

from __future__ import annotations

import mmap
import os
import time
import uuid
from collections.abc import Iterator, Sequence
from contextlib import contextmanager
from dataclasses import dataclass, field
from datetime import timedelta

import numpy as np
import torch
import torch.distributed as dist

from . import _native

__all__ = [
    "CommStats",
    "comm_stats",
    "record_comm",
    "init_distributed",
    "shutdown_distributed",
    "current_device",
    "is_distributed",
    "get_rank",
    "get_world_size",
    "is_primary",
    "barrier",
    "all_reduce",
    "all_reduce_coalesced",
    "all_gather_into_tensor",
    "reduce_scatter_tensor",
    "broadcast",
    "print_rank0",
    "ResidentGroup",
    "IpcGroup",
    "StreamWork",
    "zeros_for_collective",
    "record_all_reduce",
]


# --------------------------------------------------------------------------
# Byte accounting (reference comm.py:50-113, same formulas)
# --------------------------------------------------------------------------


@dataclass
class _OpStat:
    count: int = 0
    payload_bytes: int = 0
    bus_bytes: int = 0


@dataclass
class CommStats:
    """Per-collective counters: ``payload_bytes`` (caller's tensor) and
    ``bus_bytes`` (ring-algorithm interconnect volume): all-reduce
    ``2(W-1)/W*N``, all-gather ``(W-1)/W*N_out``, reduce-scatter
    ``(W-1)/W*N_in``, broadcast ``N``."""

    enabled: bool = False
    ops: dict[str, _OpStat] = field(default_factory=dict)

    def add(self, op: str, payload_bytes: int, bus_bytes: int) -> None:
        if not self.enabled:
            return
        stat = self.ops.setdefault(op, _OpStat())
        stat.count += 1
        stat.payload_bytes += payload_bytes
        stat.bus_bytes += bus_bytes

    def reset(self) -> None:
        self.ops.clear()

    def total_bus_bytes(self) -> int:
        return sum(s.bus_bytes for s in self.ops.values())

    def as_rows(self) -> list[tuple[str, int, int, int]]:
        return sorted((name, s.count, s.payload_bytes, s.bus_bytes) for name, s in self.ops.items())


comm_stats = CommStats()


def record_all_reduce(payload_bytes: int, world: int) -> None:
    """Account one all-reduce of ``payload_bytes`` (reference comm.py:232-233)."""
    comm_stats.add("all_reduce", payload_bytes, int(2 * (world - 1) / world * payload_bytes))


@contextmanager
def record_comm() -> Iterator[CommStats]:
    """Enable byte accounting for the duration of the block."""
    previous, comm_stats.enabled = comm_stats.enabled, True
    comm_stats.reset()
    try:
        yield comm_stats
    finally:
        comm_stats.enabled = previous


# --------------------------------------------------------------------------
# Bootstrap (reference comm.py:121-202)
# --------------------------------------------------------------------------


def _default_backend() -> str:
    if torch.cuda.is_available() and dist.is_nccl_available():
        return "nccl"  # RCCL on ROCm
    return "gloo"


def init_distributed(backend: str | None = None, timeout_seconds: int = 1800) -> tuple[int, int, torch.device]:
    """Initialise the default process group from torchrun's environment.

    Falls back to a single-rank world without torchrun.  Binds the device
    before RCCL initialises (the communicator derives its topology from it).
    """
    if dist.is_initialized():
        return get_rank(), get_world_size(), current_device()
    rank = int(os.environ.get("RANK", 0))
    world_size = int(os.environ.get("WORLD_SIZE", 1))
    local_rank = int(os.environ.get("LOCAL_RANK", 0))
    backend = backend or _default_backend()
    if backend == "nccl":
        if not torch.cuda.is_available():
            raise RuntimeError("backend='nccl' requested but no GPU is available")
        torch.cuda.set_device(local_rank)
    os.environ.setdefault("MASTER_ADDR", "127.0.0.1")
    os.environ.setdefault("MASTER_PORT", "29500")
    dist.init_process_group(
        backend=backend, rank=rank, world_size=world_size, timeout=timedelta(seconds=timeout_seconds)
    )
    return rank, world_size, current_device()


def shutdown_distributed() -> None:
    if dist.is_initialized():
        dist.barrier()
        dist.destroy_process_group()


_cuda_devices: dict[int, torch.device] = {}


def current_device() -> torch.device:
    if torch.cuda.is_initialized() or torch.cuda.is_available():
        index = torch.cuda.current_device()
        device = _cuda_devices.get(index)
        if device is None:
            device = _cuda_devices[index] = torch.device("cuda", index)
        return device
    return torch.device("cpu")


def is_distributed() -> bool:
    return dist.is_available() and dist.is_initialized()


def get_rank(group=None) -> int:
    if isinstance(group, ResidentGroup):
        return group.rank()
    return dist.get_rank(group) if is_distributed() else 0


def get_world_size(group=None) -> int:
    if isinstance(group, ResidentGroup):
        return group.size()
    return dist.get_world_size(group) if is_distributed() else 1


def is_primary() -> bool:
    return get_rank() == 0


def barrier(group=None) -> None:
    if isinstance(group, ResidentGroup):
        return
    if is_distributed():
        dist.barrier(group)


def print_rank0(*args, **kwargs) -> None:
    if is_primary():
        print(*args, **kwargs, flush=True)


# --------------------------------------------------------------------------
# Resident replica group: W data-parallel replicas on one GPU
# --------------------------------------------------------------------------


class StreamWork:
    """Completion handle of a collective launched on a stream.

    ``wait()`` has NCCL-Work semantics on a GPU: it makes the *current* stream
    wait for the collective; the host does not block.  Nothing is recorded at
    launch: a waiter on the producing stream is already ordered after the
    collective, and any other waiter gets an event recorded on the producing
    stream when it waits -- later than the collective, so it may wait for more
    work than the collective, never for less.
    """

    __slots__ = ("_stream", "_event")

    def __init__(self, stream: torch.cuda.Stream):
        self._stream = stream
        self._event: torch.cuda.Event | None = None

    def _marker(self) -> torch.cuda.Event:
        if self._event is None:
            self._event = torch.cuda.Event()
            self._event.record(self._stream)
        return self._event

    def wait(self, timeout=None) -> bool:  # noqa: ARG002 - mirrors dist.Work.wait
        current = _native.current_stream(self._stream.device)
        if current != self._stream:
            current.wait_event(self._marker())
        return True

    def is_completed(self) -> bool:
        return self._marker().query()

    def synchronize(self) -> None:
        self._marker().synchronize()


_ROW_ALIGN_BYTES = 256


def _address(t: torch.Tensor) -> int:
    """The address of ``t``'s first element -- also for a tensor with no elements, whose
    ``data_ptr()`` torch reports as 0 (an empty bucket is still a place in its buffer)."""
    if t.numel():
        return t.data_ptr()
    return t.untyped_storage().data_ptr() + t.storage_offset() * t.element_size()
# A two-shot share starts a multiple of this many elements past the extent's start.
_SHARE_ALIGN_ELEMS = 64


def two_shot_shares(lo: int, hi: int, world: int, align: int = _SHARE_ALIGN_ELEMS) -> list[tuple[int, int]]:
    """Rank j's share ``[a, b)`` of the elements ``[lo, hi)`` in a two-shot all-reduce.

    The shares are contiguous and in rank order and cover ``[lo, hi)`` exactly;
    every share but the last non-empty one is a whole number of ``align``
    elements long (shares past the end are empty)."""
    if world < 1 or align < 1:
        raise ValueError("two_shot_shares: world and align must be positive")
    if hi <= lo:
        return [(lo, lo)] * world
    step = -(-(hi - lo) // (world * align)) * align  # ceil((hi - lo) / world), rounded up to align
    return [(min(lo + j * step, hi), min(lo + (j + 1) * step, hi)) for j in range(world)]


# A copy from several peers' memory goes out in chunks of this size, taken round-robin across
# the peers: a dispatch's workgroups run roughly in grid order, so spans in peer order would
# read one peer -- one xGMI link, across GPUs -- at a time.
_GATHER_CHUNK_BYTES = 1 << 20


def interleave_spans(spans: list[tuple[int, int, int]], src_esize: int, dst_esize: int,
                     chunk_bytes: int = _GATHER_CHUNK_BYTES) -> list[tuple[int, int, int]]:
    """``spans`` (src, dst, numel) cut into chunks of at most ``chunk_bytes`` of source and
    ordered round-robin: the first chunk of every span, then the second of every span, ..."""
    step = max(1, chunk_bytes // src_esize)
    chunks = [[(s + k * src_esize, d + k * dst_esize, min(step, n - k)) for k in range(0, n, step)]
              for s, d, n in spans]
    out = []
    for i in range(max((len(c) for c in chunks), default=0)):
        out.extend(c[i] for c in chunks if i < len(c))
    return out


def clip_grad_runs(runs: np.ndarray, lo: int, hi: int, grad_esize: int) -> np.ndarray:
    """The parts of an ``mdx_grad_run`` table that fall in ``[lo, hi)``.

    Each part keeps its run's order; its offset and numel are clipped to the
    window and its gradient address (0 stays 0) is advanced to the part's
    first element (``grad_esize`` bytes per element)."""
    off = runs["offset"]
    end = off + runs["numel"]
    part = runs[(runs["numel"] > 0) & (end > lo) & (off < hi) & (lo < hi)].copy()
    a = np.maximum(part["offset"], lo)
    b = np.minimum(part["offset"] + part["numel"], hi)
    moved = part["grad"] + ((a - part["offset"]) * grad_esize).astype(np.uint64)
    part["grad"] = np.where(part["grad"] != 0, moved, np.uint64(0))
    part["offset"] = a
    part["numel"] = b - a
    return part


class _Arena:
    """W equally laid-out rows (one per replica) of one symmetric allocation."""

    __slots__ = ("data", "numel", "row_elems", "dtype", "own_base", "esize", "row_ptrs", "target")

    def __init__(self, world: int, rank: int, numel: int, dtype: torch.dtype, device: torch.device):
        esize = torch.empty((), dtype=dtype).element_size()
        align = _ROW_ALIGN_BYTES // esize
        self.row_elems = max(align, (numel + align - 1) // align * align)
        self.data = torch.zeros((world, self.row_elems), dtype=dtype, device=device)
        self.numel = numel
        self.dtype = dtype
        self.esize = esize
        self.own_base = self.data[rank].data_ptr()
        self.row_ptrs = [self.data[r].data_ptr() for r in range(world)]
        self.target: torch.Tensor | None = None  # where SUM all-reduces write (None: this rank's row)

    def row(self, r: int) -> torch.Tensor:
        return self.data[r, : self.numel]

    def offset_of(self, t: torch.Tensor) -> int | None:
        p = _address(t)
        off, rem = divmod(p - self.own_base, self.esize)
        if rem or off < 0 or off + t.numel() > self.numel or t.dtype != self.dtype:
            return None
        return off


class ResidentGroup:
    """A data-parallel group of ``world_size`` replicas emulated on one GPU.

    Rank ``rank`` is the live replica driven by this process.  Its peers exist
    as their *contributions* -- what would arrive over xGMI from the other
    GPUs -- held in symmetric buffers: :meth:`zeros` allocates one row per
    replica and hands back this rank's row; :meth:`replicas` returns the W
    rows for any view of such a buffer (this rank's view at index ``rank``).
    Whoever stages an emulated step writes the peers' rows; the collectives
    then reduce over all W rows with the gfx950 kernels, in rank order.

    The group plays the role of a process group everywhere minidist takes one
    (``comm.get_world_size(group)`` is ``world_size``).  There is no
    inter-GPU traffic and no second process.
    """

    def __init__(self, world_size: int, rank: int = 0, device: torch.device | str | None = None):
        if not 1 <= world_size <= _native.MDX_MAX_WORLD:
            raise ValueError(f"world_size must be in [1, {_native.MDX_MAX_WORLD}], got {world_size}")
        if not 0 <= rank < world_size:
            raise ValueError(f"rank {rank} outside [0, {world_size})")
        self._world = world_size
        self._rank = rank
        self.device = torch.device(device) if device is not None else current_device()
        self._arenas: list[_Arena] = []

    def size(self) -> int:
        return self._world

    def rank(self) -> int:
        return self._rank

    def __repr__(self) -> str:
        return f"ResidentGroup(world_size={self._world}, rank={self._rank}, device={self.device})"

    # -- symmetric memory ---------------------------------------------------

    def zeros(self, numel: int, dtype: torch.dtype) -> torch.Tensor:
        """This rank's row of a new zero-filled symmetric buffer of ``numel`` elements."""
        arena = _Arena(self._world, self._rank, numel, dtype, self.device)
        self._arenas.append(arena)
        return arena.row(self._rank)

    def _rows_of(self, t: torch.Tensor) -> list[int]:
        """Every rank's address of ``t``'s elements in its row (``t`` lies in a symmetric buffer)."""
        if not t.is_contiguous():
            raise RuntimeError("a collective's symmetric-buffer operand must be contiguous")
        arena, off = self._locate(t)
        return [p + off * arena.esize for p in arena.row_ptrs]

    def row_addresses(self, row: torch.Tensor) -> list[int]:
        """Every rank's address of the row that :meth:`zeros` returned as ``row`` (rank order)."""
        arena, off = self._locate(row)
        if off != 0:
            raise ValueError("row_addresses takes the row that zeros() returned")
        return list(arena.row_ptrs)

    def _locate(self, t: torch.Tensor) -> tuple[_Arena, int]:
        for arena in self._arenas:
            off = arena.offset_of(t)
            if off is not None:
                return arena, off
        raise RuntimeError(
            "tensor is not part of a symmetric buffer of this ResidentGroup "
            "(allocate collective buffers with ResidentGroup.zeros)"
        )

    def replicas(self, t: torch.Tensor) -> list[torch.Tensor]:
        """The W replicas' copies of ``t`` (index ``rank`` is ``t``'s own memory)."""
        arena, off = self._locate(t)
        n = t.numel()
        return [arena.data[r, off : off + n].view(t.shape) for r in range(self._world)]

    def release(self) -> None:
        """Drop every symmetric buffer (views handed out keep their memory alive)."""
        self._arenas.clear()

    def set_reduce_target(self, row: torch.Tensor, target: torch.Tensor) -> None:
        """Make SUM all-reduces of ``row``'s symmetric buffer write into ``target``.

        ``row`` is this rank's row as :meth:`zeros` returned it; ``target`` has
        its dtype and at least its length, and receives the sum at the same
        element offsets, while the row keeps this rank's contribution -- what
        the peers read, which a real group could not overwrite while they still
        read it.  DDP registers each bucket buffer as the target of its
        contribution rows, so the reference's sequence ``gather_into_buffer``
        -> ``comm.all_reduce`` -> ``scatter_from_buffer`` ends in the same state
        as DDP's fused launch: the packed contribution in the row, the average
        in the bucket."""
        arena, off = self._locate(row)
        if off != 0 or row.numel() != arena.numel:
            raise ValueError("set_reduce_target takes the whole row that zeros() returned")
        _native.require_device_tensor(target, "all_reduce target")
        if target.dtype != arena.dtype or target.numel() < arena.numel:
            raise ValueError("the reduce target must have the row's dtype and at least its length")
        arena.target = target

    # -- collectives ----------------------------------------------------------

    def all_reduce_sum(self, tensors: Sequence[torch.Tensor], async_op: bool = False):
        """SUM over the W replicas of each tensor, rank order 0..W-1.

        In place, or into the buffer's reduce target when one is registered
        (:meth:`set_reduce_target`).  Tensors living in the same symmetric
        buffer are reduced by one dispatch (the runs must be in increasing
        offset order, as DDP's buckets are)."""
        if not tensors:
            return None
        device = tensors[0].device
        stream = _native.current_stream(device)
        groups: dict[int, tuple[_Arena, list[int], list[int]]] = {}
        for t in tensors:
            _native.require_device_tensor(t, "all_reduce input")
            arena, off = self._locate(t)
            entry = groups.setdefault(id(arena), (arena, [], []))
            entry[1].append(off)
            entry[2].append(t.numel())
        for arena, offs, nums in groups.values():
            order = sorted(range(len(offs)), key=offs.__getitem__)
            bases = arena.row_ptrs
            _native.allreduce_sum(
                bases,
                _native.dtype_code(arena.dtype),
                [offs[i] for i in order],
                [nums[i] for i in order],
                arena.own_base if arena.target is None else arena.target.data_ptr(),
                stream.cuda_stream,
            )
        return StreamWork(stream) if async_op else None

    def all_reduce_op(self, tensors: Sequence[torch.Tensor], op: int, async_op: bool = False):
        """:meth:`all_reduce_sum` with the reduction ``op`` (``_native.MDX_OP_*``): every element
        folded over the W replicas in rank order with torch's maximum / minimum / mul, in place or
        into the buffer's reduce target (``mdx_allreduce_op``, one dispatch per symmetric buffer)."""
        if op == _native.MDX_OP_SUM:
            return self.all_reduce_sum(tensors, async_op)
        if not tensors:
            return None
        stream = _native.current_stream(tensors[0].device)
        groups: dict[int, tuple[_Arena, list[int], list[int]]] = {}
        for t in tensors:
            _native.require_device_tensor(t, "all_reduce input")
            arena, off = self._locate(t)
            entry = groups.setdefault(id(arena), (arena, [], []))
            entry[1].append(off)
            entry[2].append(t.numel())
        for arena, offs, nums in groups.values():
            order = sorted(range(len(offs)), key=offs.__getitem__)
            _native.allreduce_op(
                arena.row_ptrs, _native.dtype_code(arena.dtype), op, [offs[i] for i in order],
                [nums[i] for i in order], arena.own_base if arena.target is None else arena.target.data_ptr(),
                stream.cuda_stream,
            )
        return StreamWork(stream) if async_op else None

    def all_reduce_unpack(
        self,
        buffer: torch.Tensor,
        runs,
        grad_dtype: torch.dtype,
        inv_scale: float = 1.0,
        found_inf: torch.Tensor | None = None,
        async_op: bool = False,
        bucket: torch.Tensor | None = None,
    ):
        """SUM over the W replicas of ``buffer``'s runs, delivered into gradients.

        ``runs`` is an ``mdx_grad_run`` table (numpy, ``_native.GRAD_RUN_DTYPE``)
        of (offset into ``buffer``, numel, gradient address) in increasing
        offset order.  The sum is written into ``bucket`` (same offsets and
        dtype as ``buffer``; default ``buffer`` itself, the in-place
        all-reduce) and, converted to ``grad_dtype``, multiplied by
        ``inv_scale`` and checked for inf/NaN into ``found_inf``, into each
        gradient -- one dispatch, the reduced values never re-read."""
        _native.require_device_tensor(buffer, "all_reduce input")
        arena, off = self._locate(buffer)
        esize = arena.esize
        bases = [b + off * esize for b in arena.row_ptrs]
        out = self._bucket_out(buffer, bucket)
        stream = _native.current_stream(buffer.device)
        _native.allreduce_unpack(
            bases, _native.dtype_code(arena.dtype), runs, out, _native.dtype_code(grad_dtype),
            _native.f32(inv_scale), found_inf.data_ptr() if found_inf is not None else None,
            stream.cuda_stream,
        )
        return StreamWork(stream) if async_op else None

    def all_reduce_unpack_wide(
        self,
        wire: torch.Tensor,
        bucket: torch.Tensor,
        runs,
        grad_dtype: torch.dtype,
        prescale: float,
        inv_scale: float = 1.0,
        found_inf: torch.Tensor | None = None,
        async_op: bool = False,
    ):
        """:meth:`all_reduce_unpack` for contributions narrower than the bucket.

        ``wire`` is this rank's row of bf16 or fp16 contributions (a symmetric
        buffer); every replica's element is widened to fp32 and multiplied by
        ``prescale`` where it is read, the W values are summed in rank order
        into ``bucket`` (fp32, same element offsets as ``wire``) and unpacked
        into the gradients of ``runs``."""
        _native.require_device_tensor(wire, "all_reduce input")
        _native.require_device_tensor(bucket, "all_reduce output")
        arena, off = self._locate(wire)
        if bucket.numel() < wire.numel():
            raise ValueError("all_reduce: the bucket is shorter than the contribution rows")
        bases = [b + off * arena.esize for b in arena.row_ptrs]
        stream = _native.current_stream(wire.device)
        _native.allreduce_unpack_wide(
            bases, _native.dtype_code(arena.dtype), runs, bucket.data_ptr(), _native.dtype_code(bucket.dtype),
            _native.dtype_code(grad_dtype), _native.f32(prescale), _native.f32(inv_scale),
            found_inf.data_ptr() if found_inf is not None else None, stream.cuda_stream,
        )
        return StreamWork(stream) if async_op else None

    @staticmethod
    def _bucket_out(buffer: torch.Tensor, bucket: torch.Tensor | None) -> int:
        """Address the fused all-reduce writes the sum to: ``bucket``, or ``buffer`` in place."""
        if bucket is None:
            return buffer.data_ptr()
        _native.require_device_tensor(bucket, "all_reduce output")
        if bucket.dtype != buffer.dtype or bucket.numel() < buffer.numel():
            raise ValueError("all_reduce: the bucket must have the contributions' dtype and at least their length")
        return bucket.data_ptr()

    def plan_all_reduce_unpack(
        self, buffer: torch.Tensor, runs, grad_dtype: torch.dtype, bucket: torch.Tensor | None = None
    ) -> "_native.Plan":
        """Device plan of :meth:`all_reduce_unpack` for fixed ``runs`` (one dispatch per launch)."""
        _native.require_device_tensor(buffer, "all_reduce input")
        arena, off = self._locate(buffer)
        bases = [b + off * arena.esize for b in arena.row_ptrs]
        return _native.plan_allreduce_unpack(
            bases, _native.dtype_code(arena.dtype), runs, self._bucket_out(buffer, bucket),
            _native.dtype_code(grad_dtype), buffer.device,
        )

    def plan_all_reduce_unpack_wide(
        self, wire: torch.Tensor, bucket: torch.Tensor, runs, grad_dtype: torch.dtype, prescale: float
    ) -> "_native.Plan":
        """Device plan of a widening fused all-reduce + unpack.

        ``wire`` is this rank's row of bf16 or fp16 contributions (a
        symmetric buffer); every replica's element is widened to fp32 and multiplied by
        ``prescale`` where it is read, the W values are summed in rank order
        into ``bucket`` (fp32, same element offsets as ``wire``) and unpacked
        into the gradients of ``runs``."""
        _native.require_device_tensor(wire, "all_reduce input")
        _native.require_device_tensor(bucket, "all_reduce output")
        arena, off = self._locate(wire)
        bases = [b + off * arena.esize for b in arena.row_ptrs]
        if bucket.numel() < wire.numel():
            raise ValueError("all_reduce: the bucket is shorter than the contribution rows")
        return _native.plan_allreduce_unpack_wide(
            bases, _native.dtype_code(arena.dtype), runs, bucket.data_ptr(), _native.dtype_code(bucket.dtype),
            _native.dtype_code(grad_dtype), _native.f32(prescale), wire.device,
        )

    def all_reduce_unpack_planned(
        self, plan: "_native.Plan", device: torch.device, inv_scale: float = 1.0,
        found_inf: torch.Tensor | None = None, async_op: bool = False,
    ):
        """Launch a plan from :meth:`plan_all_reduce_unpack` on the current stream."""
        _native.allreduce_unpack_planned(
            plan, _native.f32(inv_scale), found_inf.data_ptr() if found_inf is not None else None,
            _native.stream_of(device),
        )
        return StreamWork(_native.current_stream(device)) if async_op else None

    def pack_all_reduce_unpack(
        self,
        wire: torch.Tensor,
        bucket: torch.Tensor | None,
        runs,
        scale: float,
        inv_scale: float = 1.0,
        found_inf: torch.Tensor | None = None,
        clear_flag: torch.Tensor | None = None,
        async_op: bool = False,
        reduce_dtype: torch.dtype | None = None,
    ):
        """Pack this rank's gradients into its row of ``wire``, then SUM over the W rows into gradients.

        ``runs`` is an ``mdx_pack_run`` table (``_native.PACK_RUN_DTYPE``) of
        (offset into ``wire``, numel, gradient source or 0, gradient) in
        increasing offset order; gradients have ``wire``'s dtype.  Each source
        is packed as ``gather_into_buffer`` would (times ``scale`` = 1/W for a
        bucket of the wire dtype; raw into a bf16 / fp16 wire of an fp32
        ``bucket``, then every contribution times ``scale`` where it is
        widened); the rank-ordered sum lands in ``bucket`` (when given) and,
        times ``inv_scale`` and checked into ``found_inf``, in every gradient.
        ``clear_flag`` is set to 0 by the same dispatch (the scaler's flag for
        the next step).  One dispatch; this rank's contribution is summed from
        registers, not re-read from its row.  Without a ``bucket`` nothing is
        written besides the row and the gradients; ``reduce_dtype`` (default:
        the bucket's, else the wire's) is then the dtype the sum is taken in."""
        _native.require_device_tensor(wire, "all_reduce input")
        arena, off = self._locate(wire)
        bases = [b + off * arena.esize for b in arena.row_ptrs]
        reduce_dtype = _fused_reduce_dtype(wire, bucket, reduce_dtype)
        if bucket is not None:
            _native.require_device_tensor(bucket, "all_reduce output")
            if bucket.numel() < wire.numel():
                raise ValueError("all_reduce: the bucket is shorter than the contribution rows")
        stream = _native.current_stream(wire.device)
        _native.pack_allreduce_unpack(
            bases, self._rank, _native.dtype_code(arena.dtype), runs,
            None if bucket is None else bucket.data_ptr(), _native.dtype_code(reduce_dtype), _native.f32(scale),
            _native.f32(inv_scale), found_inf.data_ptr() if found_inf is not None else None,
            clear_flag.data_ptr() if clear_flag is not None else None, stream.cuda_stream,
        )
        return StreamWork(stream) if async_op else None

    def plan_pack_all_reduce_unpack(
        self, wire: torch.Tensor, bucket: torch.Tensor | None, runs, scale: float,
        reduce_dtype: torch.dtype | None = None,
    ) -> "_native.Plan":
        """Device plan of :meth:`pack_all_reduce_unpack` for fixed ``runs`` (one dispatch per launch)."""
        _native.require_device_tensor(wire, "all_reduce input")
        arena, off = self._locate(wire)
        bases = [b + off * arena.esize for b in arena.row_ptrs]
        reduce_dtype = _fused_reduce_dtype(wire, bucket, reduce_dtype)
        if bucket is not None:
            _native.require_device_tensor(bucket, "all_reduce output")
            if bucket.numel() < wire.numel():
                raise ValueError("all_reduce: the bucket is shorter than the contribution rows")
        return _native.plan_pack_allreduce_unpack(
            bases, self._rank, _native.dtype_code(arena.dtype), runs,
            None if bucket is None else bucket.data_ptr(), _native.dtype_code(reduce_dtype), _native.f32(scale),
            wire.device,
        )

    def pack_all_reduce_unpack_planned(
        self, plan: "_native.Plan", device: torch.device, inv_scale: float = 1.0,
        found_inf: torch.Tensor | None = None, clear_flag: torch.Tensor | None = None, async_op: bool = False,
    ):
        """Launch a plan from :meth:`plan_pack_all_reduce_unpack` on the current stream."""
        _native.pack_allreduce_unpack_planned(
            plan, _native.f32(inv_scale), found_inf.data_ptr() if found_inf is not None else None,
            clear_flag.data_ptr() if clear_flag is not None else None, _native.stream_of(device),
        )
        # the Work's stream object is found after the launch, off the path to the GPU
        return StreamWork(_native.current_stream(device)) if async_op else None

    def reduce_scatter_op(self, output: torch.Tensor, input_: torch.Tensor, op: int, async_op: bool = False):
        """:meth:`reduce_scatter_sum` with the reduction ``op`` (``_native.MDX_OP_*``): this rank's
        slice of the W replicas folded in rank order (``mdx_allreduce_op`` over the slices)."""
        if op == _native.MDX_OP_SUM:
            return self.reduce_scatter_sum(output, input_, async_op)
        _native.require_device_tensor(input_, "reduce_scatter input")
        rows = self._rows_of(input_)
        S = output.numel()
        if input_.numel() != S * self._world:
            raise ValueError(f"reduce_scatter: input has {input_.numel()} elements, expected {S * self._world}")
        if output.dtype != input_.dtype:
            raise TypeError("reduce_scatter: output and input dtypes differ")
        _native.require_dense(output, "reduce_scatter output")
        lo = self._rank * S * input_.element_size()
        stream = _native.current_stream(input_.device)
        _native.allreduce_op([r + lo for r in rows], _native.dtype_code(input_.dtype), op, [0], [S],
                             output.data_ptr(), stream.cuda_stream)
        return StreamWork(stream) if async_op else None

    def reduce_scatter_sum(self, output: torch.Tensor, input_: torch.Tensor, async_op: bool = False):
        """``output = sum_r replicas(input_)[r][rank*S:(rank+1)*S]``, rank order."""
        _native.require_device_tensor(input_, "reduce_scatter input")
        rows = self._rows_of(input_)
        S = output.numel()
        if input_.numel() != S * self._world:
            raise ValueError(f"reduce_scatter: input has {input_.numel()} elements, expected {S * self._world}")
        if output.dtype != input_.dtype:
            raise TypeError("reduce_scatter: output and input dtypes differ")
        _native.require_dense(output, "reduce_scatter output")
        lo = self._rank * S * input_.element_size()
        peers = [r + lo for r in rows]
        own = _native.pieces_array([(peers[self._rank], 0, S)])
        code = _native.dtype_code(input_.dtype)
        stream = _native.current_stream(input_.device)
        _native.reduce_scatter_share(
            own, peers, self._rank, code, code, False, output.data_ptr(), code, False, 1.0, None,
            stream.cuda_stream,
        )
        return StreamWork(stream) if async_op else None

    def all_gather_into(self, output: torch.Tensor, input_: torch.Tensor, async_op: bool = False):
        """``output[r*S:(r+1)*S] = replicas(input_)[r]`` for every rank r."""
        _native.require_device_tensor(input_, "all_gather input")
        _native.require_dense(output, "all_gather output")
        rows = self._rows_of(input_)
        S = input_.numel()
        if output.numel() != S * self._world or output.dtype != input_.dtype:
            raise ValueError("all_gather: output must hold world_size inputs of the same dtype")
        es, base = input_.element_size(), output.data_ptr()
        spans = self._gather_order([(rows[r], base + r * S * es, S) for r in range(self._world)], es)
        code = _native.dtype_code(input_.dtype)
        stream = _native.current_stream(input_.device)
        _native.pack(_native.spans_array(spans), code, code, 1.0, False, stream.cuda_stream)
        return StreamWork(stream) if async_op else None

    @staticmethod
    def _gather_order(spans: list[tuple[int, int, int]], esize: int) -> list[tuple[int, int, int]]:
        """The order a gather copies its spans in (the rows are all local here: as given)."""
        return spans


def _fused_reduce_dtype(wire: torch.Tensor, bucket: torch.Tensor | None, reduce_dtype: torch.dtype | None):
    """The dtype a fused pack + all-reduce sums in: the given one, else the bucket's, else the wire's."""
    if reduce_dtype is None:
        return wire.dtype if bucket is None else bucket.dtype
    if bucket is not None and bucket.dtype != reduce_dtype:
        raise TypeError(f"all_reduce: a {bucket.dtype} bucket cannot hold a {reduce_dtype} sum")
    return reduce_dtype


class _HostFence:
    """A barrier of the processes of one host, in POSIX shared memory.

    Each rank owns one 64-byte line: its epoch and two payload slots of three
    int64, used in alternate epochs.  A rank entering barrier ``e`` writes its
    payload into slot ``e % 2``, then ``e`` into its epoch, and spins until
    every rank's epoch reaches ``e`` (yielding its core once the wait is long,
    sleeping between checks after a millisecond, failing after ``timeout_s``);
    a rank can be at most one barrier ahead
    of the slowest (it cannot pass the next one alone), so the other slot still
    holds what the slowest rank reads.  Stores of aligned 8-byte words are
    single instructions and x86 keeps stores in program order, so a peer that
    sees the epoch also sees the payload written before it.  No kernel waits
    on a host flag: only the host threads of the group spin.

    Rank 0 creates the segment and unlinks its name once every rank has mapped
    it, so nothing is left in /dev/shm whatever happens to the processes."""

    LINE = 8  # int64 words per rank: epoch, payload slot 0 (3), payload slot 1 (3), pad
    PAYLOAD = 3

    def __init__(self, process_group, world: int, rank: int, timeout_s: float = 120.0):
        self._world, self._rank, self._timeout = world, rank, timeout_s
        size = world * self.LINE * 8
        path, mapped = None, None
        if rank == 0:
            try:
                path = os.path.join(self.SHM_DIR, f"mdx_fence_{uuid.uuid4().hex[:16]}")
                mapped = self._map(path, size, create=True)
            except OSError:
                path, mapped = None, None
        names: list = [None] * world
        dist.all_gather_object(names, (path, os.uname().nodename), group=process_group)
        usable = names[0][0] is not None and len({host for _, host in names}) == 1
        if usable and mapped is None:
            try:
                mapped = self._map(names[0][0], size, create=False)
            except OSError:
                mapped = None
        # every rank has mapped the segment, or the group falls back together
        ok: list = [None] * world
        dist.all_gather_object(ok, usable and mapped is not None, group=process_group)
        if rank == 0 and path is not None:
            os.unlink(path)  # the mappings stay; the name goes
        if not all(ok):
            if mapped is not None:
                mapped.close()
            raise RuntimeError("no shared host memory for the group's fences")
        self._mem = mapped
        self._lines = np.ndarray((world, self.LINE), dtype=np.int64, buffer=mapped)
        self._epoch = 0

    SHM_DIR = "/dev/shm"

    @staticmethod
    def _map(path: str, size: int, create: bool) -> mmap.mmap:
        flags = os.O_RDWR | (os.O_CREAT | os.O_EXCL if create else 0)
        fd = os.open(path, flags, 0o600)
        try:
            if create:
                os.ftruncate(fd, size)  # zero-filled
            return mmap.mmap(fd, size)
        finally:
            os.close(fd)

    def wait(self, payload: Sequence[int] | None = None) -> np.ndarray | None:
        """Meet every rank; with ``payload`` (up to three ints), return every rank's, rank order."""
        self._epoch += 1
        e, slot = self._epoch, 1 + (self._epoch % 2) * self.PAYLOAD
        line = self._lines[self._rank]
        if payload is not None:
            line[slot : slot + len(payload)] = payload
        line[0] = e
        epochs = self._lines[:, 0]
        spins, since = 0, None
        while (epochs < e).any():
            spins += 1
            if spins <= 2000:  # the peers are a few µs away: keep checking
                continue
            # a peer is further behind: give the core away, and after a millisecond sleep between checks
            now = time.monotonic()
            if since is None:
                since = now
            elif now - since > self._timeout:
                late = [r for r in range(self._world) if epochs[r] < e]
                raise RuntimeError(f"IpcGroup: ranks {late} did not reach host barrier {e} "
                                   f"within {self._timeout:.0f} s")
            if now - since > 1e-3:
                time.sleep(2e-5)
            else:
                os.sched_yield()
        if payload is None:
            return None
        return self._lines[:, slot : slot + len(payload)].copy()

    def close(self) -> None:
        self._lines = None
        self._mem.close()


class _IpcArena:
    """One symmetric buffer of an :class:`IpcGroup`: this rank's row is a tensor of its own;
    the peers' rows are inside their allocations, mapped into this process over IPC."""

    __slots__ = ("own", "pool", "numel", "dtype", "esize", "own_base", "row_ptrs", "target")

    def __init__(self, own: torch.Tensor, numel: int, row_ptrs: list[int], pool=None):
        self.own = own
        self.pool = pool  # the row's own memory pool: it lives as long as the row
        self.numel = numel
        self.dtype = own.dtype
        self.esize = own.element_size()
        self.own_base = own.data_ptr()
        self.row_ptrs = row_ptrs
        self.target: torch.Tensor | None = None

    def offset_of(self, t: torch.Tensor) -> int | None:
        p = _address(t)
        off, rem = divmod(p - self.own_base, self.esize)
        if rem or off < 0 or off + t.numel() > self.numel or t.dtype != self.dtype:
            return None
        return off


class IpcGroup(ResidentGroup):
    """W processes of a real process group whose contribution rows are mapped into each other.

    The multi-GPU design of this path, runnable here with W processes sharing
    the one GPU: each rank allocates its row of every symmetric buffer
    (:meth:`zeros`, each row an allocation below 2 GiB), exports it over IPC,
    and maps its peers' rows.  DDP and FSDP keep every symmetric buffer within
    ``segment_bytes`` (a model's buckets or units spread over several buffers
    when they need more).  The all-reduces run one of two ways
    (``algorithm``), both with the same rank-ordered kernels a
    :class:`ResidentGroup` uses, so every rank ends with bit-identical
    results.  The reference hands each bucket to ``dist.all_reduce`` instead
    (minidist/comm.py:223-234).

    * ``"one_shot"``: each rank reads all W rows and computes the whole result
      itself -- (W-1) rows pulled per rank, one exchange round.
    * ``"two_shot"``: each rank reduces its 1/W share of the extent from all W
      rows into its reduce target (the bucket), then copies the peers' reduced
      shares out of their targets while unpacking -- 2(W-1)/W of a row pulled
      per rank, two rounds.  A reduce target must then be a symmetric buffer
      too (``symmetric_targets``); without one the sums replace the rows, which
      is safe in place because a rank's share of its own row is read by no peer
      in the first round.

    Ordering is the host's: before a reduction every rank has finished
    writing its row (stream synchronisation, then a barrier over
    ``process_group``), a two-shot reduction meets again once every share is
    reduced, and after it every rank has finished reading its peers' memory
    (the same again) before anyone writes a row again.  No kernel waits on a
    flag a peer sets.  The pack cannot be fused into the reduction (a rank's
    row must be complete before its peers read it), so DDP runs the
    two-dispatch pipeline over this group (``fuses_pack`` is False).
    ``process_group`` carries only host traffic: the handles and the barriers
    (gloo is enough).
    """

    fuses_pack = False
    ALGORITHMS = ("one_shot", "two_shot")

    def __init__(self, process_group=None, device: torch.device | str | None = None, algorithm: str = "one_shot",
                 segment_bytes: int = 1 << 30):
        if algorithm not in self.ALGORITHMS:
            raise ValueError(f"IpcGroup: algorithm must be one of {self.ALGORITHMS}, got {algorithm!r}")
        if not 0 < segment_bytes <= _native.IPC_MAX_ALLOC_BYTES // 2:
            raise ValueError(f"IpcGroup: segment_bytes must be in (0, {_native.IPC_MAX_ALLOC_BYTES // 2}], "
                             f"got {segment_bytes}")
        self.process_group = process_group
        self.algorithm = algorithm
        # A row is one allocation, exported whole; DDP and FSDP split their symmetric buffers
        # into segments of at most this many bytes (the runtime maps allocations below 2 GiB).
        self.segment_bytes = segment_bytes
        # Two-shot: peers read each rank's reduced share out of its reduce target, so DDP
        # allocates its buckets as symmetric buffers, and reductions run through the
        # kernel-argument tables (a share is a different slice of the runs on every rank).
        self.symmetric_targets = algorithm == "two_shot"
        self.plans_reductions = algorithm == "one_shot"
        self._released = False
        # A peer's allocation mapped into this process, by (rank, handle bytes): every row is
        # an allocation of its own, so one mapping per peer row, unmapped once.
        self._mapped: dict[tuple[int, bytes], int] = {}
        super().__init__(dist.get_world_size(process_group), dist.get_rank(process_group), device)
        # The fences between the steps of a collective: IPC maps memory between the processes of
        # one host, so they meet in shared memory rather than over the process group's transport.
        try:
            self._fence: _HostFence | None = _HostFence(process_group, self._world, self._rank)
        except (OSError, RuntimeError):
            self._fence = None  # the process group's own barrier

    def __repr__(self) -> str:
        return (f"IpcGroup(world_size={self._world}, rank={self._rank}, device={self.device}, "
                f"algorithm={self.algorithm!r})")

    # -- symmetric memory ---------------------------------------------------

    def zeros(self, numel: int, dtype: torch.dtype) -> torch.Tensor:
        """This rank's row of a new zero-filled symmetric buffer; every rank calls it in the
        same order with the same sizes (the rows are exchanged collectively)."""
        self._check_open()
        esize = torch.empty((), dtype=dtype).element_size()
        align = _ROW_ALIGN_BYTES // esize
        row_elems = max(align, (numel + align - 1) // align * align)
        # The row is an allocation of its own (a pool of its own whose blocks are never split):
        # what a peer maps is this row and nothing else, and its size never includes a cached
        # segment that the caching allocator would otherwise have carved the row from.
        pool = torch.cuda.MemPool(no_split=True)
        with torch.cuda.use_mem_pool(pool, device=self.device):
            own = torch.zeros(row_elems, dtype=dtype, device=self.device)
        torch.cuda.current_stream(self.device).synchronize()  # the zeros are in place before a peer maps the row
        try:
            handle = _native.ipc_export(own.data_ptr())
        except RuntimeError as exc:
            raise RuntimeError(
                f"IpcGroup.zeros: the {row_elems * esize}-byte row could not be exported (the runtime maps "
                f"allocations below {_native.IPC_MAX_ALLOC_BYTES} bytes: keep symmetric buffers within the "
                f"group's segment_bytes): {exc}"
            ) from exc
        raw: list = [None] * self._world
        dist.all_gather_object(raw, (handle.to_bytes(), row_elems, str(dtype)), group=self.process_group)
        # every kernel reads all W rows over this rank's extent: the rows must agree
        if any((n, d) != (row_elems, str(dtype)) for _, n, d in raw):
            raise RuntimeError(f"IpcGroup.zeros: the ranks asked for different buffers {[(n, d) for _, n, d in raw]}")
        row_ptrs = []
        for r in range(self._world):
            if r == self._rank:
                row_ptrs.append(own.data_ptr())
                continue
            h = _native.IpcHandle.from_bytes(raw[r][0])
            if h.offset + row_elems * esize > h.alloc_bytes:
                raise RuntimeError(f"IpcGroup.zeros: rank {r}'s row is not inside the allocation it exported")
            key = (r, bytes(h.bytes))
            base = self._mapped.get(key)
            if base is None:
                base = _native.ipc_open(h) - int(h.offset)
                self._mapped[key] = base
            row_ptrs.append(base + int(h.offset))
        arena = _IpcArena(own, numel, row_ptrs, pool)
        self._arenas.append(arena)
        return own[:numel]

    def replicas(self, t: torch.Tensor) -> list[torch.Tensor]:
        raise NotImplementedError("an IpcGroup's peer rows belong to other processes (only addresses are mapped)")

    def release(self) -> None:
        """Unmap every peer row (collective: no rank still reads a row when it is released)."""
        torch.cuda.current_stream(self.device).synchronize()
        self._barrier()
        for base in self._mapped.values():
            _native.ipc_close_base(base)
        self._mapped.clear()
        self._arenas.clear()
        # plans built over this group still hold the peers' (now unmapped) addresses
        self._released = True
        if self._fence is not None:
            self._fence.close()
            self._fence = None

    # -- the one-shot protocol ----------------------------------------------

    def _check_open(self) -> None:
        if self._released:
            raise RuntimeError("IpcGroup: the peers' rows were released; no collective can run over them")

    def _barrier(self) -> None:
        if self._fence is not None:
            self._fence.wait()
        else:
            dist.barrier(group=self.process_group)

    def rows_written(self) -> None:
        """Every rank's writes to its rows are complete (this one's: its stream is drained)."""
        self._check_open()
        torch.cuda.current_stream(self.device).synchronize()
        self._barrier()

    def rows_read(self) -> None:
        """Every rank has finished reading its peers' rows."""
        torch.cuda.current_stream(self.device).synchronize()
        self._barrier()

    def _one_shot(self, launch, async_op: bool):
        self.rows_written()
        launch()
        self.rows_read()
        return _CompletedWork() if async_op else None

    # -- the two-shot protocol ----------------------------------------------

    def set_reduce_target(self, row: torch.Tensor, target: torch.Tensor) -> None:
        if self.symmetric_targets:
            self._target_rows(target, row.dtype, row.numel())
        super().set_reduce_target(row, target)

    def _target_rows(self, target: torch.Tensor, dtype: torch.dtype, numel: int) -> list[int]:
        """Every rank's address of ``target``, a two-shot reduce target (a symmetric buffer)."""
        _native.require_device_tensor(target, "all_reduce output")
        if target.dtype != dtype or target.numel() < numel:
            raise ValueError("all_reduce: the reduce target must have the reduction's dtype and at least its length")
        if not target.is_contiguous():
            raise ValueError("all_reduce: the reduce target must be contiguous")
        try:
            return self._rows_of(target)
        except RuntimeError:
            raise ValueError(
                "a two-shot IpcGroup reduces into symmetric buffers (IpcGroup.zeros): "
                "the peers read each rank's reduced share from its target"
            ) from None

    @staticmethod
    def _runs_extent(runs: np.ndarray) -> tuple[int, int]:
        live = runs[runs["numel"] > 0]
        if len(live) == 0:
            return 0, 0
        return int(live["offset"].min()), int((live["offset"] + live["numel"]).max())

    def _runs_agreed(self, runs: np.ndarray) -> None:
        """:meth:`rows_written` of a two-shot reduction.  Its barrier carries the runs'
        signature (first element, end, a hash of every run's offset and length), and every
        rank checks that all the others handed in the same -- each reduces its share of the
        runs for all the others.  Over the process group's own barrier the same check is a
        MAX of the signature and of its negation."""
        self._check_open()
        torch.cuda.current_stream(self.device).synchronize()
        live = runs[runs["numel"] > 0]
        lo, hi = self._runs_extent(runs)
        # tuples of ints hash the same in every process (no per-process salt)
        sig = hash(tuple(zip(live["offset"].tolist(), live["numel"].tolist()))) & ((1 << 62) - 1)
        mine = [lo, hi, sig]
        if self._fence is not None:
            agreed = bool((self._fence.wait(mine) == np.array(mine, dtype=np.int64)).all())
        else:
            both = torch.tensor(mine + [-x for x in mine], dtype=torch.int64)
            dist.all_reduce(both, op=dist.ReduceOp.MAX, group=self.process_group)
            agreed = [int(x) for x in both[:3]] == [-int(x) for x in both[3:]]
        if not agreed:
            raise RuntimeError(f"IpcGroup two-shot: the ranks reduce different runs (this rank: elements "
                               f"[{lo}, {hi}) in {len(live)} runs)")

    def _two_shot(self, runs: np.ndarray, esize: int, outs: list[int], code: int, reduce_share, after_gather,
                  async_op: bool):
        """The two rounds over the extent of ``runs`` (an ``mdx_grad_run`` table) in targets
        ``outs`` (every rank's address of element 0, ``esize`` bytes per element):
        ``reduce_share(a, b)`` reduces this rank's share [a, b) from all W rows into its target;
        then the runs' elements in every peer's share are copied out of that peer's target into
        this rank's (one copy over all peers, in interleaved chunks), and
        ``after_gather(peer_shares)`` runs on the peers' [a, b) ranges."""
        lo, hi = self._runs_extent(runs)
        shares = two_shot_shares(lo, hi, self._world)
        me = self._rank
        self._runs_agreed(runs)  # every row is written, and every rank reduces these runs
        a, b = shares[me]
        if b > a:
            reduce_share(a, b)
        self.rows_written()  # every share is reduced (and no peer reads a row any more)
        peer_shares = [(j, a, b) for j, (a, b) in enumerate(shares) if j != me and b > a]
        spans = [(outs[j] + o * esize, outs[me] + o * esize, n)
                 for j, a, b in peer_shares for o, n, _ in clip_grad_runs(runs, a, b, 0).tolist()]
        if spans:
            stream = torch.cuda.current_stream(self.device).cuda_stream
            _native.pack(_native.spans_array(interleave_spans(spans, esize, esize)), code, code, 1.0, False, stream)
            after_gather([(a, b) for _, a, b in peer_shares])
        self.rows_read()  # no peer reads this rank's target any more
        return _CompletedWork() if async_op else None

    # -- collectives ----------------------------------------------------------

    def all_reduce_sum(self, tensors: Sequence[torch.Tensor], async_op: bool = False):
        """SUM over the W ranks' rows, rank order 0..W-1, into the buffer's reduce target.

        Without a target the sum replaces the rows' contents, as the reference's
        in-place ``dist.all_reduce`` does.  One-shot: a rank's row is still read
        by its peers while its own reduction runs, so the sums go to a private
        buffer first and are copied into the rows once every rank has read them.
        Two-shot: each rank reduces its share in place (no peer reads that part
        of its row in the first round) and copies the peers' reduced shares out
        of their rows in the second."""
        self._check_open()
        if self.algorithm == "two_shot":
            return self._all_reduce_sum_two_shot(tensors, async_op)
        return self._one_shot_all_reduce(tensors, lambda: ResidentGroup.all_reduce_sum(self, tensors), async_op)

    def all_reduce_op(self, tensors: Sequence[torch.Tensor], op: int, async_op: bool = False):
        """:meth:`ResidentGroup.all_reduce_op` over the mapped rows, one-shot whatever the group's
        algorithm (PRODUCT, MIN and MAX carry flags and small tensors)."""
        if op == _native.MDX_OP_SUM:
            return self.all_reduce_sum(tensors, async_op)
        self._check_open()
        return self._one_shot_all_reduce(tensors, lambda: ResidentGroup.all_reduce_op(self, tensors, op), async_op)

    def _one_shot_all_reduce(self, tensors: Sequence[torch.Tensor], reduce, async_op: bool):
        """``reduce()`` over the mapped rows between the fences; a buffer without a reduce target
        is reduced into a private copy first, copied into the rows once every rank has read them."""
        arenas = {id(a): a for a in (self._locate(t)[0] for t in tensors)}
        staged = [a for a in arenas.values() if a.target is None]
        for arena in staged:
            arena.target = torch.empty_like(arena.own)
        try:
            work = self._one_shot(reduce, async_op)
            for t in tensors:
                arena, off = self._locate(t)
                if arena in staged:
                    t.copy_(arena.target[off : off + t.numel()].view(t.shape))
        finally:
            for arena in staged:
                arena.target = None
        return work

    def _all_reduce_sum_two_shot(self, tensors: Sequence[torch.Tensor], async_op: bool):
        by_arena: dict[int, tuple[_IpcArena, list[tuple[int, int, int]]]] = {}
        for t in tensors:
            _native.require_device_tensor(t, "all_reduce input")
            arena, off = self._locate(t)
            by_arena.setdefault(id(arena), (arena, []))[1].append((off, t.numel(), 0))
        stream = torch.cuda.current_stream(self.device).cuda_stream
        work = None
        for arena, parts in by_arena.values():
            runs = _native.grad_runs_array(sorted(parts))
            rows = arena.row_ptrs
            outs = rows if arena.target is None else self._target_rows(arena.target, arena.dtype, arena.numel)
            code = _native.dtype_code(arena.dtype)

            def reduce_share(a, b, runs=runs, rows=rows, outs=outs, code=code):
                part = clip_grad_runs(runs, a, b, 0)
                _native.allreduce_sum(rows, code, part["offset"].tolist(), part["numel"].tolist(),
                                      outs[self._rank], stream)

            work = self._two_shot(runs, arena.esize, outs, code, reduce_share, lambda peer_shares: None, async_op)
        return work

    def all_reduce_unpack(self, buffer, runs, grad_dtype, inv_scale=1.0, found_inf=None, async_op=False,
                          bucket=None):
        """:meth:`ResidentGroup.all_reduce_unpack` over the mapped rows.  Two-shot: the
        fused reduction + unpack of this rank's share (its part of every gradient), then,
        for each peer, the same kernel over one replica -- the peer's reduced share in its
        bucket -- copied into this rank's bucket and unpacked into the rest of the gradients."""
        if self.algorithm == "one_shot":
            return self._one_shot(lambda: ResidentGroup.all_reduce_unpack(
                self, buffer, runs, grad_dtype, inv_scale, found_inf, bucket=bucket), async_op)
        self._check_open()
        _native.require_device_tensor(buffer, "all_reduce input")
        arena, off = self._locate(buffer)
        rows = [p + off * arena.esize for p in arena.row_ptrs]
        outs = rows if bucket is None else self._target_rows(bucket, buffer.dtype, buffer.numel())
        code = _native.dtype_code(arena.dtype)
        return self._two_shot_unpack(outs, runs, grad_dtype, inv_scale, found_inf, async_op,
                                     lambda part, out, gcode, inv, flag, st: _native.allreduce_unpack(
                                         rows, code, part, out, gcode, inv, flag, st), arena.dtype)

    def all_reduce_unpack_wide(self, wire, bucket, runs, grad_dtype, prescale, inv_scale=1.0, found_inf=None,
                               async_op=False):
        """:meth:`ResidentGroup.all_reduce_unpack_wide` over the mapped rows; two-shot as in
        :meth:`all_reduce_unpack`, the peers' reduced shares copied in the bucket dtype."""
        if self.algorithm == "one_shot":
            return self._one_shot(lambda: ResidentGroup.all_reduce_unpack_wide(
                self, wire, bucket, runs, grad_dtype, prescale, inv_scale, found_inf), async_op)
        self._check_open()
        _native.require_device_tensor(wire, "all_reduce input")
        arena, off = self._locate(wire)
        rows = [p + off * arena.esize for p in arena.row_ptrs]
        outs = self._target_rows(bucket, bucket.dtype, wire.numel())
        wcode, bcode, pre = _native.dtype_code(arena.dtype), _native.dtype_code(bucket.dtype), _native.f32(prescale)
        return self._two_shot_unpack(outs, runs, grad_dtype, inv_scale, found_inf, async_op,
                                     lambda part, out, gcode, inv, flag, st: _native.allreduce_unpack_wide(
                                         rows, wcode, part, out, bcode, gcode, pre, inv, flag, st), bucket.dtype)

    def _two_shot_unpack(self, outs, runs, grad_dtype, inv_scale, found_inf, async_op, reduce_unpack,
                         out_dtype: torch.dtype):
        out_code, osize = _native.dtype_code(out_dtype), torch.empty((), dtype=out_dtype).element_size()
        gcode, gsize = _native.dtype_code(grad_dtype), torch.empty((), dtype=grad_dtype).element_size()
        inv, flag = _native.f32(inv_scale), (found_inf.data_ptr() if found_inf is not None else None)
        stream = torch.cuda.current_stream(self.device).cuda_stream
        me = self._rank

        def unpack_peer_shares(peer_shares):
            # the copied sums -> the gradients they cover (the fused kernel's unpack epilogue)
            spans = [(outs[me] + o * osize, g, n) for a, b in peer_shares
                     for o, n, g in clip_grad_runs(runs, a, b, gsize).tolist()]
            if spans:
                _native.unpack(_native.spans_array(spans), out_code, gcode, inv, flag, stream)

        return self._two_shot(
            runs, osize, outs, out_code,
            lambda a, b: reduce_unpack(clip_grad_runs(runs, a, b, gsize), outs[me], gcode, inv, flag, stream),
            unpack_peer_shares, async_op,
        )

    def _one_shot_only(self, what: str) -> None:
        if self.algorithm != "one_shot":
            raise NotImplementedError(f"IpcGroup: {what} is one-shot only (a two-shot group reduces "
                                      "through kernel-argument tables: the shares differ from rank to rank)")

    def plan_all_reduce_unpack(self, *args, **kwargs):
        self._one_shot_only("plan_all_reduce_unpack")
        return super().plan_all_reduce_unpack(*args, **kwargs)

    def plan_all_reduce_unpack_wide(self, *args, **kwargs):
        self._one_shot_only("plan_all_reduce_unpack_wide")
        return super().plan_all_reduce_unpack_wide(*args, **kwargs)

    def all_reduce_unpack_planned(self, plan, device, inv_scale=1.0, found_inf=None, async_op=False):
        self._one_shot_only("all_reduce_unpack_planned")
        return self._one_shot(lambda: ResidentGroup.all_reduce_unpack_planned(
            self, plan, device, inv_scale, found_inf), async_op)

    def pack_all_reduce_unpack(self, *args, **kwargs):
        raise NotImplementedError("IpcGroup: a rank's row must be complete before its peers read it (no fused pack)")

    pack_all_reduce_unpack_planned = pack_all_reduce_unpack

    def reduce_scatter_sum(self, output, input_, async_op: bool = False):
        """``output`` = this rank's slice of the rank-ordered SUM of every rank's ``input_`` (a row
        of a symmetric buffer), read one-shot from the mapped rows."""
        self._check_open()
        return self._one_shot(lambda: ResidentGroup.reduce_scatter_sum(self, output, input_), async_op)

    def reduce_scatter_op(self, output, input_, op: int, async_op: bool = False):
        """:meth:`ResidentGroup.reduce_scatter_op` read one-shot from the mapped rows."""
        self._check_open()
        return self._one_shot(lambda: ResidentGroup.reduce_scatter_op(self, output, input_, op), async_op)

    @staticmethod
    def _gather_order(spans: list[tuple[int, int, int]], esize: int) -> list[tuple[int, int, int]]:
        """Peers' rows are read in interleaved chunks, so that one copy draws on every peer at once."""
        return interleave_spans(spans, esize, esize)

    def all_gather_into(self, output, input_, async_op: bool = False):
        """``output[r*S:(r+1)*S]`` = rank r's ``input_`` (a row of a symmetric buffer), copied
        one-shot from the mapped rows."""
        self._check_open()
        return self._one_shot(lambda: ResidentGroup.all_gather_into(self, output, input_), async_op)


def zeros_for_collective(numel: int, dtype: torch.dtype, device: torch.device, group=None) -> torch.Tensor:
    """A zero-filled flat buffer that ``group``'s collectives can operate on.

    For a :class:`ResidentGroup` this is this rank's row of a symmetric
    buffer; otherwise a plain ``torch.zeros`` (reference ddp.py:83-84)."""
    if isinstance(group, ResidentGroup):
        return group.zeros(numel, dtype)
    return torch.zeros(numel, dtype=dtype, device=device)


# --------------------------------------------------------------------------
# Instrumented collectives (reference comm.py:210-277)
# --------------------------------------------------------------------------


def _nbytes(t: torch.Tensor) -> int:
    return t.numel() * t.element_size()


# --------------------------------------------------------------------------
# torch.distributed calls of this package.  RCCL (and NCCL) collectives take
# device tensors as they are.  gloo moves host memory: a device tensor is
# copied to the host (a synchronous copy, which also waits for the kernels
# that produced it), the collective runs there synchronously, and the result
# is copied back in the current stream's order.  The Work returned for
# async_op is then already complete.
# --------------------------------------------------------------------------


class _CompletedWork:
    def wait(self, timeout=None) -> bool:
        return True

    def is_completed(self) -> bool:
        return True


def _via_host(tensor: torch.Tensor, group) -> bool:
    return tensor.is_cuda and dist.get_backend(group) == "gloo"


def dist_all_reduce(tensor: torch.Tensor, op=dist.ReduceOp.SUM, group=None, async_op: bool = False):
    if _via_host(tensor, group):
        host = tensor.cpu()
        dist.all_reduce(host, op=op, group=group)
        tensor.copy_(host)
        return _CompletedWork() if async_op else None
    return dist.all_reduce(tensor, op=op, group=group, async_op=async_op)


def dist_broadcast(tensor: torch.Tensor, src: int, group=None, async_op: bool = False):
    if _via_host(tensor, group):
        host = tensor.cpu()
        dist.broadcast(host, src=src, group=group)
        tensor.copy_(host)
        return _CompletedWork() if async_op else None
    return dist.broadcast(tensor, src=src, group=group, async_op=async_op)


def broadcast_module_state(module: torch.nn.Module, group=None, src: int = 0, buffer_filter=None) -> None:
    """A wrapper's construction-time sync: every parameter, then every buffer that
    ``buffer_filter`` accepts (all of them when it is None), from rank ``src`` of ``group``
    (of the default group: always rank 0).  ``dist.broadcast`` takes the source's global
    rank, so a group rank is translated first."""
    root = 0 if group is None else dist.get_global_rank(group, src)
    buffers = [b for b in module.buffers() if buffer_filter is None or buffer_filter(b)]
    with torch.no_grad():
        for t in (*module.parameters(), *buffers):
            dist_broadcast(t.data, src=root, group=group)


def dist_all_gather_into_tensor(output: torch.Tensor, input_: torch.Tensor, group=None, async_op: bool = False):
    if _via_host(output, group):
        host_out = torch.empty(output.shape, dtype=output.dtype)
        dist.all_gather_into_tensor(host_out, input_.cpu(), group=group)
        output.copy_(host_out)
        return _CompletedWork() if async_op else None
    return _all_gather_single(output, input_, group=group, async_op=async_op)


def dist_reduce_scatter_tensor(
    output: torch.Tensor, input_: torch.Tensor, op=dist.ReduceOp.SUM, group=None, async_op: bool = False
):
    if _via_host(output, group):
        host_out = torch.empty(output.shape, dtype=output.dtype)
        dist.reduce_scatter_tensor(host_out, input_.cpu(), op=op, group=group)
        output.copy_(host_out)
        return _CompletedWork() if async_op else None
    return _reduce_scatter_single(output, input_, op=op, group=group, async_op=async_op)


def _all_gather_single(*args, **kwargs):
    return (getattr(dist, "all_gather_single", None) or dist.all_gather_into_tensor)(*args, **kwargs)


def _reduce_scatter_single(*args, **kwargs):
    return (getattr(dist, "reduce_scatter_single", None) or dist.reduce_scatter_tensor)(*args, **kwargs)


def all_reduce(tensor: torch.Tensor, op=dist.ReduceOp.SUM, group=None, async_op: bool = False):
    world = get_world_size(group)
    if world == 1:
        return None
    record_all_reduce(_nbytes(tensor), world)
    if isinstance(group, ResidentGroup):
        return group.all_reduce_op([tensor], _resident_op(op, "all_reduce"), async_op=async_op)
    return dist_all_reduce(tensor, op=op, group=group, async_op=async_op)


def _resident_op(op, what: str) -> int:
    """The ``mdx_allreduce_op`` code of a ``dist.ReduceOp`` a ResidentGroup reduces with."""
    for red, code in ((dist.ReduceOp.SUM, _native.MDX_OP_SUM), (dist.ReduceOp.PRODUCT, _native.MDX_OP_PRODUCT),
                      (dist.ReduceOp.MIN, _native.MDX_OP_MIN), (dist.ReduceOp.MAX, _native.MDX_OP_MAX)):
        if op == red:
            return code
    raise NotImplementedError(f"ResidentGroup {what} implements SUM, PRODUCT, MIN and MAX, not {op}")


def all_reduce_coalesced(tensors: Sequence[torch.Tensor], group=None, async_op: bool = False):
    """SUM all-reduce of several tensors issued as one collective call.

    Same accounting as one :func:`all_reduce` per tensor.  A ResidentGroup
    reduces every tensor of one symmetric buffer in a single dispatch; a real
    group issues the per-tensor collectives back to back and returns the last
    Work (collectives on one communicator complete in order)."""
    world = get_world_size(group)
    if world == 1 or not tensors:
        return None
    for t in tensors:
        record_all_reduce(_nbytes(t), world)
    if isinstance(group, ResidentGroup):
        return group.all_reduce_sum(list(tensors), async_op=async_op)
    work = None
    for t in tensors:
        work = dist_all_reduce(t, group=group, async_op=async_op)
    return work


def all_gather_into_tensor(output: torch.Tensor, input_: torch.Tensor, group=None, async_op: bool = False):
    world = get_world_size(group)
    if world == 1:
        output.copy_(input_)
        return None
    payload = _nbytes(output)
    comm_stats.add("all_gather", payload, int((world - 1) / world * payload))
    if isinstance(group, ResidentGroup):
        return group.all_gather_into(output, input_, async_op=async_op)
    return dist_all_gather_into_tensor(output, input_, group=group, async_op=async_op)


def reduce_scatter_tensor(
    output: torch.Tensor, input_: torch.Tensor, op=dist.ReduceOp.SUM, group=None, async_op: bool = False
):
    world = get_world_size(group)
    if world == 1:
        output.copy_(input_)
        return None
    payload = _nbytes(input_)
    comm_stats.add("reduce_scatter", payload, int((world - 1) / world * payload))
    if isinstance(group, ResidentGroup):
        return group.reduce_scatter_op(output, input_, _resident_op(op, "reduce_scatter"), async_op=async_op)
    return dist_reduce_scatter_tensor(output, input_, op=op, group=group, async_op=async_op)


def broadcast(tensor: torch.Tensor, src: int, group=None, async_op: bool = False):
    if get_world_size(group) == 1:
        return None
    comm_stats.add("broadcast", _nbytes(tensor), _nbytes(tensor))
    if isinstance(group, ResidentGroup):
        return None  # peers are staged by the caller; nothing to send
    return dist_broadcast(tensor, src=src, group=group, async_op=async_op)
