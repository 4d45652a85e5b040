"""Fully Sharded Data Parallel (ZeRO-3): shard parameters, gradients and optimizer state.

A drop-in for the reference's minidist/fsdp.py.  What a caller can observe is
kept: the names and signatures (``MixedPrecisionPolicy`` :72-105,
``_FSDPUnit`` :108-244, ``FullyShardedDataParallel`` :247-504), the unit
partition (:315-357), the shard layout and padding (:130-161), the hook
order and semantics, the ``_flat_shard_{i}`` parameter names, the
``memory_summary`` keys and values and the error texts.  The machinery
underneath is this package's own:

* :func:`_partition` decides once which module owns which parameter;
* every unit registers (and removes) its own hooks, which reach the unit and
  the wrapper only through weak references (:class:`_UnitHooks`);
* the unit's two arithmetic steps run as gfx950 kernels:

  - ``unshard`` (:172-182): the fp32 master shard is cast to ``param_dtype``
    (bf16 or fp16, round-to-nearest-even) *straight into this rank's slot*
    of the gather buffer, so the all-gather needs no separate input; with a
    real process group the all-gather then runs in place, with a
    :class:`~minidist.comm.ResidentGroup` the peers' resident shards are
    copied into their slots by one multi-span dispatch;
  - ``reduce_scatter_grads`` (:215-241): with a ResidentGroup, one
    ``mdx_reduce_scatter_share`` dispatch reads this rank's slice of its own
    gradients straight from the ``p.grad`` tensors (no padded flat copy),
    the peers' slices from their resident full-size contributions, widens
    each to ``reduce_dtype``, divides by W, sums in rank order and writes --
    or accumulates into -- ``flat_shard.grad``.  Peers contribute their
    gradients in ``param_dtype`` (what they would send); widening is exact
    and the division is applied per contribution exactly as the reference's
    ``buf.div_(W)`` does, so the result is the reference's bit for bit;

* over a :class:`~minidist.comm.IpcGroup` (W processes) every rank
  publishes its shard and its full-size gradients in its rows of two
  symmetric buffers (per segment of units, within the group's
  ``segment_bytes``), and after a barrier copies the peers' shards from their
  mapped rows, or sums its slice of all W rows with the same share kernel;
* units that are ready together (``unit_batch``, ``summon_full_params``,
  the flush after ``no_sync``) go out as one multi-unit dispatch per step
  of the exchange;
* ``comm_streams=True`` moves every unit's gather onto one side stream and
  every reduce-scatter onto another (both default priority), ordered with
  events against the caller's stream, so that a unit's gather cast and
  another unit's reduce-scatter share -- which touch disjoint buffers -- run
  concurrently instead of each paying its own dispatch ramp and tail.
"""

from __future__ import annotations

import weakref
from collections.abc import Iterator, Sequence
from contextlib import contextmanager
from typing import NamedTuple

import torch
from torch import nn

from . import _native, comm

__all__ = ["FullyShardedDataParallel", "FSDP", "MixedPrecisionPolicy"]


class MixedPrecisionPolicy:
    """Dtypes for the gathered parameters, the gradient reduction, and the shard."""

    def __init__(
        self,
        param_dtype: torch.dtype = torch.float32,
        reduce_dtype: torch.dtype = torch.float32,
        keep_low_precision_shard: bool = False,
    ):
        self.param_dtype = param_dtype
        self.reduce_dtype = reduce_dtype
        self.keep_low_precision_shard = keep_low_precision_shard

    def __repr__(self) -> str:
        return f"MixedPrecisionPolicy(param={self.param_dtype}, reduce={self.reduce_dtype})"


def _copy_spans(rows, src_dtype: torch.dtype, dst_dtype: torch.dtype, device: torch.device) -> None:
    if rows:
        _native.pack(
            _native.spans_array(rows),
            _native.dtype_code(src_dtype),
            _native.dtype_code(dst_dtype),
            1.0,
            False,
            _native.stream_of(device),
        )


def _emulates_peers(group) -> bool:
    """A ResidentGroup whose peers are staged in this process (an IpcGroup's are processes)."""
    return isinstance(group, comm.ResidentGroup) and not isinstance(group, comm.IpcGroup)


def _check_grad(g: torch.Tensor) -> None:
    """A full-size gradient the kernels read as a flat span: on the GPU and dense."""
    _native.require_device_tensor(g, "FSDP gradient")
    if not g.is_contiguous():
        raise RuntimeError("FSDP gradient is not contiguous")


class _SideStreams:
    """The gather and reduce-scatter streams of one FSDP wrapper (default priority).

    Work enqueued on a side stream first waits for everything already on the
    caller's stream (the optimizer's update of a master shard, the backward
    kernels that produced a gradient).  The caller's stream waits for a
    unit's gather before the unit's parameters are read or freed
    (:meth:`_FSDPUnit.wait_gathered`), and for both side streams at the end
    of backward and in ``finish_gradient_sync`` (:meth:`join`).

    Tensors that side-stream work reads or writes but the caller may drop
    (a unit's full-size gradients, a fresh shard gradient) are held here
    until that work is known to be done -- its event has completed, or the
    caller's stream has joined -- rather than marked with ``record_stream``:
    on this stack every event the allocator would record on the side stream
    is a queue packet of its own between two dispatches."""

    __slots__ = ("device", "gather", "reduce", "_held")

    def __init__(self, device: torch.device):
        self.device = device
        self.gather = torch.cuda.Stream(device=device)
        self.reduce = torch.cuda.Stream(device=device)
        self._held: list[tuple[torch.cuda.Event | None, list[torch.Tensor]]] = []

    def run(self, stream: torch.cuda.Stream, work, keep: list[torch.Tensor] | None = None,
            event: bool = False) -> torch.cuda.Event | None:
        """``work()`` enqueued on ``stream`` after the caller's stream.

        ``keep``: tensors to hold until the work is done.  With ``event`` (or
        ``keep``) a completion event is recorded on ``stream``; it is returned
        when ``event`` is set."""
        stream.wait_stream(torch.cuda.current_stream(self.device))
        with torch.cuda.stream(stream):
            work()
        done = None
        if event or keep:
            done = torch.cuda.Event()
            done.record(stream)
        if keep:
            self._release_finished()
            self._held.append((done, keep))
        return done if event else None

    def _release_finished(self) -> None:
        self._held = [(ev, ts) for ev, ts in self._held if not ev.query()]

    def join(self) -> None:
        """Order the caller's stream after everything enqueued on both side streams."""
        current = torch.cuda.current_stream(self.device)
        current.wait_stream(self.reduce)
        current.wait_stream(self.gather)
        self._held.clear()  # later work on the caller's stream is ordered after their last use


class _IpcRows(NamedTuple):
    """A unit's blocks in the two symmetric buffers of an :class:`~minidist.comm.IpcGroup`:
    its padded full-size gradient and its gathered-dtype shard, as this rank's tensors and at
    every rank's (mapped) address."""

    grads: torch.Tensor
    grad_ptrs: list[int]
    shard: torch.Tensor
    shard_ptrs: list[int]


class _FSDPUnit:
    """One shard-gather-free granule: a module plus the parameters it owns."""

    def __init__(
        self,
        module: nn.Module,
        params: list[nn.Parameter],
        group,
        policy: MixedPrecisionPolicy,
        reshard_after_forward: bool,
        device: torch.device,
        name: str,
        peer_grads: torch.Tensor | None = None,
        arena_offset: int = 0,
    ):
        self.module = module
        self.params = params
        self.group = group
        self.policy = policy
        self.reshard_after_forward = reshard_after_forward
        self.name = name
        self.world = comm.get_world_size(group)
        self.rank = comm.get_rank(group)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise RuntimeError("minidist FSDP runs its shard arithmetic as HIP kernels; pass a GPU device")
        self.streams: _SideStreams | None = None  # set by the wrapper when it runs with comm_streams
        self._gathered: torch.cuda.Event | None = None  # the pending side-stream gather, if any

        self.shapes = [p.shape for p in params]
        self.numels = [p.numel() for p in params]
        self.total_numel = sum(self.numels)
        # Pad so the flat parameter divides evenly (fsdp.py:132-136).
        self.shard_numel = (self.total_numel + self.world - 1) // self.world
        self.padded_numel = self.shard_numel * self.world

        src_dtype = params[0].dtype
        shard_dtype = policy.param_dtype if policy.keep_low_precision_shard else src_dtype

        # Full flat parameter (pack kernel) in the first parameter's dtype, each parameter
        # converted as the reference's copy_ converts it; this rank's slice as the master shard.
        flat = torch.zeros(self.padded_numel, dtype=src_dtype, device=self.device)
        staged = [p.detach().to(self.device).contiguous() for p in params]
        by_dtype: dict[torch.dtype, list[tuple[int, int, int]]] = {}
        off = 0
        for t, n in zip(staged, self.numels, strict=True):
            by_dtype.setdefault(t.dtype, []).append((t.data_ptr(), flat.data_ptr() + off * flat.element_size(), n))
            off += n
        for dtype, rows in by_dtype.items():
            _copy_spans(rows, dtype, src_dtype, self.device)
        S, r0 = self.shard_numel, self.rank * self.shard_numel
        master = torch.empty(S, dtype=shard_dtype, device=self.device)
        _copy_spans([(flat[r0:].data_ptr(), master.data_ptr(), S)], src_dtype, shard_dtype, self.device)
        self.flat_shard = nn.Parameter(master)

        # Emulated peers (ResidentGroup): their gathered shards (what their
        # all-gather contributions carry) and their full-size gradients.
        self._peer_shards: torch.Tensor | None = None
        self._peer_grads: torch.Tensor | None = None
        self._ipc: _IpcRows | None = None  # set by the wrapper over an IpcGroup
        if _emulates_peers(group) and self.world > 1:
            # A peer's gathered shard is its master shard in param_dtype; the
            # master is either the init value (src dtype) or that value already
            # rounded to param_dtype, so one conversion of the init slice gives it.
            self._peer_shards = torch.zeros((self.world, S), dtype=policy.param_dtype, device=self.device)
            rows = [
                (flat[r * S :].data_ptr(), self._peer_shards[r].data_ptr(), S)
                for r in range(self.world)
                if r != self.rank
            ]
            _copy_spans(rows, src_dtype, policy.param_dtype, self.device)
            if peer_grads is None:
                peer_grads = torch.zeros((self.world, self.padded_numel), dtype=policy.param_dtype, device=self.device)
            elif peer_grads.shape != (self.world, self.padded_numel) or peer_grads.dtype != policy.param_dtype:
                raise ValueError("peer_grads must be a [world, padded_numel] view in param_dtype")
            self._peer_grads = peer_grads
        # element offset of this unit's padded block in the rows of the wrapper's shared
        # peer-gradient arena (the multi-unit share addresses every unit from one set of rows),
        # and which set of rows that is (several over an IpcGroup whose buffers are bounded)
        self.arena_offset = arena_offset
        self.segment = 0
        torch.cuda.current_stream(self.device).synchronize()
        del flat, staged

        # The gathered buffer; parameter views into it are assigned once.
        self._full = torch.empty(self.padded_numel, dtype=policy.param_dtype, device=self.device)
        offset = 0
        for p, n, shape in zip(params, self.numels, self.shapes, strict=True):
            p.data = self._full[offset : offset + n].view(shape)
            offset += n
        self._unsharded = True
        self.reshard()

        self._grads_pending = 0
        # set when this step's backward has completed the unit's gradients, cleared by the
        # next forward: a batched backward gather must not bring such a unit back
        self._backward_done = False
        self._hook_handles: list[torch.utils.hooks.RemovableHandle] = []

    # -- hooks ----------------------------------------------------------------

    def attach(self, hooks: _UnitHooks) -> None:
        """Register ``hooks`` on this unit's module and parameters.

        Order per unit, as the reference registers them (fsdp.py:359-377):
        forward pre-hook, forward hook, full backward pre-hook (only when the
        unit reshards after forward), then each trainable parameter's
        post-accumulate-grad hook."""
        m = self.module
        handles = [m.register_forward_pre_hook(hooks.before_forward), m.register_forward_hook(hooks.after_forward)]
        if self.reshard_after_forward:
            handles.append(m.register_full_backward_pre_hook(hooks.before_backward))
        handles += [p.register_post_accumulate_grad_hook(hooks.grad_ready) for p in self.params if p.requires_grad]
        self._hook_handles.extend(handles)

    # -- emulation staging ----------------------------------------------------

    def peer_param_shards(self) -> torch.Tensor:
        """[W, S] gathered-dtype shards of every rank (ResidentGroup; row ``rank`` unused)."""
        if self._peer_shards is None:
            raise RuntimeError("peer shards exist only under a ResidentGroup with world > 1")
        return self._peer_shards

    def peer_grad_contributions(self) -> torch.Tensor:
        """[W, padded] full-size gradients of every rank in ``param_dtype`` (row ``rank`` unused)."""
        if self._peer_grads is None:
            raise RuntimeError("peer gradients exist only under a ResidentGroup with world > 1")
        return self._peer_grads

    # -- shard / unshard ----------------------------------------------------

    @property
    def is_unsharded(self) -> bool:
        return self._unsharded

    def _on_gather_side(self, work) -> None:
        """Run ``work`` on the caller's stream, or on the gather stream with its event kept."""
        if self.streams is None:
            work()
            return
        self._gathered = self.streams.run(self.streams.gather, work, event=True)

    def _require_gathered_storage(self) -> None:
        if not self._unsharded:
            raise RuntimeError(f"FSDP unit {self.name}: the gather buffer is freed (the unit is sharded)")

    def _cast_own_slot_now(self) -> None:
        self._require_gathered_storage()
        S = self.shard_numel
        dst = self._full[self.rank * S : (self.rank + 1) * S]
        src = self.flat_shard.detach()
        stream = _native.stream_of(self.device)
        if src.dtype == torch.float32 and dst.dtype == torch.bfloat16:
            _native.cast_f32_bf16(src.data_ptr(), dst.data_ptr(), S, stream)
        else:
            _copy_spans([(src.data_ptr(), dst.data_ptr(), S)], src.dtype, dst.dtype, self.device)

    def _cast_into_own_slot(self) -> None:
        """This rank's master shard -> its slot of the gather buffer (fsdp.py:178-180)."""
        self._on_gather_side(self._cast_own_slot_now)

    def _own_slot_span(self) -> tuple[int, int, int]:
        """(master shard, this rank's slot of the gather buffer, S): the unshard cast."""
        self._require_gathered_storage()
        S = self.shard_numel
        return (self.flat_shard.detach().data_ptr(), self._full[self.rank * S :].data_ptr(), S)

    def _peer_slot_spans(self) -> list[tuple[int, int, int]]:
        """(peer's gathered shard, its slot, S) for every peer (ResidentGroup): the all-gather."""
        self._require_gathered_storage()
        S = self.shard_numel
        return [(self._peer_shards[r].data_ptr(), self._full[r * S :].data_ptr(), S)
                for r in range(self.world) if r != self.rank]

    def _account_all_gather(self) -> None:
        if self.world > 1:
            payload = self._full.numel() * self._full.element_size()
            comm.comm_stats.add("all_gather", payload, int((self.world - 1) / self.world * payload))

    def _gather_now(self) -> None:
        self._cast_own_slot_now()
        S = self.shard_numel
        if self.world > 1:
            self._account_all_gather()
            if self._ipc is not None:
                self._gather_over_ipc()
            elif isinstance(self.group, comm.ResidentGroup):
                _copy_spans(self._peer_slot_spans(), self._full.dtype, self._full.dtype, self.device)
            else:
                own = self._full[self.rank * S : (self.rank + 1) * S]
                comm.dist_all_gather_into_tensor(self._full, own, group=self.group)

    def _gather_over_ipc(self) -> None:
        """The all-gather as one-shot copies: this rank publishes its cast shard in its row of the
        shard buffer; once every rank has, each copies the peers' shards from their mapped rows
        into their slots of its gather buffer; and no rank republishes before all have copied."""
        S, dt, es = self.shard_numel, self._full.dtype, self._full.element_size()
        base, ipc = self._full.data_ptr(), self._ipc
        _copy_spans([(base + self.rank * S * es, ipc.shard.data_ptr(), S)], dt, dt, self.device)
        self.group.rows_written()
        reads = [(ipc.shard_ptrs[r], base + r * S * es, S) for r in range(self.world) if r != self.rank]
        _copy_spans(comm.interleave_spans(reads, es, es), dt, dt, self.device)
        self.group.rows_read()

    def unshard(self) -> None:
        """Gather the full parameters (fsdp.py:172-182).  With side streams the gather is
        only enqueued; :meth:`wait_gathered` orders the caller's stream after it."""
        if self._unsharded:
            return
        # allocated on the caller's stream, which waits for the gather before freeing it
        self._full.untyped_storage().resize_(self.padded_numel * self._full.element_size())
        self._unsharded = True
        self._on_gather_side(self._gather_now)

    def wait_gathered(self) -> None:
        """Make the caller's stream wait for a gather still pending on the side stream."""
        if self._gathered is not None:
            torch.cuda.current_stream(self.device).wait_event(self._gathered)
            self._gathered = None

    def reshard(self) -> None:
        """Free the gathered parameters (storage only; views survive)."""
        if not self._unsharded:
            return
        self.wait_gathered()
        self._full.untyped_storage().resize_(0)
        self._unsharded = False

    # -- gradients ----------------------------------------------------------

    def arm_gradient_reduction(self) -> None:
        self._grads_pending = sum(1 for p in self.params if p.requires_grad)
        self._backward_done = False

    def on_param_grad_ready(self, sync: bool) -> None:
        self._grads_pending -= 1
        if self._grads_pending > 0:
            return
        self._backward_done = True
        if sync:
            self.reduce_scatter_grads()
        self.reshard()

    def holds_grads(self) -> bool:
        """Whether any parameter still has a full-size gradient (left by a ``no_sync`` backward)."""
        return any(p.grad is not None for p in self.params)

    def _own_pieces(self) -> list[tuple[int, int, int]]:
        """(own grad address | 0, shard position, numel) covering the whole shard."""
        S, lo = self.shard_numel, self.rank * self.shard_numel
        hi = lo + S
        rows, cursor, off = [], lo, 0
        for p, n in zip(self.params, self.numels, strict=True):
            a, b = max(off, lo), min(off + n, hi)
            if a < b:
                g = p.grad
                if g is None:
                    rows.append((0, a - lo, b - a))
                else:
                    _check_grad(g)
                    rows.append((g.data_ptr() + (a - off) * g.element_size(), a - lo, b - a))
                cursor = b
            off += n
        if cursor < hi:  # padding at the end of the last shard
            rows.append((0, cursor - lo, hi - cursor))
        return rows

    def _grad_out(self) -> tuple[torch.Tensor, bool]:
        g = self.flat_shard.grad
        if g is None:
            return torch.empty(self.shard_numel, dtype=self.flat_shard.dtype, device=self.device), False
        return g, True

    def _reduce_now(self, out: torch.Tensor, accumulate: bool, grad_dtype: torch.dtype) -> None:
        reduce_dtype = self.policy.reduce_dtype
        shard_dtype = self.flat_shard.dtype
        stream = _native.stream_of(self.device)
        if self._ipc is not None and self.world > 1:
            self._reduce_over_ipc(out, accumulate, grad_dtype, stream)
            return
        if isinstance(self.group, comm.ResidentGroup) or self.world == 1:
            lo = self.rank * self.shard_numel
            peers = (
                [self._peer_grads[r, lo:].data_ptr() for r in range(self.world)]
                if self.world > 1
                else [0]
            )
            _native.reduce_scatter_share(
                _native.pieces_array(self._own_pieces()), peers, self.rank,
                _native.dtype_code(grad_dtype), _native.dtype_code(reduce_dtype), True,
                out.data_ptr(), _native.dtype_code(shard_dtype), accumulate, 1.0, None, stream,
            )
            return
        # Real process group: pack + pre-divide locally, reduce-scatter over
        # RCCL, then convert / accumulate into the shard gradient.
        buf = torch.empty(self.padded_numel, dtype=reduce_dtype, device=self.device)
        rows, off = [], 0
        for p, n in zip(self.params, self.numels, strict=True):
            g = p.grad
            if g is not None:
                _check_grad(g)
            rows.append((g.data_ptr() if g is not None else 0, buf.data_ptr() + off * buf.element_size(), n))
            off += n
        if off < self.padded_numel:
            rows.append((0, buf.data_ptr() + off * buf.element_size(), self.padded_numel - off))
        _native.pack(
            _native.spans_array(rows), _native.dtype_code(grad_dtype), _native.dtype_code(reduce_dtype),
            float(self.world), True, stream,
        )
        red = torch.empty(self.shard_numel, dtype=reduce_dtype, device=self.device)
        comm.dist_reduce_scatter_tensor(red, buf, group=self.group)
        _native.reduce_scatter_share(
            _native.pieces_array([(red.data_ptr(), 0, self.shard_numel)]), [0], 0,
            _native.dtype_code(reduce_dtype), _native.dtype_code(reduce_dtype), False,
            out.data_ptr(), _native.dtype_code(shard_dtype), accumulate, 1.0, None, stream,
        )

    def _reduce_over_ipc(self, out: torch.Tensor, accumulate: bool, grad_dtype: torch.dtype, stream: int) -> None:
        """The reduce-scatter as a one-shot share: this rank publishes its full-size gradient in its
        row of the gradient buffer (zeros for missing gradients and the padding); once every rank
        has, each sums its slice of all W rows in rank order -- the share kernel over the mapped
        rows -- and no rank republishes before all have read."""
        ipc = self._ipc
        if grad_dtype != ipc.grads.dtype:
            raise RuntimeError(f"FSDP over an IpcGroup: gradients in {grad_dtype}, rows in {ipc.grads.dtype}")
        code, es, base = _native.dtype_code(grad_dtype), ipc.grads.element_size(), ipc.grads.data_ptr()
        spans, off = [], 0
        for p, n in zip(self.params, self.numels, strict=True):
            g = p.grad
            if g is not None:
                _check_grad(g)
            spans.append((0 if g is None else g.data_ptr(), base + off * es, n))
            off += n
        if off < self.padded_numel:
            spans.append((0, base + off * es, self.padded_numel - off))
        _native.pack(_native.spans_array(spans), code, code, 1.0, False, stream)
        self.group.rows_written()
        lo = self.rank * self.shard_numel
        peers = [ptr + lo * es for ptr in ipc.grad_ptrs]
        _native.reduce_scatter_share(
            _native.pieces_array([(peers[self.rank], 0, self.shard_numel)]), peers, self.rank, code,
            _native.dtype_code(self.policy.reduce_dtype), True, out.data_ptr(), _native.dtype_code(self.flat_shard.dtype),
            accumulate, 1.0, None, stream,
        )
        self.group.rows_read()

    def _account_reduce_scatter(self) -> None:
        if self.world > 1:
            payload = self.padded_numel * torch.empty((), dtype=self.policy.reduce_dtype).element_size()
            comm.comm_stats.add("reduce_scatter", payload, int((self.world - 1) / self.world * payload))

    def _finish_reduce_scatter(self, out: torch.Tensor, accumulate: bool) -> None:
        if not accumulate:
            self.flat_shard.grad = out
        # Drop the full-size gradients -- the memory FSDP exists to save.
        for p in self.params:
            p.grad = None

    def reduce_scatter_grads(self) -> None:
        """Reduce full gradients across the group, keeping only this rank's shard."""
        out, accumulate = self._grad_out()
        grad_dtype = self._grad_dtype()
        self._account_reduce_scatter()
        if self.streams is None:
            self._reduce_now(out, accumulate, grad_dtype)
        else:
            # the full-size gradients and the shard gradient stay allocated until the side work is done
            keep = [out, *(p.grad for p in self.params if p.grad is not None)]
            self.streams.run(self.streams.reduce, lambda: self._reduce_now(out, accumulate, grad_dtype), keep=keep)
        self._finish_reduce_scatter(out, accumulate)

    def _grad_dtype(self) -> torch.dtype:
        for p in self.params:
            if p.grad is not None:
                return p.grad.dtype
        return self.policy.param_dtype

    def numel_report(self) -> tuple[int, int]:
        return self.total_numel, self.shard_numel


class _UnitHooks:
    """The hook callables of one unit, bound to it and its wrapper through weak references.

    torch keeps a parameter's post-accumulate-grad hooks out of the cycle
    collector's sight, so a hook that held the wrapper or the unit (which
    holds the parameter) would keep every shard, gather buffer and resident
    peer buffer alive after the caller drops the wrapper.  Module hooks are
    visible to the collector, but sharing one object keeps the rule simple:
    once either side is gone every hook is a no-op, and the wrapper's
    finalizer removes them."""

    __slots__ = ("_unit", "_wrapper")

    def __init__(self, unit: _FSDPUnit, wrapper: FullyShardedDataParallel):
        self._unit = weakref.ref(unit)
        self._wrapper = weakref.ref(wrapper)

    def _pair(self) -> tuple[_FSDPUnit | None, FullyShardedDataParallel | None]:
        unit, wrapper = self._unit(), self._wrapper()
        if unit is None or wrapper is None:
            return None, None
        return unit, wrapper

    def before_forward(self, module, args) -> None:
        unit, wrapper = self._pair()
        if unit is None:
            return
        wrapper._gather(unit, forward=True)
        if torch.is_grad_enabled():
            unit.arm_gradient_reduction()

    def after_forward(self, module, args, output) -> None:
        unit, _ = self._pair()
        # Without autograd no backward will come to free the unit, whatever its policy.
        if unit is not None and (unit.reshard_after_forward or not torch.is_grad_enabled()):
            unit.reshard()

    def before_backward(self, module, grad_output) -> None:
        unit, wrapper = self._pair()
        if unit is not None:
            wrapper._gather(unit, forward=False)

    def grad_ready(self, param) -> None:
        unit, wrapper = self._pair()
        if unit is not None:
            wrapper._on_grad_ready(unit)


class _UnitSpec(NamedTuple):
    module: nn.Module
    name: str
    params: list[nn.Parameter]
    is_root: bool


def _partition(root: nn.Module, unit_types: tuple[type, ...]) -> list[_UnitSpec]:
    """Which parameters each unit owns (the reference's rule, fsdp.py:315-357).

    Modules of ``unit_types`` below the root become units in pre-order; each
    takes the parameters of its subtree that no earlier unit took, so an
    outer match swallows its nested matches and a shared parameter belongs
    to the first unit that reaches it.  A unit left with nothing is dropped.
    Whatever no unit took forms a last unit on the root itself."""
    owner: dict[int, int] = {}
    heads = [(name, m) for name, m in root.named_modules() if m is not root and isinstance(m, unit_types)]
    specs = []
    for k, (name, m) in enumerate(heads):
        taken = [p for p in m.parameters() if owner.setdefault(id(p), k) == k]
        if taken:
            specs.append(_UnitSpec(m, name, taken, False))
    rest = [p for p in root.parameters() if id(p) not in owner]
    if rest:
        specs.append(_UnitSpec(root, "<root>", rest, True))
    return specs


# A kernel-argument table carries up to this many runs (kRunsPerLaunch of the
# library); a batch with more goes out through a device plan in one dispatch.
_KERNARG_RUNS = 48
_ARENA_ALIGN_ELEMS = 128  # unit blocks of the shared peer-gradient rows start 256-byte aligned (16-bit)


class _PlanCache:
    """The last device plan built for each kind of batched launch, keyed by its exact table:
    a step that repeats the previous one's addresses launches without a rebuild."""

    __slots__ = ("_plans",)

    def __init__(self):
        self._plans: dict = {}

    def get(self, kind, table_key, build):
        hit = self._plans.get(kind)
        if hit is None or hit[0] != table_key:
            hit = (table_key, build())
            self._plans[kind] = hit
        return hit[1]


def _peer_grad_arena(specs, world: int, dtype: torch.dtype, device) -> tuple[torch.Tensor, list[int]]:
    """One [W, cols] allocation holding every unit's emulated peer gradients, so that a single
    multi-unit share addresses all units from one set of rows; and each unit's column offset."""
    offsets, cols = [], 0
    for spec in specs:
        total = sum(p.numel() for p in spec.params)
        padded = (total + world - 1) // world * world
        offsets.append(cols)
        cols += (padded + _ARENA_ALIGN_ELEMS - 1) // _ARENA_ALIGN_ELEMS * _ARENA_ALIGN_ELEMS
    return torch.zeros((world, max(cols, 1)), dtype=dtype, device=device), offsets


def _attach_ipc_rows(units: list[_FSDPUnit], group, dtype: torch.dtype) -> list[list[int]]:
    """Two symmetric buffers of ``group`` (an IpcGroup) for the units' blocks: the full-size
    gradients each rank publishes for the reduce-scatter and the shards it publishes for the
    all-gather.  Units go into consecutive segments, each pair of buffers within the group's
    ``segment_bytes``; returns every segment's gradient-buffer row addresses.  Collective:
    every rank allocates them in the same order and sizes."""
    es = torch.empty((), dtype=dtype).element_size()
    limit = group.segment_bytes
    segments: list[list[tuple[_FSDPUnit, int, int]]] = [[]]
    g_total = s_total = 0
    for u in units:
        # a unit starts at an aligned offset; the buffer ends with the last unit's rows
        g_len = -(-u.padded_numel // _ARENA_ALIGN_ELEMS) * _ARENA_ALIGN_ELEMS
        s_len = -(-u.shard_numel // _ARENA_ALIGN_ELEMS) * _ARENA_ALIGN_ELEMS
        if u.padded_numel * es > limit:
            raise ValueError(f"FSDP over an IpcGroup: unit {u.name!r} needs {u.padded_numel * es} bytes of "
                             f"gradient rows, more than the group's segment_bytes ({limit})")
        if segments[-1] and (g_total + u.padded_numel) * es > limit:
            segments.append([])
            g_total = s_total = 0
        segments[-1].append((u, g_total, s_total))
        g_total += g_len
        s_total += s_len
    share_rows = []
    for seg, members in enumerate(segments):
        last, go_last, so_last = members[-1]
        grads = group.zeros(go_last + last.padded_numel, dtype)
        shards = group.zeros(so_last + last.shard_numel, dtype)
        g_rows, s_rows = group.row_addresses(grads), group.row_addresses(shards)
        for u, go, so in members:
            u._ipc = _IpcRows(grads[go : go + u.padded_numel], [r + go * es for r in g_rows],
                              shards[so : so + u.shard_numel], [r + so * es for r in s_rows])
            u.arena_offset = go
            u.segment = seg
        share_rows.append(g_rows)
    return share_rows


def _state_footprint(units: list[_FSDPUnit], param_dtype: torch.dtype) -> dict[str, float]:
    """Per-rank state in MiB beside DDP's (fsdp.py:472-489): parameters + gradients + Adam's
    two moments are four shard-dtype copies, sharded under FSDP and whole under DDP; the
    transient gather is the largest unit in ``param_dtype``."""
    full = [u.total_numel for u in units]
    shard = [u.shard_numel for u in units]
    master_bytes = units[0].flat_shard.element_size()
    gather_bytes = torch.empty((), dtype=param_dtype).element_size()

    def mib(elems: int, nbytes: int, copies: int = 1) -> float:
        return elems * nbytes * copies / 2**20

    return {
        "params_total_M": sum(full) / 1e6,
        "shard_params_MB": mib(sum(shard), master_bytes),
        "replicated_params_MB": mib(sum(full), master_bytes),
        "fsdp_state_MB": mib(sum(shard), master_bytes, 4),
        "ddp_state_MB": mib(sum(full), master_bytes, 4),
        "transient_gather_MB": mib(max(full), gather_bytes),
        "num_units": len(units),
    }


class FullyShardedDataParallel(nn.Module):
    """Shard a module's parameters, gradients and optimizer state across a group.

    Parameters follow the reference (fsdp.py:247-281); ``process_group`` may
    be a :class:`~minidist.comm.ResidentGroup`.  Two additions, results
    bit-identical either way:

    * ``comm_streams`` runs every unit's gather on one side stream and every
      reduce-scatter on another, ordered against the caller's stream with
      events;
    * ``unit_batch`` issues the hooks' work for up to that many units at a
      time: a unit gathered for its forward (or backward) brings the next
      units along in one batched unshard (one cast dispatch), and the
      reduce-scatters of units whose gradients are complete are held until
      ``unit_batch`` of them are ready -- or backward ends -- and, under a
      ResidentGroup, go out as one multi-unit dispatch.  Each dispatch of a
      unit is short (tens of MB at GPT-2-XL's 1.5B parameters), so the
      per-dispatch ramp and tail are a large share of its time; batching
      pays them once per group.  Over a real process group every unit's
      all-gather and reduce-scatter remain a collective of their own.  The
      cost is memory: up to ``unit_batch`` units' gathered parameters, and
      their full-size gradients, are resident at once.
    """

    def __init__(
        self,
        module: nn.Module,
        unit_types: Sequence[type] = (),
        process_group=None,
        mixed_precision: MixedPrecisionPolicy | None = None,
        reshard_after_forward: bool = True,
        reshard_root_after_forward: bool = False,
        broadcast_parameters: bool = True,
        device: torch.device | None = None,
        comm_streams: bool = False,
        unit_batch: int = 1,
    ):
        super().__init__()
        if not isinstance(unit_batch, int) or unit_batch < 1:
            raise ValueError(f"unit_batch must be a positive int, got {unit_batch!r}")
        self.module = module
        self.process_group = process_group
        self.world_size = comm.get_world_size(process_group)
        self.policy = mixed_precision or MixedPrecisionPolicy()
        self.require_backward_grad_sync = True
        resident = _emulates_peers(process_group)
        ipc = isinstance(process_group, comm.IpcGroup)
        if ipc and comm_streams:
            raise ValueError("comm_streams with an IpcGroup: its collectives synchronise with the host")
        self.unit_batch = unit_batch
        if device is None:
            device = process_group.device if isinstance(process_group, comm.ResidentGroup) else comm.current_device()
        if broadcast_parameters and self.world_size > 1 and not resident:
            # every parameter and buffer (fsdp.py:307-313); an IpcGroup's ranks meet over its host group
            comm.broadcast_module_state(module, process_group.process_group if ipc else process_group)

        specs = _partition(module, tuple(unit_types))
        # Emulated peers' gradients (ResidentGroup): one arena for all units.
        self._peer_arena: torch.Tensor | None = None
        offsets = [0] * len(specs)
        if resident and self.world_size > 1 and specs:
            self._peer_arena, offsets = _peer_grad_arena(specs, self.world_size, self.policy.param_dtype,
                                                          torch.device(device))
        self._units = [
            _FSDPUnit(spec.module, spec.params, process_group, self.policy,
                      reshard_root_after_forward if spec.is_root else reshard_after_forward, device, spec.name,
                      peer_grads=None if self._peer_arena is None else self._peer_arena[:, off : off + self._padded(spec)],
                      arena_offset=off)
            for spec, off in zip(specs, offsets, strict=True)
        ]
        if not self._units:
            raise ValueError("FSDP wrapped a module with no parameters")
        # The W rows a multi-unit share reads, per segment: the emulated peers' arena (one
        # segment), or the IpcGroup's buffers of published gradients (each unit's arena_offset
        # is its block in its segment's rows).
        self._share_rows: list[list[int]] | None = None
        if self._peer_arena is not None:
            self._share_rows = [[self._peer_arena[r].data_ptr() for r in range(self.world_size)]]
        if ipc and self.world_size > 1:
            self._share_rows = _attach_ipc_rows(self._units, process_group, self.policy.param_dtype)
        self._plans = _PlanCache()
        # The optimizer's state: only the shards (the original parameters are forward-only views).
        self._shards = nn.ParameterList([u.flat_shard for u in self._units])
        self._streams = _SideStreams(torch.device(device)) if comm_streams else None
        # unit_batch: the units a batched gather walks (every unit but the root, in order),
        # and the reduce-scatters held until unit_batch units are ready
        self._chain = [u for u, spec in zip(self._units, specs, strict=True) if not spec.is_root]
        self._chain_index = {id(u): i for i, u in enumerate(self._chain)}
        self._held_reductions: list[_FSDPUnit] = []
        self._prefetched_for_backward: list[_FSDPUnit] = []
        self._prefetched_for_forward: dict[int, _FSDPUnit] = {}
        self._end_queued = False
        for unit in self._units:
            unit.streams = self._streams
            unit.attach(_UnitHooks(unit, self))
        weakref.finalize(self, _detach_all, [u._hook_handles for u in self._units])

    def _padded(self, spec: _UnitSpec) -> int:
        total = sum(p.numel() for p in spec.params)
        return (total + self.world_size - 1) // self.world_size * self.world_size

    # -- batched launches (units that are ready at the same time) --------------

    def _copy_many(self, kind: str, spans: list[tuple[int, int, int]], src: torch.dtype, dst: torch.dtype) -> None:
        """Span copies in one dispatch (a device plan beyond one kernel-argument table)."""
        if not spans:
            return
        device = self._units[0].device
        table = _native.spans_array(spans)
        stream = _native.stream_of(device)
        s_code, d_code = _native.dtype_code(src), _native.dtype_code(dst)
        if len(spans) <= _KERNARG_RUNS:
            _native.pack(table, s_code, d_code, 1.0, False, stream)
            return
        plan = self._plans.get((kind, src, dst), tuple(spans), lambda: _native.plan_spans(table, s_code, d_code, device))
        _native.pack_planned(plan, 1.0, False, stream)

    def _cast_own_slots(self, units: list[_FSDPUnit]) -> None:
        """The unshard cast of several units (master shard -> own slot of the gather buffer),
        batched: one dispatch per dtype pair."""
        by_dtype: dict[tuple[torch.dtype, torch.dtype], list] = {}
        for u in units:
            by_dtype.setdefault((u.flat_shard.dtype, u._full.dtype), []).append(u._own_slot_span())

        def work():
            for (src, dst), spans in by_dtype.items():
                self._copy_many("cast", spans, src, dst)

        self._on_gather_side_many(units, work)

    def _on_gather_side_many(self, units: list[_FSDPUnit], work) -> None:
        if self._streams is None:
            work()
            return
        done = self._streams.run(self._streams.gather, work, event=True)
        for u in units:
            u._gathered = done

    def _unshard_many(self, units: list[_FSDPUnit]) -> None:
        """``unshard`` of several units with the casts (and, under a ResidentGroup, the peers'
        gather copies) batched into single dispatches."""
        units = [u for u in units if not u.is_unsharded]
        if not units:
            return
        for u in units:
            u._full.untyped_storage().resize_(u.padded_numel * u._full.element_size())
            u._unsharded = True
        resident = isinstance(self.process_group, comm.ResidentGroup)
        ipc = isinstance(self.process_group, comm.IpcGroup) and self.world_size > 1

        def work():
            by_dtype: dict[tuple[torch.dtype, torch.dtype], list] = {}
            for u in units:
                by_dtype.setdefault((u.flat_shard.dtype, u._full.dtype), []).append(u._own_slot_span())
            for (src, dst), spans in by_dtype.items():
                self._copy_many("cast", spans, src, dst)
            if ipc:
                # one publish, fence, read, fence for all of them (_FSDPUnit._gather_over_ipc, batched)
                dt = self.policy.param_dtype
                self._copy_many("publish", [(span[1], u._ipc.shard.data_ptr(), span[2])
                                            for u in units for span in [u._own_slot_span()]], dt, dt)
                self.process_group.rows_written()
                reads = []
                for u in units:
                    u._account_all_gather()
                    S, es, base = u.shard_numel, u._full.element_size(), u._full.data_ptr()
                    reads += [(u._ipc.shard_ptrs[r], base + r * S * es, S) for r in range(u.world) if r != u.rank]
                es = torch.empty((), dtype=dt).element_size()
                self._copy_many("gather", comm.interleave_spans(reads, es, es), dt, dt)
                self.process_group.rows_read()
            elif self.world_size > 1:
                peer: dict[torch.dtype, list] = {}
                for u in units:
                    u._account_all_gather()
                    if resident:
                        peer.setdefault(u._full.dtype, []).extend(u._peer_slot_spans())
                    else:
                        S = u.shard_numel
                        own = u._full[u.rank * S : (u.rank + 1) * S]
                        comm.dist_all_gather_into_tensor(u._full, own, group=u.group)
                for dt, spans in peer.items():
                    self._copy_many("gather", spans, dt, dt)

        self._on_gather_side_many(units, work)

    def _reduce_scatter_many(self, units: list[_FSDPUnit]) -> None:
        """``reduce_scatter_grads`` of several units (a ResidentGroup or an IpcGroup): the shares
        of all of them in one multi-unit dispatch per (gradient dtype, shard dtype, set /
        accumulate), over the W rows of ``_share_rows`` -- the emulated peers' arena, or the
        IpcGroup's gradient buffer, into which every rank first publishes its units' gradients."""
        rank = self._units[0].rank
        ipc = isinstance(self.process_group, comm.IpcGroup)
        if ipc:
            for u in units:
                if u._grad_dtype() != u._ipc.grads.dtype:
                    raise RuntimeError(f"FSDP over an IpcGroup: gradients in {u._grad_dtype()}, "
                                       f"rows in {u._ipc.grads.dtype}")
            spans = []
            for u in units:
                es, base, off = u._ipc.grads.element_size(), u._ipc.grads.data_ptr(), 0
                for p, n in zip(u.params, u.numels, strict=True):
                    if p.grad is not None:
                        _check_grad(p.grad)
                    spans.append((0 if p.grad is None else p.grad.data_ptr(), base + off * es, n))
                    off += n
                if off < u.padded_numel:
                    spans.append((0, base + off * es, u.padded_numel - off))
            dt = self.policy.param_dtype
            self._copy_many("publish-grads", spans, dt, dt)
            self.process_group.rows_written()
        reduce_dtype = self.policy.reduce_dtype
        groups: dict[tuple, tuple[list, list, list]] = {}
        for u in units:
            out, accumulate = u._grad_out()
            gdt = u._grad_dtype()
            pieces, outs, members = groups.setdefault((gdt, out.dtype, accumulate, u.segment), ([], [], []))
            base = u.arena_offset + rank * u.shard_numel
            es = out.element_size()
            for ptr, pos, n in u._own_pieces():
                pieces.append((ptr, base + pos, n))
                outs.append(out.data_ptr() + pos * es)
            members.append((u, out, accumulate))
            u._account_reduce_scatter()
        device = self._units[0].device

        def share(gdt, sdt, accumulate, seg, pieces, outs):
            peers = self._share_rows[seg]
            table = _native.pieces_array(pieces)
            stream = _native.stream_of(device)
            g_code, s_code = _native.dtype_code(gdt), _native.dtype_code(sdt)
            if len(pieces) > _KERNARG_RUNS and reduce_dtype == torch.float32 and sdt == torch.float32:
                plan = self._plans.get(("share", gdt, accumulate, seg), (tuple(pieces), tuple(outs)),
                                       lambda: _native.plan_reduce_scatter_share_multi(table, outs, peers, rank,
                                                                                       g_code, device))
                _native.reduce_scatter_share_multi_planned(plan, True, accumulate, 1.0, None, stream)
            else:
                _native.reduce_scatter_share_multi(table, outs, peers, rank, g_code, _native.dtype_code(reduce_dtype),
                                                   True, s_code, accumulate, 1.0, None, stream)

        for (gdt, sdt, accumulate, seg), (pieces, outs, members) in groups.items():
            work = (lambda g=gdt, d=sdt, a=accumulate, k=seg, pc=pieces, o=outs: share(g, d, a, k, pc, o))
            if self._streams is None:
                work()
            else:
                keep = [out for _, out, _ in members]
                keep += [p.grad for u, _, _ in members for p in u.params if p.grad is not None]
                self._streams.run(self._streams.reduce, work, keep=keep)
        if ipc:
            self.process_group.rows_read()
        for _, (_, _, members) in groups.items():
            for u, out, accumulate in members:
                u._finish_reduce_scatter(out, accumulate)

    # -- backward-time machinery ---------------------------------------------

    def _gather(self, unit: _FSDPUnit, forward: bool) -> None:
        """Gather ``unit`` before its forward (or backward) and make the caller's stream wait for it.

        With ``unit_batch`` > 1 a unit that is not gathered yet is gathered together with
        the units that are expected next -- the following ones in forward, the preceding
        ones in backward, up to ``unit_batch`` in all -- in one batched unshard.  The
        expectation is registration order; where the model runs its units in another
        order, a backward batch leaves out every unit whose backward this step has
        already completed (gathering it again would keep pre-update weights past the
        optimizer step), and a unit it brought along whose backward then never comes --
        or, in forward, whose forward never comes -- is freed when the engine finishes the
        backward, so every unit is sharded after backward, as in the reference."""
        if forward:
            self._prefetched_for_forward.pop(id(unit), None)  # it runs after all
        if not unit.is_unsharded:
            k = self.unit_batch
            i = self._chain_index.get(id(unit))
            if k == 1 or i is None:
                unit.unshard()
            elif forward:
                batch = [u for u in self._chain[i : i + k] if not u.is_unsharded]
                self._unshard_many(batch)
                self._prefetched_for_forward.update((id(u), u) for u in batch if u is not unit)
            else:
                ahead = [u for u in self._chain[max(0, i - k + 1) : i][::-1]
                         if not u.is_unsharded and not u._backward_done]
                self._unshard_many([unit, *ahead])
                if ahead:
                    self._prefetched_for_backward.extend(ahead)
                    self._queue_end_of_backward()
        unit.wait_gathered()

    def _queue_end_of_backward(self) -> None:
        if not self._end_queued:
            self._end_queued = True
            torch.autograd.Variable._execution_engine.queue_callback(self._end_of_backward)

    def _on_grad_ready(self, unit: _FSDPUnit) -> None:
        if self._streams is not None or self.unit_batch > 1:
            # Held reduce-scatters are flushed, and shard gradients written on the reduce
            # stream ordered before whatever follows on the caller's stream (the optimizer),
            # when the engine finishes this backward.
            self._queue_end_of_backward()
        sync = self.require_backward_grad_sync
        if self.unit_batch == 1:
            unit.on_param_grad_ready(sync=sync)
            return
        unit._grads_pending -= 1
        if unit._grads_pending > 0:
            return
        unit._backward_done = True
        # The unit's gradients are complete: its reduce-scatter waits for the next ones'
        # (it reads the gradients, not the gathered parameters, so the unit reshards now).
        if sync:
            self._held_reductions.append(unit)
            if len(self._held_reductions) >= self.unit_batch:
                self._reduce_held()
        unit.reshard()

    def _reduce_held(self) -> None:
        """The reduce-scatters held back by ``unit_batch``, as one multi-unit dispatch."""
        units, self._held_reductions = self._held_reductions, []
        if len(units) > 1 and self._share_rows is not None:
            self._reduce_scatter_many(units)
        else:
            for unit in units:
                unit.reduce_scatter_grads()

    def _end_of_backward(self) -> None:
        self._end_queued = False
        self._reduce_held()
        prefetched, self._prefetched_for_backward = self._prefetched_for_backward, []
        prefetched += self._prefetched_for_forward.values()
        self._prefetched_for_forward = {}
        for unit in prefetched:
            unit.reshard()
        if self._streams is not None:
            self._streams.join()

    # -- public API ---------------------------------------------------------

    def forward(self, *args, **kwargs):
        return self.module(*args, **kwargs)

    def named_parameters(self, prefix: str = "", recurse: bool = True, remove_duplicate: bool = True):
        """Only the flat shards: what the optimizer must update."""
        lead = f"{prefix}." if prefix else ""
        return ((f"{lead}_flat_shard_{i}", unit.flat_shard) for i, unit in enumerate(self._units))

    def parameters(self, recurse: bool = True):
        return (p for _, p in self.named_parameters(recurse=recurse))

    @contextmanager
    def no_sync(self) -> Iterator[None]:
        """Accumulate unsharded gradients locally without reduce-scatter."""
        saved, self.require_backward_grad_sync = self.require_backward_grad_sync, False
        try:
            yield
        finally:
            self.require_backward_grad_sync = saved

    @contextmanager
    def summon_full_params(self) -> Iterator[None]:
        """Temporarily gather every unit so parameters can be read; afterwards only
        the units gathered here are freed again (the prior state is restored)."""
        opened = [u for u in self._units if not u.is_unsharded]
        self._unshard_many(opened)
        for unit in self._units:
            unit.wait_gathered()
        try:
            yield
        finally:
            for unit in opened:
                unit.reshard()

    def finish_gradient_sync(self) -> None:
        """Flush any unit whose gradients were accumulated under ``no_sync``.

        Under a ResidentGroup the flushed units' shares go out together, as one
        multi-unit dispatch (bit-identical to one share per unit)."""
        self._reduce_held()
        if self.world_size > 1:
            ready = [u for u in self._units if u.holds_grads()]
            if self._share_rows is not None and len(ready) > 1:
                self._reduce_scatter_many(ready)
            else:
                for unit in ready:
                    unit.reduce_scatter_grads()
            for unit in ready:
                if unit.reshard_after_forward:
                    unit.reshard()
        if self._streams is not None:
            self._streams.join()

    def memory_summary(self) -> dict[str, float]:
        return _state_footprint(self._units, self.policy.param_dtype)

    def unit_summary(self) -> list[tuple[str, int, int]]:
        return [(unit.name, *unit.numel_report()) for unit in self._units]

    def __getattr__(self, name: str):
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(self.module, name)


def _detach_all(handle_lists: list) -> None:
    for handles in handle_lists:
        while handles:
            handles.pop().remove()


FSDP = FullyShardedDataParallel
