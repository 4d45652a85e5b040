"""Fully Sharded Data Parallel (ZeRO-3): shard parameters, gradients and optimizer state.

Same public surface, unit layout and lifecycle as the reference's
minidist/fsdp.py (``MixedPrecisionPolicy`` :72-105, ``_FSDPUnit`` :108-244,
``FullyShardedDataParallel`` :247-504).  The two arithmetic steps of the unit
run as gfx950 kernels:

* ``unshard`` (:172-182): the fp32 master shard is cast to ``param_dtype``
  (bf16 or fp16, round-to-nearest-even) *straight into this rank's slot* of the gather
  buffer, so the all-gather needs no separate input; with a real process
  group the all-gather then runs in place, with a
  :class:`~minidist.comm.ResidentGroup` the peers' resident shards are copied
  into their slots by one multi-span dispatch.
* ``reduce_scatter_grads`` (:215-241): with a ResidentGroup, one
  ``mdx_reduce_scatter_share`` dispatch reads this rank's slice of its own
  gradients straight from the ``p.grad`` tensors (no padded flat copy), the
  peers' slices from their resident full-size contributions, widens each to
  ``reduce_dtype``, divides by W, sums in rank order and writes -- or
  accumulates into -- ``flat_shard.grad``.  Peers contribute their gradients
  in ``param_dtype`` (what they would send); widening is exact and the
  division is applied per contribution exactly as the reference's
  ``buf.div_(W)`` does, so the result is the reference's bit for bit.
"""

from __future__ import annotations

import weakref
from collections.abc import Iterator, Sequence
from contextlib import contextmanager

import torch
import torch.distributed as dist
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

        self.shapes = [p.shape for p in params]
        self.numels = [p.numel() for p in params]
        self.total_numel = sum(self.numels)
        # Pad so the flat parameter divides evenly (fsdp.py:132-136).
        self.shard_numel = (self.total_numel + self.world - 1) // self.world
        self.padded_numel = self.shard_numel * self.world

        src_dtype = params[0].dtype
        shard_dtype = policy.param_dtype if policy.keep_low_precision_shard else src_dtype

        # Full flat parameter (pack kernel), this rank's slice as the master shard.
        flat = torch.zeros(self.padded_numel, dtype=src_dtype, device=self.device)
        staged = [p.detach().to(self.device).contiguous() for p in params]
        rows, off = [], 0
        for t, n in zip(staged, self.numels, strict=True):
            rows.append((t.data_ptr(), flat.data_ptr() + off * flat.element_size(), n))
            off += n
        _copy_spans(rows, src_dtype, src_dtype, self.device)
        S, r0 = self.shard_numel, self.rank * self.shard_numel
        master = torch.empty(S, dtype=shard_dtype, device=self.device)
        _copy_spans([(flat[r0:].data_ptr(), master.data_ptr(), S)], src_dtype, shard_dtype, self.device)
        self.flat_shard = nn.Parameter(master)

        # Emulated peers (ResidentGroup): their gathered shards (what their
        # all-gather contributions carry) and their full-size gradients.
        self._peer_shards: torch.Tensor | None = None
        self._peer_grads: torch.Tensor | None = None
        if isinstance(group, comm.ResidentGroup) and self.world > 1:
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
            self._peer_grads = torch.zeros(
                (self.world, self.padded_numel), dtype=policy.param_dtype, device=self.device
            )
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
        self._hook_handles: list[torch.utils.hooks.RemovableHandle] = []

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

    def _cast_into_own_slot(self) -> None:
        S = self.shard_numel
        dst = self._full[self.rank * S : (self.rank + 1) * S]
        src = self.flat_shard.detach()
        stream = _native.stream_of(self.device)
        if src.dtype == torch.float32 and dst.dtype == torch.bfloat16:
            _native.cast_f32_bf16(src.data_ptr(), dst.data_ptr(), S, stream)
        else:
            _copy_spans([(src.data_ptr(), dst.data_ptr(), S)], src.dtype, dst.dtype, self.device)

    def unshard(self) -> None:
        if self._unsharded:
            return
        self._full.untyped_storage().resize_(self.padded_numel * self._full.element_size())
        self._cast_into_own_slot()
        S = self.shard_numel
        if self.world > 1:
            payload = self._full.numel() * self._full.element_size()
            comm.comm_stats.add("all_gather", payload, int((self.world - 1) / self.world * payload))
            if isinstance(self.group, comm.ResidentGroup):
                rows = [
                    (self._peer_shards[r].data_ptr(), self._full[r * S :].data_ptr(), S)
                    for r in range(self.world)
                    if r != self.rank
                ]
                _copy_spans(rows, self._full.dtype, self._full.dtype, self.device)
            else:
                own = self._full[self.rank * S : (self.rank + 1) * S]
                comm.dist_all_gather_into_tensor(self._full, own, group=self.group)
        self._unsharded = True

    def reshard(self) -> None:
        """Free the gathered parameters (storage only; views survive)."""
        if not self._unsharded:
            return
        self._full.untyped_storage().resize_(0)
        self._unsharded = False

    # -- gradients ----------------------------------------------------------

    def arm_gradient_reduction(self) -> None:
        self._grads_pending = sum(1 for p in self.params if p.requires_grad)

    def on_param_grad_ready(self, sync: bool) -> None:
        self._grads_pending -= 1
        if self._grads_pending > 0:
            return
        if sync:
            self.reduce_scatter_grads()
        self.reshard()

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
                    _native.require_device_tensor(g, "FSDP gradient")
                    if not g.is_contiguous():
                        raise RuntimeError("FSDP gradient is not contiguous")
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

    def reduce_scatter_grads(self) -> None:
        """Reduce full gradients across the group, keeping only this rank's shard."""
        reduce_dtype = self.policy.reduce_dtype
        shard_dtype = self.flat_shard.dtype
        out, accumulate = self._grad_out()
        stream = _native.stream_of(self.device)
        grad_dtype = self._grad_dtype()
        payload = self.padded_numel * torch.empty((), dtype=reduce_dtype).element_size()
        if self.world > 1:
            comm.comm_stats.add("reduce_scatter", payload, int((self.world - 1) / self.world * payload))
        if isinstance(self.group, comm.ResidentGroup) or self.world == 1:
            S, lo = self.shard_numel, self.rank * self.shard_numel
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
        else:
            # Real process group: pack + pre-divide locally, reduce-scatter over
            # RCCL, then convert / accumulate into the shard gradient.
            buf = torch.empty(self.padded_numel, dtype=reduce_dtype, device=self.device)
            rows, off = [], 0
            for p, n in zip(self.params, self.numels, strict=True):
                g = p.grad
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
        if not accumulate:
            self.flat_shard.grad = out
        # Drop the full-size gradients -- the memory FSDP exists to save.
        for p in self.params:
            p.grad = None

    def _grad_dtype(self) -> torch.dtype:
        for p in self.params:
            if p.grad is not None:
                return p.grad.dtype
        return self.policy.param_dtype

    def numel_report(self) -> tuple[int, int]:
        return self.total_numel, self.shard_numel


class FullyShardedDataParallel(nn.Module):
    """Shard a module's parameters, gradients and optimizer state across a group.

    Parameters follow the reference (fsdp.py:247-281); ``process_group`` may
    be a :class:`~minidist.comm.ResidentGroup`.
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
    ):
        super().__init__()
        self.module = module
        self.process_group = process_group
        self.world_size = comm.get_world_size(process_group)
        self.policy = mixed_precision or MixedPrecisionPolicy()
        self.require_backward_grad_sync = True
        if device is None:
            device = process_group.device if isinstance(process_group, comm.ResidentGroup) else comm.current_device()

        if broadcast_parameters and self.world_size > 1 and not isinstance(process_group, comm.ResidentGroup):
            self._broadcast_module_states()

        self._units = self._build_units(
            module, tuple(unit_types), reshard_after_forward, reshard_root_after_forward, device
        )
        self._shards = nn.ParameterList([u.flat_shard for u in self._units])
        self._register_hooks()

    # -- construction -------------------------------------------------------

    def _broadcast_module_states(self) -> None:
        src = 0 if self.process_group is None else dist.get_global_rank(self.process_group, 0)
        with torch.no_grad():
            for p in self.module.parameters():
                comm.dist_broadcast(p.data, src=src, group=self.process_group)
            for b in self.module.buffers():
                comm.dist_broadcast(b.data, src=src, group=self.process_group)

    def _build_units(self, root, unit_types, reshard_after_forward, reshard_root, device) -> list[_FSDPUnit]:
        """Pre-order claim of unit modules, then a root unit for leftovers (fsdp.py:315-357)."""
        units: list[_FSDPUnit] = []
        claimed: set[int] = set()
        for name, m in root.named_modules():
            if m is root or not isinstance(m, unit_types):
                continue
            params = [p for p in m.parameters() if id(p) not in claimed]
            if not params:
                continue
            claimed.update(id(p) for p in params)
            units.append(
                _FSDPUnit(m, params, self.process_group, self.policy, reshard_after_forward, device, name or "root")
            )
        leftovers = [p for p in root.parameters() if id(p) not in claimed]
        if leftovers:
            units.append(
                _FSDPUnit(root, leftovers, self.process_group, self.policy, reshard_root, device, "<root>")
            )
        if not units:
            raise ValueError("FSDP wrapped a module with no parameters")
        return units

    def _register_hooks(self) -> None:
        for unit in self._units:
            unit._hook_handles.append(unit.module.register_forward_pre_hook(self._make_pre_forward(unit)))
            unit._hook_handles.append(unit.module.register_forward_hook(self._make_post_forward(unit)))
            if unit.reshard_after_forward:
                unit._hook_handles.append(
                    unit.module.register_full_backward_pre_hook(self._make_pre_backward(unit))
                )
            for p in unit.params:
                if p.requires_grad:
                    unit._hook_handles.append(p.register_post_accumulate_grad_hook(self._make_grad_ready(unit)))
        weakref.finalize(self, _remove_param_hooks, [u._hook_handles for u in self._units])

    def _make_pre_forward(self, unit: _FSDPUnit):
        def hook(module, args):
            unit.unshard()
            if torch.is_grad_enabled():
                unit.arm_gradient_reduction()

        return hook

    def _make_post_forward(self, unit: _FSDPUnit):
        def hook(module, args, output):
            if unit.reshard_after_forward or not torch.is_grad_enabled():
                unit.reshard()

        return hook

    def _make_pre_backward(self, unit: _FSDPUnit):
        def hook(module, grad_output):
            unit.unshard()

        return hook

    def _make_grad_ready(self, unit: _FSDPUnit):
        # Weak references: the cycle collector does not see a parameter's
        # post-accumulate-grad hooks, so a hook holding the wrapper or the unit
        # (which holds the parameter) would keep every shard, gather buffer and
        # resident peer buffer alive after the caller drops the wrapper.
        owner_ref, unit_ref = weakref.ref(self), weakref.ref(unit)

        def hook(param):
            owner, u = owner_ref(), unit_ref()
            if owner is not None and u is not None:
                u.on_param_grad_ready(sync=owner.require_backward_grad_sync)

        return hook

    # -- public API ---------------------------------------------------------

    def forward(self, *args, **kwargs):
        return self.module(*args, **kwargs)

    def named_parameters(self, prefix: str = "", recurse: bool = True, remove_duplicate: bool = True):
        """Yield only the flat shards (the optimizer's view)."""
        for i, unit in enumerate(self._units):
            name = f"{prefix}{'.' if prefix else ''}_flat_shard_{i}"
            yield name, unit.flat_shard

    def parameters(self, recurse: bool = True):
        for _, p in self.named_parameters(recurse=recurse):
            yield p

    @contextmanager
    def no_sync(self) -> Iterator[None]:
        """Accumulate unsharded gradients locally without reduce-scatter."""
        previous = self.require_backward_grad_sync
        self.require_backward_grad_sync = False
        try:
            yield
        finally:
            self.require_backward_grad_sync = previous

    @contextmanager
    def summon_full_params(self) -> Iterator[None]:
        """Temporarily gather every unit so parameters can be read."""
        was_unsharded = [u.is_unsharded for u in self._units]
        for unit in self._units:
            unit.unshard()
        try:
            yield
        finally:
            for unit, was in zip(self._units, was_unsharded, strict=True):
                if not was:
                    unit.reshard()

    def finish_gradient_sync(self) -> None:
        """Flush any unit whose gradients were accumulated under ``no_sync``."""
        if self.world_size == 1:
            return
        for unit in self._units:
            if any(p.grad is not None for p in unit.params):
                unit.reduce_scatter_grads()
                if unit.reshard_after_forward:
                    unit.reshard()

    def memory_summary(self) -> dict[str, float]:
        total = sum(u.total_numel for u in self._units)
        sharded = sum(u.shard_numel for u in self._units)
        shard_bytes = self._units[0].flat_shard.element_size()
        largest_unit = max(u.total_numel for u in self._units)
        param_bytes = torch.empty((), dtype=self.policy.param_dtype).element_size()
        mb = 1024**2
        return {
            "params_total_M": total / 1e6,
            "shard_params_MB": sharded * shard_bytes / mb,
            "replicated_params_MB": total * shard_bytes / mb,
            "fsdp_state_MB": sharded * shard_bytes * 4 / mb,
            "ddp_state_MB": total * shard_bytes * 4 / mb,
            "transient_gather_MB": largest_unit * param_bytes / mb,
            "num_units": len(self._units),
        }

    def unit_summary(self) -> list[tuple[str, int, int]]:
        return [(u.name, u.total_numel, u.shard_numel) for u in self._units]

    def __getattr__(self, name: str):
        try:
            return super().__getattr__(name)
        except AttributeError:
            return getattr(self.module, name)


def _remove_param_hooks(handle_lists: list) -> None:
    for handles in handle_lists:
        for h in handles:
            h.remove()
        handles.clear()


FSDP = FullyShardedDataParallel
