"""Mixed precision and the collective grad scaler.

Same surface and arithmetic as the reference's minidist/amp.py
(``PrecisionConfig`` :61-81, ``resolve_precision`` :84-111,
``DistributedGradScaler`` :114-267).  ``unscale_`` is where the data path
changes: instead of ~6 ATen launches per gradient tensor (``mul_``,
``isfinite``, ``~``, ``any``, ``to``, ``+=``, amp.py:208-213) it issues one
multi-tensor ``mdx_unscale_found_inf`` dispatch per dtype, whose waves store
a 1 into a flag when they produce a non-finite value.  Gradients that
a DDP wrapper already unscaled in its unpack epilogue (``grad_scaler=``) are
skipped.  The flag is then all-reduced with MAX across a real process group
and read -- the path's only host synchronisation, as in the reference
(amp.py:216-219).  On a GPU the flag lives in pinned host memory that the
kernels store into, so the read is a stream synchronisation and a host load,
with no device-to-host copy.
"""

from __future__ import annotations

from contextlib import nullcontext
from dataclasses import dataclass

import torch
import torch.distributed as dist

from . import _native, comm

__all__ = ["PrecisionConfig", "DistributedGradScaler", "resolve_precision"]


@dataclass
class PrecisionConfig:
    """The precision decisions for one training run."""

    dtype: torch.dtype
    device_type: str
    enabled: bool

    @property
    def needs_grad_scaler(self) -> bool:
        return self.enabled and self.dtype == torch.float16

    def autocast(self):
        if not self.enabled:
            return nullcontext()
        return torch.autocast(device_type=self.device_type, dtype=self.dtype)

    def __repr__(self) -> str:
        if not self.enabled:
            return "PrecisionConfig(fp32)"
        return f"PrecisionConfig({str(self.dtype).replace('torch.', '')} autocast)"


def resolve_precision(name: str, device: torch.device | None = None) -> PrecisionConfig:
    """``'fp32' | 'fp16' | 'bf16' | 'auto'`` -> configuration (amp.py:84-111).

    ``auto`` picks bf16 wherever the device supports it natively (every
    MI355X does), which avoids loss scaling altogether.
    """
    device = device or comm.current_device()
    device_type = device.type
    if name == "auto":
        if device_type == "cuda":
            name = "bf16" if torch.cuda.is_bf16_supported() else "fp16"
        else:
            name = "bf16"
    if name == "fp32":
        return PrecisionConfig(torch.float32, device_type, enabled=False)
    if name == "bf16":
        return PrecisionConfig(torch.bfloat16, device_type, enabled=True)
    if name == "fp16":
        if device_type == "cpu":
            raise ValueError("fp16 autocast is not useful on CPU; use bf16 or fp32")
        return PrecisionConfig(torch.float16, device_type, enabled=True)
    raise ValueError(f"unknown precision {name!r}")


class _HostFlag:
    """A found-inf flag in pinned host memory.

    Kernels store into it through its device address (:meth:`data_ptr`); it
    is cleared in stream order by a one-lane dispatch (:meth:`zero_`), and the
    host reads it after synchronising the stream -- without the
    device-to-host copy a flag in device memory needs (~12 us per step on an
    MI355X, more than a third of a small configuration's step)."""

    __slots__ = ("host", "_addr", "device")

    def __init__(self, host: torch.Tensor, addr: int, device: torch.device):
        self.host = host  # int32[1] view of the pinned pair
        self._addr = addr
        self.device = device

    def data_ptr(self) -> int:
        return self._addr

    def zero_(self) -> _HostFlag:
        _native.clear_flag(self._addr, _native.stream_of(self.device))
        return self

    def settle(self) -> None:
        """Wait until the kernels that may set the flag (on the current stream, or on streams
        it joined) are done, so that the host load sees their stores."""
        _native.current_stream(self.device).synchronize()


class DistributedGradScaler:
    """Adaptive loss scaling whose skip/scale decisions are agreed across ranks.

    Parameters and state follow the reference (amp.py:114-176).
    ``process_group`` spans every rank holding a piece of the gradient; a
    :class:`~minidist.comm.ResidentGroup` needs no flag exchange (this rank's
    kernels saw every value that exists in this process).
    """

    def __init__(
        self,
        init_scale: float = 2.0**16,
        growth_factor: float = 2.0,
        backoff_factor: float = 0.5,
        growth_interval: int = 2000,
        enabled: bool = True,
        process_group=None,
        min_scale: float = 1.0,
    ):
        self.enabled = enabled
        self.process_group = process_group
        self._scale = float(init_scale)
        self._growth_factor = growth_factor
        self._backoff_factor = backoff_factor
        self._growth_interval = growth_interval
        self._min_scale = min_scale
        self._good_steps = 0
        self._found_inf_this_step = False
        self._unscaled = False
        self.num_skipped = 0
        self.num_steps = 0
        # Device-side found-inf flags: a pair of int32 per device, used in
        # alternate steps (``_parity`` picks this step's), so that a dispatch
        # that sets this step's flag can clear the next step's.  ``_flag_armed``:
        # devices whose flag of this step is zero (or will be, by a clear already
        # requested); ``_next_armed``: devices whose next-step flag a dispatch of
        # this step clears.  ``_prescaled``: the id sets of params whose grads a
        # fused producer (DDP unpack) already unscaled this step, one per launch.
        self._flags: dict[torch.device, tuple[torch.Tensor, torch.Tensor]] = {}
        self._parity = 0
        self._flag_armed: set[torch.device] = set()
        self._next_armed: set[torch.device] = set()
        self._prescaled: list[frozenset] = []

    # -- state --------------------------------------------------------------

    @property
    def scale(self) -> float:
        return self._scale if self.enabled else 1.0

    def state_dict(self) -> dict:
        return {
            "scale": self._scale,
            "good_steps": self._good_steps,
            "num_skipped": self.num_skipped,
            "num_steps": self.num_steps,
        }

    def load_state_dict(self, state: dict) -> None:
        self._scale = state["scale"]
        self._good_steps = state["good_steps"]
        self.num_skipped = state.get("num_skipped", 0)
        self.num_steps = state.get("num_steps", 0)

    # -- device flag ----------------------------------------------------------

    def _flag(self, device: torch.device, defer_clear: bool = False) -> tuple[torch.Tensor, bool]:
        """This step's found-inf flag on ``device`` and whether it still needs clearing.

        The flag is zeroed on its first use in a step, with a fill kernel (not
        a memset) so that the step can be captured into a HIP graph; with
        ``defer_clear`` the caller enqueues that clear itself (``flag.zero_()``)
        before anything that sets the flag."""
        pair = self._flags.get(device)
        pending = False
        if pair is None:
            pair = self._new_flag_pair(device)
            self._flags[device] = pair
            self._flag_armed.add(device)
            self._next_armed.add(device)  # both flags start at zero
            flag = pair[self._parity]
        elif device not in self._flag_armed:
            flag = pair[self._parity]
            if defer_clear:
                pending = True
            else:
                flag.zero_()
            self._flag_armed.add(device)
        else:
            flag = pair[self._parity]
        return flag, pending

    def _flag_exchange(self) -> tuple[bool, object]:
        """Whether unscale_ takes the MAX of the flag over a process group, and the group
        (None: the default group).

        Not under a ResidentGroup (this process saw every value there is).  An
        IpcGroup's ranks are processes: DDP's reductions (one- or two-shot) give
        each the same flag, but FSDP's ranks check different shards, so the flag
        is exchanged over the group's host process group (4 bytes)."""
        group = self.process_group
        if isinstance(group, comm.IpcGroup):
            return group.size() > 1, group.process_group
        if isinstance(group, comm.ResidentGroup):
            return False, None
        return comm.is_distributed() and comm.get_world_size(group) > 1, group

    def _new_flag_pair(self, device: torch.device):
        """Both flags, zeroed: in pinned host memory on a GPU (unless an RCCL group must
        exchange them, which needs device memory), else in ``device``'s memory."""
        exchange, group = self._flag_exchange()
        if device.type == "cuda" and (not exchange or dist.get_backend(group) == "gloo"):
            storage = torch.zeros(2, dtype=torch.int32, pin_memory=True)
            base = _native.host_device_address(storage.data_ptr())
            return (_HostFlag(storage[0:1], base, device), _HostFlag(storage[1:2], base + 4, device))
        storage = torch.zeros(2, dtype=torch.int32, device=device)
        return (storage[0:1], storage[1:2])

    def _next_flag(self, device: torch.device) -> torch.Tensor:
        """The flag the next step uses on ``device`` (which nothing reads or sets during this step).

        A producer that clears it in stream order with its own dispatch reports so
        with :meth:`_next_flag_cleared`; the next step then needs no clear of its own."""
        if device not in self._flags:
            self._flag(device)
        return self._flags[device][self._parity ^ 1]

    def _next_flag_cleared(self, device: torch.device) -> None:
        self._next_armed.add(device)

    def _begin_fused_unscale(
        self, device: torch.device, param_ids: frozenset, defer_clear: bool = False
    ) -> tuple[float, torch.Tensor] | tuple[float, torch.Tensor, bool]:
        """Hand a producer (DDP's unpack) the inverse scale and the device flag.

        The producer writes these params' grads already multiplied by
        ``1/scale`` and flags non-finite results; ``unscale_`` then skips them.
        Gradients must not be accumulated on top of unscaled values, so a
        second synchronised backward before ``step``/``update`` is an error.
        With ``defer_clear`` a third value says whether the producer must clear
        the flag (first producer of the step) before its kernels run."""
        if self._unscaled:
            raise RuntimeError("gradients were already unscaled this step; call update() first")
        if not all(ids.isdisjoint(param_ids) for ids in self._prescaled):
            raise RuntimeError(
                "a second synchronised backward ran before scaler.step()/update(): its gradients "
                "would accumulate onto already-unscaled ones"
            )
        self._prescaled.append(param_ids)
        flag, pending = self._flag(device, defer_clear)
        if defer_clear:
            return 1.0 / self._scale, flag, pending
        return 1.0 / self._scale, flag

    # -- the training-loop surface -----------------------------------------

    def scale_loss(self, loss: torch.Tensor) -> torch.Tensor:
        if not self.enabled:
            return loss
        return loss * self._scale

    scale_tensor = scale_loss

    def unscale_(self, optimizer: torch.optim.Optimizer) -> bool:
        """Divide gradients by the scale and detect overflow (amp.py:188-221).

        Idempotent within a step.  Returns whether any rank found an inf/NaN.
        """
        if not self.enabled:
            return False
        if self._unscaled:
            return self._found_inf_this_step

        inv_scale = _native.f32(1.0 / self._scale)
        device = comm.current_device()
        flag, _ = self._flag(device)

        prescaled = self._prescaled[0] if len(self._prescaled) == 1 else frozenset().union(*self._prescaled)
        groups: dict[torch.dtype, list[tuple[int, int, int]]] = {}
        for group in optimizer.param_groups:
            for p in group["params"]:
                if id(p) in prescaled:  # unscaled by a producer (a set lookup is cheaper than .grad)
                    continue
                g = p.grad
                if g is None:
                    continue
                _native.require_device_tensor(g, "gradient")
                if not g.is_contiguous():
                    raise RuntimeError("unscale_: gradient is not contiguous")
                groups.setdefault(g.dtype, []).append((g.data_ptr(), g.data_ptr(), g.numel()))
        stream = _native.stream_of(flag.device)
        for dtype, rows in groups.items():
            _native.unscale_found_inf(
                _native.spans_array(rows), _native.dtype_code(dtype), inv_scale, flag.data_ptr(), stream
            )

        if isinstance(flag, _HostFlag):
            flag.settle()
            flag = flag.host
        # The collective that makes the decision unanimous under FSDP / TP.
        exchange, group = self._flag_exchange()
        if exchange:
            comm.dist_all_reduce(flag, op=dist.ReduceOp.MAX, group=group)

        self._found_inf_this_step = bool(flag.item() > 0)
        self._unscaled = True
        return self._found_inf_this_step

    def step(self, optimizer: torch.optim.Optimizer) -> bool:
        """Run ``optimizer.step()`` unless the group agreed an overflow occurred."""
        self.num_steps += 1
        if not self.enabled:
            optimizer.step()
            return True
        found_inf = self.unscale_(optimizer)
        if found_inf:
            self.num_skipped += 1
            return False
        optimizer.step()
        return True

    def update(self) -> None:
        """Adapt the scale, then reset per-step state (amp.py:240-258)."""
        if not self.enabled:
            return
        if self._found_inf_this_step:
            self._scale = max(self._min_scale, self._scale * self._backoff_factor)
            self._good_steps = 0
        else:
            self._good_steps += 1
            if self._good_steps >= self._growth_interval:
                self._scale *= self._growth_factor
                self._good_steps = 0
        self._found_inf_this_step = False
        self._unscaled = False
        self._parity ^= 1
        self._flag_armed, self._next_armed = self._next_armed, set()
        self._prescaled.clear()

    def summary(self) -> str:
        if not self.enabled:
            return "grad scaler disabled (bf16 or fp32)"
        pct = 100.0 * self.num_skipped / max(1, self.num_steps)
        return f"scale={self._scale:g}  skipped={self.num_skipped}/{self.num_steps} ({pct:.1f}%)"
