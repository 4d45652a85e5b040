"""minidist for MI355X -- the per-rank gradient-communication path on gfx950 kernels.

A drop-in for the data-parallel gradient path of the reference ``minidist``
(minidist/__init__.py): the DDP bucketer, the collective grad scaler, the FSDP
flat-parameter unit and the collective hook keep their names, signatures and
hook semantics; their data movement runs as hand-written HIP kernels in
``libmdx.so`` (C ABI: include/mdx.h).

:mod:`minidist.profiling` keeps the reference's collective breakdown and
overlap analysis, and knows the path's own kernels as collectives.  Names
of the reference outside this path (tensor / pipeline parallelism, the 3D
mesh) are not part of this package; importing one raises an ImportError
that says so.
"""

from .amp import DistributedGradScaler, PrecisionConfig, resolve_precision
from .comm import (
    IpcGroup,
    ResidentGroup,
    barrier,
    comm_stats,
    get_rank,
    get_world_size,
    init_distributed,
    is_primary,
    print_rank0,
    record_comm,
    shutdown_distributed,
)
from .ddp import DDP, DistributedDataParallel
from .fsdp import FSDP, FullyShardedDataParallel, MixedPrecisionPolicy
from .profiling import analyze_kernel_trace, analyze_trace, format_collective_table, profile_steps, summarize_collectives

__version__ = "0.1.0"

_OUT_OF_SCOPE = {
    "ParallelMesh",
    "PipelineStage",
    "build_schedule",
    "partition_layers",
    "theoretical_bubble_fraction",
    "ColumnParallelLinear",
    "RowParallelLinear",
    "VocabParallelEmbedding",
    "vocab_parallel_cross_entropy",
}


def __getattr__(name: str):
    if name in _OUT_OF_SCOPE:
        raise ImportError(
            f"minidist.{name} belongs to the reference's tensor/pipeline/mesh layers, which this "
            "build does not provide (it implements the data-parallel gradient path only)"
        )
    raise AttributeError(f"module 'minidist' has no attribute {name!r}")


__all__ = [
    "DDP",
    "DistributedDataParallel",
    "FSDP",
    "FullyShardedDataParallel",
    "MixedPrecisionPolicy",
    "DistributedGradScaler",
    "PrecisionConfig",
    "ResidentGroup",
    "IpcGroup",
    "resolve_precision",
    "init_distributed",
    "shutdown_distributed",
    "barrier",
    "get_rank",
    "get_world_size",
    "is_primary",
    "print_rank0",
    "comm_stats",
    "record_comm",
    "profile_steps",
    "summarize_collectives",
    "format_collective_table",
    "analyze_trace",
    "analyze_kernel_trace",
    "__version__",
]
