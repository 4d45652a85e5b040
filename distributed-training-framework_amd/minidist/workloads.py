"""Parameter tables of the benchmark / test workloads, in registration order.

The bucket layout of DDP and the unit layout of FSDP depend only on the
ordered list of parameter shapes and dtypes, so the workloads are described
by that list.  GPT shapes follow the reference model's registration order
(minidist/models/gpt.py:169-224 with weight-then-bias linears,
minidist/tensor_parallel.py:246-420): ``nn.Module.parameters()`` yields a
module's own parameters before its children's, so the embedding's ``wpe``
comes before ``wte.weight``.  The Llama table is the standard decoder layout
the Llama-7B benchmark configuration names (the reference has no Llama model).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch


@dataclass(frozen=True)
class ParamSpec:
    name: str
    shape: tuple[int, ...]
    dtype: torch.dtype = torch.float32

    @property
    def numel(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    @property
    def nbytes(self) -> int:
        return self.numel * torch.empty((), dtype=self.dtype).element_size()


def gpt_block_specs(layer: int, h: int, dtype: torch.dtype = torch.float32) -> list[ParamSpec]:
    """One pre-norm block: ln1, attn.qkv, attn.proj, ln2, mlp.fc, mlp.proj (gpt.py:153-166)."""
    p = f"blocks.{layer}"
    return [
        ParamSpec(f"{p}.ln1.weight", (h,), dtype),
        ParamSpec(f"{p}.ln1.bias", (h,), dtype),
        ParamSpec(f"{p}.attn.qkv.weight", (3 * h, h), dtype),
        ParamSpec(f"{p}.attn.qkv.bias", (3 * h,), dtype),
        ParamSpec(f"{p}.attn.proj.weight", (h, h), dtype),
        ParamSpec(f"{p}.attn.proj.bias", (h,), dtype),
        ParamSpec(f"{p}.ln2.weight", (h,), dtype),
        ParamSpec(f"{p}.ln2.bias", (h,), dtype),
        ParamSpec(f"{p}.mlp.fc.weight", (4 * h, h), dtype),
        ParamSpec(f"{p}.mlp.fc.bias", (4 * h,), dtype),
        ParamSpec(f"{p}.mlp.proj.weight", (h, 4 * h), dtype),
        ParamSpec(f"{p}.mlp.proj.bias", (h,), dtype),
    ]


def gpt_specs(
    n_layer: int, n_embd: int, vocab: int, ctx: int, untied_head: bool = False, dtype: torch.dtype = torch.float32
) -> list[ParamSpec]:
    """Whole GPT in ``parameters()`` order; ``untied_head`` adds lm_head.head.weight."""
    h = n_embd
    specs = [
        ParamSpec("embedding.wpe", (ctx, h), dtype),
        ParamSpec("embedding.wte.weight", (vocab, h), dtype),
    ]
    for i in range(n_layer):
        specs += gpt_block_specs(i, h, dtype)
    specs += [ParamSpec("lm_head.ln_f.weight", (h,), dtype), ParamSpec("lm_head.ln_f.bias", (h,), dtype)]
    if untied_head:
        specs.append(ParamSpec("lm_head.head.weight", (vocab, h), dtype))
    return specs


def llama_specs(
    n_layer: int = 32, h: int = 4096, ffn: int = 11008, vocab: int = 32000, dtype: torch.dtype = torch.bfloat16
) -> list[ParamSpec]:
    """Llama decoder: embed, per layer (attn_norm, q, k, v, o, ffn_norm, gate, up, down), norm, head."""
    specs = [ParamSpec("embed.weight", (vocab, h), dtype)]
    for i in range(n_layer):
        p = f"layers.{i}"
        specs += [
            ParamSpec(f"{p}.attn_norm.weight", (h,), dtype),
            ParamSpec(f"{p}.attn.q.weight", (h, h), dtype),
            ParamSpec(f"{p}.attn.k.weight", (h, h), dtype),
            ParamSpec(f"{p}.attn.v.weight", (h, h), dtype),
            ParamSpec(f"{p}.attn.o.weight", (h, h), dtype),
            ParamSpec(f"{p}.ffn_norm.weight", (h,), dtype),
            ParamSpec(f"{p}.ffn.gate.weight", (ffn, h), dtype),
            ParamSpec(f"{p}.ffn.up.weight", (ffn, h), dtype),
            ParamSpec(f"{p}.ffn.down.weight", (h, ffn), dtype),
        ]
    specs += [ParamSpec("norm.weight", (h,), dtype), ParamSpec("lm_head.weight", (vocab, h), dtype)]
    return specs


# The benchmark configurations (cfg0..cfg4) the bench and the full-size tests use.
TINY_GPT = dict(n_layer=4, n_embd=256, vocab=1024, ctx=128)        # cfg0, W=4
GPT2_SMALL = dict(n_layer=12, n_embd=768, vocab=50257, ctx=1024)    # cfg1, W=8
GPT2_MEDIUM = dict(n_layer=24, n_embd=1024, vocab=50257, ctx=1024)  # cfg2, W=4
GPT2_XL = dict(n_layer=48, n_embd=1600, vocab=50257, ctx=1024)      # cfg3, W=8 (FSDP)
LLAMA_7B = dict(n_layer=32, h=4096, ffn=11008, vocab=32000)         # cfg4, W=8 (bf16)


def total_numel(specs: list[ParamSpec]) -> int:
    return sum(s.numel for s in specs)


class SpecModule(torch.nn.Module):
    """A module whose parameters have the given specs' shapes and dtypes, registered in order.

    Values are left uninitialised: DDP's bucket layout and FSDP's unit layout
    depend only on the ordered shapes and dtypes, and the workloads supply the
    gradients themselves."""

    def __init__(self, specs: list[ParamSpec], device: torch.device | str):
        super().__init__()
        self.specs = list(specs)
        self.ps = torch.nn.ParameterList(
            [torch.nn.Parameter(torch.empty(s.shape, dtype=s.dtype, device=device)) for s in specs]
        )
