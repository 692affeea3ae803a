"""Parameter-list shapes of the benchmark workloads.

Shapes in ``Module.parameters()`` order (namitorch/nn/module.py:150-209) of
the models the optimizer-step benchmarks are quoted on, plus the
weight-decay grouping of ``decay_parameter_groups``
(namitorch/training/runner.py:83-90: decay on ndim >= 2, none on vectors).
"""

from __future__ import annotations


def gpt2_shapes(vocab=50257, ctx=1024, d=768, layers=12, ffn=None) -> list[tuple[int, ...]]:
    """GPT-2 layout: tied head, learned positions, biases, LayerNorm weight+bias."""
    ffn = 4 * d if ffn is None else ffn
    shapes: list[tuple[int, ...]] = [(vocab, d), (ctx, d)]
    for _ in range(layers):
        shapes += [
            (d,), (d,),                 # ln_1 weight, bias
            (d, 3 * d), (3 * d,),       # attn c_attn
            (d, d), (d,),               # attn c_proj
            (d,), (d,),                 # ln_2 weight, bias
            (d, ffn), (ffn,),           # mlp c_fc
            (ffn, d), (d,),             # mlp c_proj
        ]
    shapes += [(d,), (d,)]              # ln_f
    return shapes


def gpt_1p3b_shapes() -> list[tuple[int, ...]]:
    return gpt2_shapes(vocab=50304, ctx=2048, d=2048, layers=24, ffn=8192)


def llama7b_shapes(vocab=32000, d=4096, layers=32, ffn=11008) -> list[tuple[int, ...]]:
    """Llama layout (RMSNorm weights, no biases, untied head)."""
    shapes: list[tuple[int, ...]] = [(vocab, d)]
    for _ in range(layers):
        shapes += [(d,), (d, d), (d, d), (d, d), (d, d), (d,), (ffn, d), (ffn, d), (d, ffn)]
    shapes += [(d,), (vocab, d)]
    return shapes


WORKLOADS = {
    "gpt2-124m": gpt2_shapes,
    "gpt-1.3b": gpt_1p3b_shapes,
    "llama-7b": llama7b_shapes,
}


def numel(shape: tuple[int, ...]) -> int:
    total = 1
    for dimension in shape:
        total *= dimension
    return total


def shard_shapes(shapes, world: int) -> list[tuple[int, ...]]:
    """One rank's share when every tensor's flat storage is split into
    `world` equal contiguous slices (the last rank's slices may be shorter;
    this returns the full-length ones)."""
    return [((numel(shape) + world - 1) // world,) for shape in shapes]


def total_params(shapes) -> int:
    return sum(numel(shape) for shape in shapes)


def decay_mask(shapes) -> list[bool]:
    """True where weight decay applies (ndim >= 2)."""
    return [len(shape) >= 2 for shape in shapes]
