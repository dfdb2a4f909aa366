"""Nested batch axes folded into the library's one flat batch (splax/_batching.py:32-115).

The reference's kernels take one batch axis, so ``nested_vmap`` flattens nested ``jax.vmap``
axes into it, outer axis major (splax/_batching.py:75-103): an operand batched over every axis is
reshaped, one batched over some axes only is tiled (batched over the inner axes) or repeated
(batched over the outer ones) to the full batch, and an unbatched operand stays shared by every
image. Here the axes are the operands' leading dimensions, aligned from the right as in
broadcasting: the batch shape is the broadcast of every operand's leading shape, an operand whose
leading shape is that whole shape is reshaped to one flat axis, one with a partial leading shape
(size-1 or missing axes) is expanded to it first (the tile / repeat rule), and one with no
leading dimensions (or only size-1 ones) stays shared. Gradients of expanded operands sum over
the expanded axes (autograd of ``expand``); shared operands are folded by the library itself.
"""

from __future__ import annotations

import math

import torch


def batch_shape(named: dict[str, tuple[torch.Tensor | None, int]]) -> tuple[int, ...]:
    """Broadcast of the leading shapes (the dims before each operand's ``base_ndim`` trailing
    ones); raises ValueError like the reference when the operands disagree."""
    leads = []
    for name, (t, base) in named.items():
        if t is None:
            continue
        if t.ndim < base:
            raise ValueError(f"{name}: expected at least {base} dims, got {tuple(t.shape)}")
        leads.append((name, tuple(t.shape[: t.ndim - base])))
    try:
        return tuple(torch.broadcast_shapes(*(lead for _, lead in leads)))
    except RuntimeError as e:
        raise ValueError("inconsistent batch shapes: " +
                         ", ".join(f"{n}{lead}" for n, lead in leads)) from e


def shared_background(background: torch.Tensor) -> torch.Tensor:
    """A background whose leading dims are all of size 1 as one shared (3,) colour: the
    reference reshapes its background to (1, 3) inside rasterize
    (splax/_rasterize/_rasterize.py:131), so a (1, 3) background renders an unbatched image, and
    such size-1 dims are no batch axes."""
    if background.ndim > 1 and math.prod(background.shape[:-1]) == 1:
        return background.reshape(background.shape[-1])
    return background


def fold(t: torch.Tensor | None, base: int, shape: tuple[int, ...],
         expand_shared: bool = False) -> torch.Tensor | None:
    """``t`` with its leading dims folded into one flat axis of prod(shape) rows, outer axis
    major; an operand without leading dims (or with only size-1 ones) stays shared (its base
    shape) unless ``expand_shared``."""
    if t is None:
        return None
    base_shape = tuple(t.shape[t.ndim - base:]) if base else ()
    lead = tuple(t.shape[: t.ndim - base])
    flat = math.prod(shape)
    if not shape:
        return t
    if math.prod(lead) == 1 and not expand_shared:
        return t.reshape(base_shape)
    if lead != shape:  # partially batched: tile / repeat to the full batch
        t = t.reshape((1,) * (len(shape) - len(lead)) + lead + base_shape)
        t = t.expand(shape + base_shape)
    return t.reshape((flat,) + base_shape)
