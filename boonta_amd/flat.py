"""Flat parameter storage of the learner.

Every parameter leaf lives at a 256-byte aligned offset of one fp32 buffer;
the gradient, Adam mu and Adam nu buffers share that layout, so the optimizer
is one bandwidth-bound pass over four flat arrays.  Dense kernels keep flax's
[in, out] orientation with the output axis padded to a multiple of 4 floats
(16-byte rows for the GEMM loads).  When the actor and critic heads read the
same features, their kernels share one [in, A+1 (padded)] matrix (actor
columns first, the value column after), so one GEMM computes logits and value;
the leaves the user sees are strided views into it.  Padding is zero in every
buffer and stays zero (its gradient is zero, so Adam leaves it at zero).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

ALIGN = 64  # floats


def round_up(x: int, m: int) -> int:
    return (x + m - 1) // m * m


@dataclass
class Leaf:
    path: tuple            # full path inside params["params"], ending in the leaf name
    offset: int            # element offset of the view's first element
    shape: tuple
    strides: tuple


@dataclass
class Region:
    offset: int
    rows: int
    ld: int                # row pitch (elements)

    @property
    def size(self) -> int:
        return self.rows * self.ld


@dataclass
class FlatLayout:
    leaves: dict = field(default_factory=dict)   # path -> Leaf
    size: int = 0

    def region(self, rows: int, ld: int) -> Region:
        off = round_up(self.size, ALIGN)
        self.size = off + rows * ld
        return Region(off, rows, ld)

    def add_leaf(self, path, offset, shape, strides):
        self.leaves[tuple(path)] = Leaf(tuple(path), offset, tuple(shape), tuple(strides))

    def finish(self):
        self.size = round_up(max(self.size, 4), ALIGN)


def tree_from_flat(layout: FlatLayout, buf: torch.Tensor) -> dict:
    """Nested dict of strided views into ``buf`` following the leaf paths."""
    out: dict = {}
    for path, lf in layout.leaves.items():
        node = out
        for k in path[:-1]:
            node = node.setdefault(k, {})
        node[path[-1]] = torch.as_strided(buf, lf.shape, lf.strides, lf.offset)
    return out


def load_tree(layout: FlatLayout, buf: torch.Tensor, tree: dict):
    """Copies a nested dict of arrays (numpy or torch) into the flat buffer."""
    views = tree_from_flat(layout, buf)

    def walk(dst, src, path):
        for k, v in dst.items():
            if isinstance(v, dict):
                walk(v, src[k], path + (k,))
            else:
                s = src[k]
                t = s if isinstance(s, torch.Tensor) else torch.from_numpy(np.asarray(s, np.float32))
                if tuple(t.shape) != tuple(v.shape):
                    raise ValueError(f"leaf {'/'.join(path + (k,))}: shape {tuple(t.shape)} != {tuple(v.shape)}")
                v.copy_(t.to(device=v.device, dtype=v.dtype))

    walk(views, tree, ())


def tree_to_numpy(tree) -> dict:
    if isinstance(tree, dict):
        return {k: tree_to_numpy(v) for k, v in tree.items()}
    return tree.detach().cpu().numpy().copy()
