"""Random programs over the Tensor API, evaluated twice: by the device under
test and by an independent float64 numpy interpreter of the same ops.

The numpy side restates each op's meaning from the reference's definitions,
not from this build's C++ front end: broadcasting binary ops and keep-dim
reductions (tensor.rs:461-479, 665-681, 1068-1092), relu as
Where(0 < x, x, 0) (tensor.rs:517-531), Max as (a > b) ? a : b, matmul as the
broadcast product summed over k (tensor.rs:762-778), log_softmax as
(x - max) - log(sum(exp(x - max))) (tensor.rs:715-743), views (permute,
reshape, expand, narrow: shape.rs). So a mistake in the shared front end
(schedule, rangeify, index rules, fusions) that the oracle would repeat shows
up here as a disagreement.

Alongside each value the interpreter carries a magnitude: an upper bound of
the absolute terms that feed each element (sums of |terms| for add, sum and
matmul, products of magnitudes for mul, the row maximum for max and
log_softmax, exp's derivative for exp; sqrt, 1/z and log of z = x*x + 1 add
z's bound times the derivative at z). An element passes when
|got - want| <= 1e-4 * magnitude + 1e-6: f32 rounding over these short
programs stays orders of magnitude inside that, and an indexing or
partitioning mistake moves elements by their own size."""
from __future__ import annotations

import numpy as np

SHAPES = [(4, 6), (6, 4), (3, 4, 5), (8, 16), (16, 8), (2, 3, 4, 2), (32,), (5, 7)]
# Above the small-kernel limits (4096 outputs), so the row-reduce,
# column-reduce, elementwise and GEMM kernel classes render too.
LARGE_SHAPES = [(64, 96), (96, 64), (128, 48), (16, 24, 20), (256, 32), (32, 256), (6, 8, 10, 12), (5000,)]
# Unit axes and extents off every lane, tile and workgroup multiple, on both
# sides of the one-workgroup limits.
ODD_SHAPES = [(1, 7), (7, 1), (1, 1), (3, 1, 5), (33, 17), (1, 4099), (4099, 1), (1031, 3), (3, 1031), (65, 65), (1,)]


class Node:
    def __init__(self, t, v, m):
        self.t, self.v, self.m = t, v, m  # device tensor, float64 value, float64 magnitude


_LEAVES = []  # the leaves of the program random_program is building


def leaf(fg, dev, rng, shape):
    a = rng.uniform(-1, 1, shape).astype(np.float32)
    v = a.astype(np.float64)
    n = Node(fg.Tensor.new(a, list(shape), dev), v, np.abs(v))
    _LEAVES.append(n)
    return n


def _scalar(fg, dev, c):
    return fg.Tensor.scalar(float(np.float32(c)), dev)


def random_program(fg, dev, seed, depth=7, large=False, leaves=None, odd=False):
    """Build a random program; returns the nodes to realise (the last one and
    up to two earlier ones). `large` draws from LARGE_SHAPES, `odd` from
    ODD_SHAPES; `leaves`, a list, receives the program's input nodes."""
    rng = np.random.default_rng(seed)
    _LEAVES.clear()
    shapes = ODD_SHAPES if odd else LARGE_SHAPES if large else SHAPES
    widths = [1, 3, 33] if odd else [3, 64, 96, 130] if large else [3, 5, 8]
    pool = [leaf(fg, dev, rng, shapes[rng.integers(len(shapes))]) for _ in range(2)]
    for _ in range(depth):
        x = pool[rng.integers(len(pool))]
        shape = x.v.shape
        op = rng.choice(["unary", "binary", "bcast", "reduce", "permute", "reshape", "narrow", "matmul",
                         "log_softmax", "contiguous"])
        out = None
        if op == "unary":
            u = rng.choice(["neg", "relu", "exp", "scale", "sqrt1p", "recip1p", "log1p"])
            if u == "neg":
                out = Node(x.t.neg(), -x.v, x.m)
            elif u == "relu":
                out = Node(x.t.relu(), np.where(0 < x.v, x.v, 0.0), x.m)
            elif u == "exp":
                # exp of a damped input keeps values bounded
                c = 0.5 / max(1.0, float(np.max(np.abs(x.v))))
                y, ym = x.v * np.float32(c), x.m * abs(np.float32(c))
                e = np.exp(y)
                out = Node(x.t.mul(_scalar(fg, dev, c)).exp(), e, e * (1.0 + ym))
            elif u == "scale":
                c = float(rng.choice([0.5, -2.0, 0.125, 3.0]))
                out = Node(x.t.mul(_scalar(fg, dev, c)), x.v * c, x.m * abs(c))
            else:
                # f(x*x + 1) for f = sqrt, 1/z, log: z >= 1 keeps each defined;
                # the magnitude adds z's own bound times |f'(z)|.
                z = x.v * x.v + 1.0
                zm = 2 * x.m * np.abs(x.v) + 1.0
                zt = x.t.mul(x.t).add(_scalar(fg, dev, 1.0))
                if u == "sqrt1p":
                    out = Node(zt.sqrt(), np.sqrt(z), np.sqrt(z) + zm / (2 * np.sqrt(z)))
                elif u == "recip1p":
                    out = Node(zt.reciprocal(), 1.0 / z, 1.0 / z + zm / (z * z))
                else:
                    out = Node(zt.log(), np.log(z), np.log(z) + zm / z + 1.0)
        elif op == "binary":
            same = [p for p in pool if p.v.shape == shape and p is not x]
            y = same[rng.integers(len(same))] if same and rng.random() < 0.6 else leaf(fg, dev, rng, shape)
            b = rng.choice(["add", "sub", "mul"])
            if b == "add":
                out = Node(x.t.add(y.t), x.v + y.v, x.m + y.m)
            elif b == "sub":
                out = Node(x.t.sub(y.t), x.v - y.v, x.m + y.m)
            else:
                out = Node(x.t.mul(y.t), x.v * y.v, x.m * y.m)
        elif op == "bcast" and len(shape) >= 2:
            axes = sorted(rng.choice(len(shape), size=rng.integers(1, len(shape)), replace=False).tolist())
            y = leaf(fg, dev, rng, shape)
            r = y.t.sum(axes)
            rv, rm = y.v.sum(axis=tuple(axes), keepdims=True), y.m.sum(axis=tuple(axes), keepdims=True)
            if rng.random() < 0.5:
                out = Node(x.t.add(r), x.v + rv, x.m + rm)  # broadcast by the binary op
            else:
                out = Node(x.t.mul(r.expand(list(shape))), x.v * rv, x.m * rm)
        elif op == "reduce":
            axes = sorted(rng.choice(len(shape), size=rng.integers(1, len(shape) + 1), replace=False).tolist())
            if rng.random() < 0.5:
                out = Node(x.t.sum(axes), x.v.sum(axis=tuple(axes), keepdims=True),
                           x.m.sum(axis=tuple(axes), keepdims=True))
            else:
                out = Node(x.t.max(axes), x.v.max(axis=tuple(axes), keepdims=True),
                           x.m.max(axis=tuple(axes), keepdims=True))
        elif op == "permute" and len(shape) >= 2:
            order = rng.permutation(len(shape)).tolist()
            out = Node(x.t.permute(order), x.v.transpose(order), x.m.transpose(order))
        elif op == "reshape":
            # Squeezes and unsqueezes only: the reference's index rules take any
            # other reshape only over a one-dimensional buffer (indexing.rs:143-169).
            dims = list(shape)
            ones = [i for i, d in enumerate(dims) if d == 1]
            if ones and len(dims) > 1 and rng.random() < 0.5:
                i = int(rng.choice(ones))
                new = dims[:i] + dims[i + 1:]
            else:
                i = int(rng.integers(len(dims) + 1))
                new = dims[:i] + [1] + dims[i:]
            out = Node(x.t.reshape(new), x.v.reshape(new), x.m.reshape(new))
        elif op == "narrow":
            ax = [i for i, d in enumerate(shape) if d > 1]
            if not ax:
                continue
            d = int(rng.choice(ax))
            start = int(rng.integers(shape[d] - 1))
            length = int(rng.integers(1, shape[d] - start + 1))
            sl = [slice(None)] * len(shape)
            sl[d] = slice(start, start + length)
            out = Node(x.t.narrow(d, start, length), x.v[tuple(sl)], x.m[tuple(sl)])
        elif op == "matmul" and len(shape) == 2:
            n = int(rng.choice(widths))
            y = leaf(fg, dev, rng, (shape[1], n))
            out = Node(x.t.matmul(y.t), x.v @ y.v, x.m @ y.m)
        elif op == "log_softmax" and len(shape) == 2:
            ax = int(rng.integers(2))
            mx = x.v.max(axis=ax, keepdims=True)
            s = np.exp(x.v - mx).sum(axis=ax, keepdims=True)
            mag = 4.0 * x.m.max(axis=ax, keepdims=True) + 1.0
            out = Node(x.t.log_softmax(ax), (x.v - mx) - np.log(s), np.broadcast_to(mag, x.v.shape))
        elif op == "contiguous":
            out = Node(x.t.contiguous(), x.v, x.m)
        if out is not None:
            assert out.t.shape == out.v.shape, (op, out.t.shape, out.v.shape)
            pool.append(out)
    # Realised together, producers first: schedule_many compiles roots in the
    # order given and replaces each only after compiling it
    # (schedule.rs:118-133), so a root listed before one it reads would
    # inline that root's reduction as a nested reduce.
    idx = sorted(set(rng.choice(len(pool) - 1, size=min(2, len(pool) - 1), replace=False).tolist()) | {len(pool) - 1})
    if leaves is not None:
        leaves.extend(_LEAVES)
    _LEAVES.clear()
    return [pool[i] for i in idx]


def check(nodes, fg):
    """Realise the nodes together; the worst |got - want| / bound."""
    fg.Tensor.realize_many([n.t for n in nodes])
    worst = 0.0
    for n in nodes:
        got = n.t.numpy().astype(np.float64).reshape(n.v.shape)
        bound = 1e-4 * n.m + 1e-6
        worst = max(worst, float(np.max(np.abs(got - n.v) / bound)))
    return worst
