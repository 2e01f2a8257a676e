"""Restickify placement: choose the stick of every buffer of a graph so that
the relayouts (restickifies) it needs move as few elements as possible.

Restates the reference's optimiser, torch_spyre/_inductor/optimize_restickify.py
(EdgeCostMap :43-112, AllSameNode :151-168, FixedInOutNode :171-203,
AnyInNode :206-224, greedy_local_min_cost :300-356, the beam search
BeamState / Frontier / beam_global_min_cost :375-503 with BEAM_WIDTH 64,
optimize_restickify_locations :506-514), over a small dataflow IR instead of
Inductor's, with the candidate-layout rules of
torch_spyre/_inductor/propagate_layouts.py: multi-argument pointwise
(:586-690), matmul (:522-579), single-argument ops and reductions
(:209-262), clone (:352-417).  The plan lists each restickify with its
target layout; its cost is the sum of the restickified buffers' sizes, as
the reference's tests count it (tests/inductor/test_restickify.py:42-48).

IR.  ``Buffer``s (graph inputs and op outputs) have a host size.  ``View``s
(``t``, ``transpose``, ``permute``, ``unsqueeze``, ``expand``) re-index a
buffer without a copy.  Every op runs over loop variables -- its output dims
``i0, i1, ...`` plus the dims it reduces -- and each input is read through an
access that maps the buffer's dims to loop variables (None for a broadcast
dim).  A buffer's layout is the dim that holds its stick (``SPARSE`` when no
dim does, after a reduction along the stick); the default is the last dim,
as the default SpyreTensorLayout tiling puts it.  The stick variable of an
access is the loop variable indexing the stick dim.

Edge cost of reading a buffer laid out ``L`` where the op needs stick
variable ``v`` (compute_restickify_needed, torch_spyre/_inductor/pass_utils.py:856-900):
0 if the access's stick variable is ``v`` (or the stick dim is the one the
op reduces and the output stick is sparse); the buffer's element count if
some dim of the buffer carries ``v`` (a restickify moves the stick there);
otherwise infinite ("no mechanism to gather / scatter", optimize_restickify.py:227-238).

Host logic only; the restickifies a plan lists run on the GPU through
``restickify`` (``schedule`` gives each as a source and target
SpyreTensorLayout).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import torch

from .layout import SpyreTensorLayout

INF = math.inf
SPARSE = -1
BEAM_WIDTH = 64


class NoFeasibleLayout(NotImplementedError):
    """No candidate output layout of an op has a finite cost (the reference's
    _no_feasible_layout_error, optimize_restickify.py:248-297)."""


@dataclass(frozen=True)
class Layout:
    """A buffer's stick placement: ``stick`` is the host dim holding the stick, or SPARSE."""

    size: Tuple[int, ...]
    stick: int

    @property
    def numel(self) -> int:
        return math.prod(self.size)

    def stl(self, dtype: torch.dtype = torch.float16) -> SpyreTensorLayout:
        """The SpyreTensorLayout of a contiguous host tensor of this size with
        the stick on ``stick`` (dim_order ends with it; -1 when sparse)."""
        n = len(self.size)
        strides = [math.prod(self.size[d + 1:]) for d in range(n)]
        if self.stick == SPARSE:
            order = list(range(n)) + [-1]
        else:
            order = [d for d in range(n) if d != self.stick] + [self.stick]
        return SpyreTensorLayout(list(self.size), strides, dtype, order)


@dataclass(eq=False)
class Buffer:
    name: str
    size: Tuple[int, ...]
    op: Optional["Op"] = None  # producer (None for a graph input)
    layouts: List[Layout] = field(default_factory=list)  # candidates, in preference order
    committed: Optional[Layout] = None

    @property
    def numel(self) -> int:
        return math.prod(self.size)


@dataclass(frozen=True)
class View:
    """A view of ``base``: view dim j is base dim ``dims[j]`` (None: a new
    broadcast dim of size ``size[j]``)."""

    base: Buffer
    dims: Tuple[Optional[int], ...]
    size: Tuple[int, ...]

    @staticmethod
    def of(x) -> "View":
        if isinstance(x, View):
            return x
        return View(x, tuple(range(len(x.size))), tuple(x.size))

    def permute(self, *order) -> "View":
        return View(self.base, tuple(self.dims[o] for o in order), tuple(self.size[o] for o in order))

    def transpose(self, d0: int, d1: int) -> "View":
        order = list(range(len(self.size)))
        order[d0], order[d1] = order[d1], order[d0]
        return self.permute(*order)

    def t(self) -> "View":
        return self.transpose(0, 1)

    def unsqueeze(self, d: int) -> "View":
        d = d % (len(self.size) + 1)
        return View(self.base, self.dims[:d] + (None,) + self.dims[d:], self.size[:d] + (1,) + self.size[d:])

    def expand(self, *size) -> "View":
        lead = len(size) - len(self.size)
        dims = (None,) * lead + self.dims
        out = []
        for j, s in enumerate(size):
            cur = 1 if j < lead else self.size[j - lead]
            out.append(cur if s == -1 else s)
        return View(self.base, dims, tuple(out))


@dataclass(frozen=True)
class Access:
    """How an op reads a buffer: base dim b is indexed by loop variable vars[b]."""

    buf: Buffer
    vars: Tuple[Optional[str], ...]

    def stick_var(self, layout: Layout) -> Optional[str]:
        return None if layout.stick == SPARSE else self.vars[layout.stick]

    def dim_of(self, var: str) -> Optional[int]:
        for b, v in enumerate(self.vars):
            if v == var:
                return b
        return None


def _access(view: View, out_vars: Sequence[Optional[str]]) -> Access:
    """Access of ``view`` whose dims are indexed by ``out_vars`` (one per view
    dim); broadcast dims (size-1 view dims or new dims) carry no variable."""
    vars_: List[Optional[str]] = [None] * len(view.base.size)
    for j, b in enumerate(view.dims):
        if b is not None and view.base.size[b] != 1:
            vars_[b] = out_vars[j]
    return Access(view.base, tuple(vars_))


# ---- cost nodes (optimize_restickify.py:43-224) ----------------------------

class EdgeCostMap:
    """Cost of one op input: (committed input layout, needed stick variable)
    -> 0 / buffer size / INF, with the restickify target layout."""

    def __init__(self, access: Access, reduced: Tuple[str, ...] = ()):
        self.access = access
        self.reduced = reduced

    def cost(self, in_layout: Layout, var: Optional[str]) -> float:
        have = self.access.stick_var(in_layout)
        if have == var:
            return 0.0
        if var is None and have in self.reduced:
            return 0.0  # reduction along the stick: the output stick is sparse
        if have is None or var is None:
            return INF  # no mechanism to gather into / scatter from one stick
        return float(self.access.buf.numel) if self.access.dim_of(var) is not None else INF

    def target(self, var: Optional[str]) -> Optional[Layout]:
        """Layout of the restickified input (stick on the dim carrying var)."""
        d = None if var is None else self.access.dim_of(var)
        return None if d is None else Layout(self.access.buf.size, d)


class AllSameNode:
    """Every input stick must match the output stick (pointwise, single-input ops)."""

    def __init__(self, edges: List[EdgeCostMap], out_var):
        self.edges = edges
        self.out_var = out_var  # Layout -> stick variable of the output

    def cost(self, in_layouts: Sequence[Layout], out: Layout) -> float:
        v = self.out_var(out)
        return sum(e.cost(l, v) for e, l in zip(self.edges, in_layouts))

    def required(self, out: Layout) -> List[Tuple[EdgeCostMap, Optional[str]]]:
        v = self.out_var(out)
        return [(e, v) for e in self.edges]


class FixedInOutNode:
    """Input and output sticks fixed by the op (matmul)."""

    def __init__(self, edges: List[EdgeCostMap], out_layout: Layout, req_vars: List[str]):
        self.edges = edges
        self.out_layout = out_layout
        self.req_vars = req_vars

    def cost(self, in_layouts: Sequence[Layout], out: Layout) -> float:
        if out != self.out_layout:
            return INF
        return sum(e.cost(l, v) for e, l, v in zip(self.edges, in_layouts, self.req_vars))

    def required(self, out: Layout) -> List[Tuple[EdgeCostMap, Optional[str]]]:
        return list(zip(self.edges, self.req_vars))


class AnyInNode:
    """Any input layout, fixed output layout (clone: it relays by itself)."""

    edges: List[EdgeCostMap] = []

    def cost(self, in_layouts, out) -> float:
        return 0.0

    def required(self, out):
        return []


@dataclass(eq=False)
class Op:
    name: str
    kind: str
    accesses: List[Access]
    out: Buffer
    cost_fn: object = None


# ---- graph construction with candidate layouts (propagate_layouts.py) ------

class Graph:
    """Ops in topological order (each built from already-built values)."""

    def __init__(self):
        self.inputs: List[Buffer] = []
        self.ops: List[Op] = []
        self._n = 0

    def input(self, name: str, size: Sequence[int]) -> Buffer:
        b = Buffer(name, tuple(int(s) for s in size))
        b.layouts = [Layout(b.size, len(b.size) - 1)]  # as transferred: default tiling
        self.inputs.append(b)
        return b

    def _new(self, kind: str, size) -> Buffer:
        self._n += 1
        return Buffer(f"buf{self._n - 1}", tuple(size))

    @staticmethod
    def _out_vars(r: int) -> List[str]:
        return [f"i{d}" for d in range(r)]

    def pointwise(self, *xs, kind: str = "add") -> Buffer:
        """A multi- or single-input pointwise op (add, mul, exp, ...) with
        numpy broadcasting (_multi_arg_pointwise_layouts / _single_arg_op_layout)."""
        views = [View.of(x) for x in xs]
        r = max(len(v.size) for v in views)
        size = []
        for d in range(r):
            s = 1
            for v in views:
                j = d - (r - len(v.size))
                if j >= 0 and v.size[j] != 1:
                    s = v.size[j]
            size.append(s)
        ov = self._out_vars(r)
        accesses = [_access(v, ov[r - len(v.size):]) for v in views]
        out = self._new(kind, size)
        # Candidate output sticks: every input's stick variable over all its
        # candidate layouts, in loop-variable order; none -> the last dim.
        sticks = sorted({a.stick_var(l) for a in accesses for l in a.buf.layouts} - {None},
                        key=lambda v: int(v[1:]))
        out.layouts = [Layout(out.size, int(v[1:])) for v in sticks] or [Layout(out.size, r - 1)]
        edges = [EdgeCostMap(a) for a in accesses]
        var_of = lambda l: None if l.stick == SPARSE else ov[l.stick]  # noqa: E731
        op = Op(f"op_{out.name}", kind, accesses, out, AllSameNode(edges, var_of))
        return self._add(op)

    def add(self, x, y) -> Buffer:
        return self.pointwise(x, y, kind="add")

    def matmul(self, x, y) -> Buffer:
        """x [..., M, K] @ y [..., K, N] (_matmul_layouts): x's stick on the
        reduction variable, y's on the generated one; output stick on N."""
        xv, yv = View.of(x), View.of(y)
        bx, by = xv.size[:-2], yv.size[:-2]
        rb = max(len(bx), len(by))
        batch = [max(a, b) for a, b in zip((1,) * (rb - len(bx)) + bx, (1,) * (rb - len(by)) + by)]
        size = batch + [xv.size[-2], yv.size[-1]]
        ov = self._out_vars(len(size))
        xa = _access(xv, ov[rb - len(bx):rb] + [ov[rb], "k"])
        ya = _access(yv, ov[rb - len(by):rb] + ["k", ov[rb + 1]])
        out = self._new("matmul", size)
        out_layout = Layout(out.size, len(size) - 1)
        out.layouts = [out_layout]
        fn = FixedInOutNode([EdgeCostMap(xa), EdgeCostMap(ya)], out_layout, ["k", ov[rb + 1]])
        return self._add(Op(f"op_{out.name}", "matmul", [xa, ya], out, fn))

    def sum(self, x, dim: int) -> Buffer:
        """Reduction over ``dim`` (single-argument op layouts, :226-262): an
        input stick on a kept dim passes through; on the reduced dim the
        output stick is sparse."""
        xv = View.of(x)
        dim = dim % len(xv.size)
        size = [s for d, s in enumerate(xv.size) if d != dim]
        ov = self._out_vars(len(size))
        vars_ = ov[:dim] + ["r"] + ov[dim:]
        a = _access(xv, vars_)
        out = self._new("sum", size)
        cands = []
        for l in a.buf.layouts:
            v = a.stick_var(l)
            cand = Layout(out.size, SPARSE if v in (None, "r") else int(v[1:]))
            if cand not in cands:
                cands.append(cand)
        out.layouts = cands
        var_of = lambda l: None if l.stick == SPARSE else ov[l.stick]  # noqa: E731
        fn = AllSameNode([EdgeCostMap(a, reduced=("r",))], var_of)
        return self._add(Op(f"op_{out.name}", "sum", [a], out, fn))

    def clone(self, x) -> Buffer:
        """clone: materialises the default layout from any input (AnyInNode)."""
        xv = View.of(x)
        a = _access(xv, self._out_vars(len(xv.size)))
        out = self._new("clone", xv.size)
        out.layouts = [Layout(out.size, len(out.size) - 1)]
        return self._add(Op(f"op_{out.name}", "clone", [a], out, AnyInNode()))

    def _add(self, op: Op) -> Buffer:
        op.out.op = op
        self.ops.append(op)
        return op.out


# ---- optimisers (optimize_restickify.py:300-514) ---------------------------

def _no_feasible(op: Op) -> NoFeasibleLayout:
    ins = ", ".join(f"{a.buf.name} stick {a.buf.committed.stick if a.buf.committed else '?'}" for a in op.accesses)
    return NoFeasibleLayout(f"{op.name} ({op.kind}): no candidate output layout is reachable from inputs [{ins}]")


def greedy_local_min_cost(graph: Graph) -> None:
    """Topological order; each op commits its cheapest candidate given its
    inputs' committed layouts (ties: the first candidate)."""
    for b in graph.inputs:
        b.committed = b.layouts[0]
    for op in graph.ops:
        ins = [a.buf.committed for a in op.accesses]
        best, best_cost = None, INF
        for cand in op.out.layouts:
            c = op.cost_fn.cost(ins, cand)
            if c < best_cost:
                best, best_cost = cand, c
        if best is None:
            raise _no_feasible(op)
        op.out.committed = best


@dataclass
class BeamState:
    """A partial assignment of layouts (parallel to Frontier.buf_names) and its cost."""

    assignments: tuple
    cost: float


class Frontier:
    def __init__(self, K: int):
        self.K = K
        self.buf_names: List[str] = []
        self._idx: Dict[str, int] = {}
        self.states: List[BeamState] = [BeamState((), 0.0)]

    def add_buf(self, name: str) -> None:
        self._idx[name] = len(self.buf_names)
        self.buf_names.append(name)

    def input_layout(self, state: BeamState, name: str) -> Layout:
        return state.assignments[self._idx[name]]

    def best(self) -> BeamState:
        return self.states[0]

    def trim(self) -> None:
        self.states.sort(key=lambda s: s.cost)  # stable: earlier candidates win ties
        self.states = self.states[: self.K]


def beam_global_min_cost(graph: Graph, beam_width: Optional[int] = None) -> int:
    """Beam search over every op's candidate layouts, keeping the
    ``beam_width`` cheapest partial assignments after each op; commits the
    best.  Returns the largest beam size reached."""
    frontier = Frontier(BEAM_WIDTH if beam_width is None else beam_width)
    for b in graph.inputs:
        b.committed = b.layouts[0]
        frontier.add_buf(b.name)
        frontier.states = [BeamState(s.assignments + (b.committed,), s.cost) for s in frontier.states]
    max_states = 1
    for op in graph.ops:
        frontier.add_buf(op.out.name)
        nxt = []
        for s in frontier.states:
            ins = [frontier.input_layout(s, a.buf.name) for a in op.accesses]
            for cand in op.out.layouts:
                c = op.cost_fn.cost(ins, cand)
                if c < INF:
                    nxt.append(BeamState(s.assignments + (cand,), s.cost + c))
        if not nxt:
            raise _no_feasible(op)
        frontier.states = nxt
        frontier.trim()
        max_states = max(max_states, len(frontier.states))
    bufs = {b.name: b for b in graph.inputs}
    bufs.update({op.out.name: op.out for op in graph.ops})
    for name, layout in zip(frontier.buf_names, frontier.best().assignments):
        bufs[name].committed = layout
    return max_states


def finalize_layouts(graph: Graph) -> Dict[str, List[dict]]:
    """The restickify plan of the committed layouts: op name -> one entry per
    input to relay ({"input", "source_layout", "target_layout", "cost"})."""
    plan: Dict[str, List[dict]] = {}
    for op in graph.ops:
        for edge, var in op.cost_fn.required(op.out.committed):
            src = edge.access.buf.committed
            c = edge.cost(src, var)
            if c == 0:
                continue
            if c == INF:
                raise _no_feasible(op)
            plan.setdefault(op.name, []).append(
                {"input": edge.access.buf.name, "source_layout": src, "target_layout": edge.target(var), "cost": c})
    return plan


def optimize_restickify_locations(graph: Graph, global_optimizer: bool = True) -> Dict[str, List[dict]]:
    """Commits a layout to every buffer (beam search, or greedy) and returns
    the restickify plan."""
    if global_optimizer:
        beam_global_min_cost(graph)
    else:
        greedy_local_min_cost(graph)
    return finalize_layouts(graph)


def plan_cost(plan: Dict[str, List[dict]]) -> int:
    """Elements moved by the plan's restickifies (test_restickify.py:42-48)."""
    return sum(math.prod(e["target_layout"].size) for entries in plan.values() for e in entries)


def schedule(plan: Dict[str, List[dict]], dtype: torch.dtype = torch.float16):
    """The plan as (op name, input buffer, source STL, target STL) tuples, in
    op order: each one is a ``relayout.restickify`` of that buffer."""
    return [(op, e["input"], e["source_layout"].stl(dtype), e["target_layout"].stl(dtype))
            for op, entries in plan.items() for e in entries]
