"""Host-side lowering of jasmine expression trees to the jas_ew_eval postfix program (Python mirror).

Mirrors what the C++ header API does at a tree's evaluation point (clone / operator
mat_t): node ele_types follow std::common_type over double > float > int
(mat_express_t.hpp:41-44), scalars become CONST nodes of their own type (a scalar operand
is stored as a 1x1 mat_t<T>, :18-33), the node shape is the elementwise max of the
children's shapes (:51-59), and operands are emitted in Sethi-Ullman order (deeper
operand first, swap flag on the binary op) so the device stack stays within 4 slots.
"""
from dataclasses import dataclass, field
from typing import Optional

F32, F64, I32, BF16 = 0, 1, 2, 3
# bf16 with bf16 or int stays bf16; with float or double it widens (jas::bf16's common_type)
RANK = {I32: 0, BF16: 1, F32: 2, F64: 3}
OPS = {"leaf": 0, "const": 1, "+": 2, "-": 3, "*": 4, "/": 5, ">": 6, "<": 7, "exp": 8, "sigmoid": 9,
       "tanh": 10, "gelu": 11, "silu": 12, "sqrt": 13, "pow": 14, "neg": 15}


def promote(a, b):
    return a if RANK[a] >= RANK[b] else b


@dataclass
class Node:
    op: str
    dtype: int
    rows: int
    cols: int
    kids: list = field(default_factory=list)
    leaf: Optional[object] = None  # jas_leaf descriptor
    imm: float = 0.0
    owner: Optional[object] = None  # the device buffer a leaf points into, kept alive with the tree

    def __add__(self, o): return bin_("+", self, o)
    def __radd__(self, o): return bin_("+", o, self)
    def __sub__(self, o): return bin_("-", self, o)
    def __rsub__(self, o): return bin_("-", o, self)
    def __mul__(self, o): return bin_("*", self, o)
    def __rmul__(self, o): return bin_("*", o, self)
    def __truediv__(self, o): return bin_("/", self, o)
    def __rtruediv__(self, o): return bin_("/", o, self)
    def __gt__(self, o): return bin_(">", self, o)
    def __lt__(self, o): return bin_("<", self, o)


def const(v, dtype=None):
    if dtype is None:
        dtype = I32 if isinstance(v, int) else F64
    return Node("const", dtype, 1, 1, imm=float(v))


def leaf(arr, dtype=F32, **kw):
    from jasmine_amd.capi import leaf as mk
    lf = mk(arr, **kw)
    return Node("leaf", dtype, lf.vrows, lf.vcols, leaf=lf, owner=arr)


def _wrap(x):
    return x if isinstance(x, Node) else const(x)


def bin_(op, a, b):
    a, b = _wrap(a), _wrap(b)
    return Node(op, promote(a.dtype, b.dtype), max(a.rows, b.rows), max(a.cols, b.cols), [a, b])


def un(op, a, imm=0.0):
    return Node(op, a.dtype, a.rows, a.cols, [a], imm=imm)


def need(n):
    if not n.kids:
        return 1
    if len(n.kids) == 1:
        return need(n.kids[0])
    l, r = need(n.kids[0]), need(n.kids[1])
    return l + 1 if l == r else max(l, r)


def lower(root):
    """-> (list of (op, dtype, arg, imm), list of jas_leaf)"""
    ins, leaves = [], []

    def emit(n):
        if n.op == "leaf":
            leaves.append(n.leaf)
            ins.append((0, n.dtype, len(leaves) - 1, 0.0))
        elif n.op == "const":
            ins.append((1, n.dtype, 0, n.imm))
        elif len(n.kids) == 1:
            emit(n.kids[0])
            ins.append((OPS[n.op], n.dtype, 0, n.imm))
        else:
            a, b = n.kids
            swap = need(b) > need(a)
            if swap:
                emit(b); emit(a)
            else:
                emit(a); emit(b)
            ins.append((OPS[n.op], n.dtype, 1 if swap else 0, 0.0))

    emit(root)
    return ins, leaves


def evaluate(jas, root, out_dtype=None):
    """Materialise `root` with jas_ew_eval; returns a numpy array of the node's ele_type."""
    import ctypes as C

    import numpy as np
    from jasmine_amd.capi import Ins, Leaf, DeviceArray, check, lib

    prog, leaves = lower(root)
    dt = root.dtype if out_dtype is None else out_dtype
    npdt = {F32: np.float32, F64: np.float64, I32: np.int32, BF16: np.uint16}[dt]
    out = DeviceArray((root.rows, root.cols), npdt)
    pa = (Ins * len(prog))(*[Ins(o, d, a, 0, i) for o, d, a, i in prog])
    la = (Leaf * max(1, len(leaves)))(*leaves)
    check(lib.jas_ew_eval(pa, len(prog), la, len(leaves), out.p, dt, root.rows, root.cols, None))
    return out.numpy()
