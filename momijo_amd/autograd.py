"""The matmul node of momijo's autograd tape on the MI355X backend.

Mirrors ``Tape`` / ``GradContext`` / ``GradTensor`` of tensor/autograd.mojo
(:212-305) for the operations on this path: leaves, ``GradTensor.matmul``
(with another GradTensor or a plain Float32 tensor, :995-1017) and
``matmul2d`` (:930-939), and ``backward`` (:1352-) with its MATMUL2D rule
(:1542-1555).  Tape values and gradients are Float32, as the reference's
``List[tensor.Tensor[Float32]]`` (:214-216), and they stay in HBM: a forward
matmul runs on the fp32 MFMA engine and a backward step is one call of
``mj_matmul_backward_f32``, which adds ``g @ b^T`` and ``a^T @ g`` into the
parents' gradients in place (``grads[p] = grads[p].add(g)``), with no host
round trip.

The backward driver is the reference's: the root's gradient is seeded with
ones, then a stack is popped until empty; each MATMUL2D node adds to both
parents' gradients and pushes p0, then p1; leaves are skipped.  (A node
reachable along several paths is therefore processed once per path, as in
the reference.)  Other op tags are outside this path and raise.
"""
from __future__ import annotations

import torch

from . import _lib
from .tensor import Tensor, _ptr, _stream, matmul as _matmul

TAG_LEAF = 0        # tensor/autograd.mojo:95
TAG_MATMUL2D = 18   # tensor/autograd.mojo:131


class Tape:
    """Values, gradients, op tags and parents of the recorded nodes."""

    def __init__(self):
        self.values: list[Tensor] = []
        self.grads: list[Tensor] = []
        self.op_tags: list[int] = []
        self.parents: list[tuple[int, int]] = []

    def _push(self, val: Tensor, op: int, p0: int, p1: int) -> int:
        t = val.torch
        if t.dtype != torch.float32:
            raise TypeError("tape values are Float32 tensors")
        self.values.append(Tensor(t.clone()))
        self.grads.append(Tensor(torch.zeros_like(t)))
        self.op_tags.append(op)
        self.parents.append((p0, p1))
        return len(self.values) - 1

    def add_leaf(self, x: Tensor) -> int:
        return self._push(x, TAG_LEAF, -1, -1)

    def add_binary(self, val: Tensor, op: int, p0: int, p1: int) -> int:
        return self._push(val, op, p0, p1)


class GradContext:
    """GradContext (tensor/autograd.mojo:275-286): the tape and the no-grad depth."""

    def __init__(self):
        self.tape = Tape()
        self.no_grad_depth = 0

    def grad_enabled(self) -> bool:
        return self.no_grad_depth == 0


def no_grad_begin(ctx: GradContext) -> None:
    ctx.no_grad_depth += 1


def no_grad_end(ctx: GradContext) -> None:
    if ctx.no_grad_depth > 0:
        ctx.no_grad_depth -= 1


class GradTensor:
    """GradTensor (tensor/autograd.mojo:302-): an id into the context's tape."""

    __slots__ = ("id", "requires_grad")

    def __init__(self, id: int, requires_grad: bool):
        self.id = id
        self.requires_grad = requires_grad

    @staticmethod
    def from_tensor(ctx: GradContext, x: Tensor, requires_grad: bool = False) -> "GradTensor":
        nid = ctx.tape.add_leaf(x)
        return GradTensor(nid, requires_grad and ctx.grad_enabled())

    def value(self, ctx: GradContext) -> Tensor:
        return ctx.tape.values[self.id].copy()

    def shape(self, ctx: GradContext) -> list[int]:
        return ctx.tape.values[self.id].shape()

    def grad(self, ctx: GradContext) -> Tensor:
        return ctx.tape.grads[self.id].copy()

    def matmul2d(self, ctx: GradContext, other: "GradTensor") -> "GradTensor":
        """matmul2d (:930-939): y = a @ b for 2-D Float32 values."""
        y = _matmul(ctx.tape.values[self.id], ctx.tape.values[other.id])
        track = (self.requires_grad or other.requires_grad) and ctx.grad_enabled()
        if not track:
            return GradTensor(ctx.tape.add_leaf(y), False)
        return GradTensor(ctx.tape.add_binary(y, TAG_MATMUL2D, self.id, other.id), True)

    def matmul(self, ctx: GradContext, other) -> "GradTensor":
        """matmul (:995-1017).  With a GradTensor, a MATMUL2D node on both;
        with a plain Float32 tensor, that tensor is stored as a leaf so the
        backward can read it, and only self is tracked."""
        a = ctx.tape.values[self.id]
        if isinstance(other, GradTensor):
            y = _matmul(a, ctx.tape.values[other.id])
            track = (self.requires_grad or other.requires_grad) and ctx.grad_enabled()
            nid = (ctx.tape.add_binary(y, TAG_MATMUL2D, self.id, other.id) if track
                   else ctx.tape.add_leaf(y))
            return GradTensor(nid, track)
        y = _matmul(a, other)
        track = self.requires_grad and ctx.grad_enabled()
        if not track:
            return GradTensor(ctx.tape.add_leaf(y), False)
        bid = ctx.tape.add_leaf(other)
        return GradTensor(ctx.tape.add_binary(y, TAG_MATMUL2D, self.id, bid), True)

    def backward(self, ctx: GradContext) -> None:
        """backward (:1352-): seed ones, pop the stack until empty."""
        tape = ctx.tape
        tape.grads[self.id] = Tensor(torch.ones_like(tape.values[self.id].torch))
        stack = [self.id]
        while stack:
            top = stack.pop()
            op = tape.op_tags[top]
            if op == TAG_LEAF:
                continue
            if op != TAG_MATMUL2D:
                raise NotImplementedError(f"op tag {op} is outside the matmul path")
            p0, p1 = tape.parents[top]
            _matmul2d_rule(tape, top, p0, p1)
            if p0 >= 0:
                stack.append(p0)
            if p1 >= 0:
                stack.append(p1)


def _matmul2d_rule(tape: Tape, top: int, p0: int, p1: int) -> None:
    """grads[p0] += g @ b^T and grads[p1] += a^T @ g (:1542-1555), in place
    on the device, in that order (so p0 == p1 accumulates both)."""
    g = tape.grads[top].torch.contiguous()
    a = tape.values[p0].torch.contiguous()
    b = tape.values[p1].torch.contiguous()
    if a.dim() != 2 or b.dim() != 2 or g.dim() != 2:
        raise NotImplementedError("the MATMUL2D rule is defined for 2-D values")
    M, K = a.shape
    N = b.shape[1]
    ga = tape.grads[p0].torch if p0 >= 0 else None
    gb = tape.grads[p1].torch if p1 >= 0 else None
    for t in (ga, gb):
        if t is not None and not t.is_contiguous():
            raise ValueError("tape gradients are contiguous")
    _lib.call("mj_matmul_backward_f32", M, N, K, _ptr(a), _ptr(b), _ptr(g), _ptr(ga), None, 1,
              _stream())
    gb = tape.grads[p1].torch if p1 >= 0 else None   # after the dA update (p0 == p1)
    _lib.call("mj_matmul_backward_f32", M, N, K, _ptr(a), _ptr(b), _ptr(g), None, _ptr(gb), 1,
              _stream())


__all__ = ["Tape", "GradContext", "GradTensor", "no_grad_begin", "no_grad_end", "TAG_LEAF",
           "TAG_MATMUL2D"]
