"""Restatement of train-station's gradtrack engine and Adam on the CPU oracle.

TEST INFRASTRUCTURE ONLY (see ``oracle/__init__.py``).

The control flow follows the reference so that gradient accumulation happens
in the same order:

* ``OTensor`` ids come from one global counter (tensor/core/mod.rs:131); the
  recorded graph is ``operations: id -> (input_ids, grad_fn)`` and
  ``gradients: id -> array`` (gradtrack/engine.rs:175-187, 265-267, 359-361).
* Tensor ops record a node only when an operand requires grad and gradtrack
  is enabled; elementwise ops list only the operands that require grad in
  ``input_ids`` while the backward returns gradients by operand position
  (ops/add.rs:127-143, ops/sub.rs:149-156); matmul always lists both operands
  (ops/matmul/mod.rs:291-307); sum/mean record whenever the input requires
  grad, ignoring the no-grad switch (reductions/sum.rs:131-138).
* ``backward`` seeds ``ones`` (or the given gradient), then runs the LIFO
  worklist of engine.rs:962-1047: pop, take the node's gradient, apply its
  GradFn, accumulate ``existing + new`` into each input
  (engine.rs:514-524) and push inputs that have an operation.
* Leaf gradients stay in the map; ``grad_by_value`` returns ``self.grad`` if
  set, else the map entry (core/utils.rs:525-534).
* ``OAdam`` follows optimizers/adam/mod.rs:485-553 and :1036-1068.

Matmul uses the f64-accumulated GEMM rounded to fp32 (the reference's blocked
fp32 kernel is wrong at the configuration shapes, kernels.rs:1092-1133).
"""
from __future__ import annotations

import itertools
import warnings
from dataclasses import dataclass, field
from typing import Optional

import numpy as np

import oracle as O

_ids = itertools.count(1)

# exp / ln / tanh in the recorded ops: False = the host libm (what the
# reference computes; the device restates glibc 2.35's evaluations, with
# the same bits), True = f64 rounded once (correctly rounded)
CORRECTLY_ROUNDED = False

# thread-local GradGraph of the reference (engine.rs:697-699); one per process here
_operations: dict[int, tuple[list[int], "GradFn"]] = {}
_gradients: dict[int, np.ndarray] = {}
_grad_enabled: list[bool] = [True]


def clear_gradients() -> None:
    """engine.rs:812-816: drops every recorded operation and gradient."""
    _operations.clear()
    _gradients.clear()


def is_grad_enabled() -> bool:
    return _grad_enabled[-1]


class NoGradTrack:
    """Context manager form of gradtrack/no_grad_track.rs:80-130."""

    def __enter__(self):
        _grad_enabled.append(False)

    def __exit__(self, *exc):
        _grad_enabled.pop()


@dataclass
class GradFn:
    kind: str
    saved: list = field(default_factory=list)      # saved arrays (reference clones)
    shapes: Optional[tuple] = None                  # original_shapes for broadcasting
    scalar: Optional[float] = None
    requires: tuple = (True, True)                  # MatMul requires_grad pair
    numel: int = 0
    dims: tuple = ()                                # sum_dims / mean_dims axes (sorted, unique)
    keepdim: bool = False
    axis: int = 0                                   # softmax


class OTensor:
    def __init__(self, data: np.ndarray, requires_grad: bool = False):
        a = np.asarray(data, dtype=np.float32)  # keeps rank 0 (ascontiguousarray would not)
        self.data = a if a.flags.c_contiguous else a.copy(order="C")
        self.id = next(_ids)
        self.requires_grad = requires_grad
        self.grad: Optional[np.ndarray] = None

    # -- construction ------------------------------------------------------
    @staticmethod
    def from_slice(values, dims) -> "OTensor":
        arr = np.asarray(values, dtype=np.float32).reshape(dims)
        return OTensor(arr.copy())

    def with_requires_grad(self) -> "OTensor":
        self.requires_grad = True
        return self

    @property
    def shape(self):
        return self.data.shape

    def size(self) -> int:
        return self.data.size

    # -- helpers -----------------------------------------------------------
    def _record(self, out: "OTensor", input_ids: list[int], fn: GradFn) -> "OTensor":
        out.requires_grad = True
        _operations[out.id] = (input_ids, fn)
        return out

    def _elementwise(self, other: "OTensor", kind: str, same, bias_fn) -> "OTensor":
        if self.shape == other.shape:
            out = OTensor(same(self.data, other.data))
            shapes = None
        else:
            out = OTensor(bias_fn(self.data, other.data))
            shapes = (self.shape, other.shape)
        if (self.requires_grad or other.requires_grad) and is_grad_enabled():
            ids = [t.id for t in (self, other) if t.requires_grad]
            saved = [self.data, other.data] if kind in ("mul", "div") else []
            self._record(out, ids, GradFn(kind, saved=saved, shapes=shapes))
        return out

    # -- recorded ops (forward) --------------------------------------------
    def add_tensor(self, other):
        return self._elementwise(other, "add", O.add, _broadcast(O.add))

    def sub_tensor(self, other):
        return self._elementwise(other, "sub", O.sub, _broadcast(O.sub))

    def mul_tensor(self, other):
        return self._elementwise(other, "mul", O.mul, _broadcast(O.mul))

    def div_tensor(self, other):
        return self._elementwise(other, "div", O.div, _broadcast(O.div))

    def _scalar_op(self, kind, fn, s):
        out = OTensor(fn(self.data, s))
        if self.requires_grad and is_grad_enabled():
            self._record(out, [self.id], GradFn(kind + "_scalar", scalar=s))
        return out

    def add_scalar(self, s):
        return self._scalar_op("add", O.add_scalar, s)

    def sub_scalar(self, s):
        return self._scalar_op("sub", O.sub_scalar, s)

    def mul_scalar(self, s):
        return self._scalar_op("mul", O.mul_scalar, s)

    def div_scalar(self, s):
        return self._scalar_op("div", O.div_scalar, s)

    def relu(self, mask_source: Optional[np.ndarray] = None):
        """ops/relu.rs:77-90.  ``mask_source`` (test hook) replaces the saved
        input whose sign decides the backward mask, so a comparison with
        another implementation can condition on that implementation's masks
        where a pre-activation lies within rounding of zero."""
        out = OTensor(O.relu(self.data))
        if self.requires_grad and is_grad_enabled():
            saved = self.data if mask_source is None else np.ascontiguousarray(mask_source, np.float32)
            assert saved.shape == self.data.shape
            self._record(out, [self.id], GradFn("relu", saved=[saved]))
        return out

    def pow_scalar(self, e: float):
        if np.float32(e) != 2.0:
            raise NotImplementedError("the oracle restates exponent 2.0 only (ops/pow.rs:124-162)")
        out = OTensor(O.pow2(self.data))
        if self.requires_grad and is_grad_enabled():
            self._record(out, [self.id], GradFn("pow", saved=[self.data], scalar=float(e)))
        return out

    def matmul(self, other):
        """ops/matmul/mod.rs:263-310: 1D.1D dot (shape []), 1D.2D, 2D.1D, 2D.2D,
        else batched with broadcast batch axes (both operands at least 2D)."""
        out = OTensor(_matmul_f64(self.data, other.data))
        if (self.requires_grad or other.requires_grad) and is_grad_enabled():
            self._record(out, [self.id, other.id],
                         GradFn("matmul", saved=[self.data, other.data],
                                requires=(self.requires_grad, other.requires_grad)))
        return out

    def sum(self):
        out = OTensor(np.array([O.sum_(self.data)], dtype=np.float32))
        if self.requires_grad:
            self._record(out, [self.id], GradFn("sum", shapes=(self.shape,)))
        return out

    def mean(self):
        out = OTensor(np.array([O.mean(self.data)], dtype=np.float32))
        if self.requires_grad:
            self._record(out, [self.id], GradFn("mean", shapes=(self.shape,), numel=self.size()))
        return out

    # -- autograd ------------------------------------------------------------
    # -- tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,softmax}.rs -----------
    def _unary(self, kind: str, slope: float = 0.0) -> "OTensor":
        out = OTensor(O.unary(kind, self.data, slope, CORRECTLY_ROUNDED))
        if self.requires_grad and is_grad_enabled():
            keep_input = kind in ("log", "leaky_relu")
            self._record(out, [self.id], GradFn(kind, saved=[self.data if keep_input else out.data],
                                                scalar=slope))
        return out

    def exp(self):
        return self._unary("exp")

    def log(self):
        return self._unary("log")

    def sqrt(self):
        return self._unary("sqrt")

    def tanh(self):
        return self._unary("tanh")

    def sigmoid(self):
        return self._unary("sigmoid")

    def leaky_relu(self, negative_slope: float):
        return self._unary("leaky_relu", negative_slope)

    def softmax(self, dim: int):
        assert dim < self.data.ndim, f"softmax dim {dim} out of bounds for rank {self.data.ndim}"
        out = OTensor(O.softmax(self.data, dim, CORRECTLY_ROUNDED))
        if self.requires_grad and is_grad_enabled():
            self._record(out, [self.id], GradFn("softmax", saved=[out.data], axis=dim))
        return out

    def sum_dims(self, dims, keepdim: bool = False):
        """reductions/sum.rs:225-306 (records whenever the input requires grad)"""
        out = OTensor(O.sum_dims(self.data, dims, keepdim))
        if self.requires_grad:
            self._record(out, [self.id], GradFn("sum_dims", shapes=(self.shape,), dims=tuple(sorted(set(dims))),
                                                keepdim=keepdim))
        return out

    def mean_dims(self, dims, keepdim: bool = False):
        """reductions/mean.rs:186-230: sum times 1/factor, factor over the axes as listed"""
        factor = int(np.prod([self.shape[d] for d in dims], dtype=np.int64))
        scale = np.float32(1.0) / np.float32(factor) if factor > 0 else np.float32(0.0)
        out = OTensor(O.mul_scalar(O.sum_dims(self.data, dims, keepdim), float(scale)))
        if self.requires_grad:
            self._record(out, [self.id], GradFn("mean_dims", shapes=(self.shape,),
                                                dims=tuple(sorted(set(dims))), keepdim=keepdim))
        return out

    def transpose(self, dim0: int, dim1: int):
        """transform/transpose.rs:156-208: axes dim0 and dim1 swapped (the
        reference's strided view, here a copy: the values are the same); the
        same axis twice is a clone that tracks no gradient (:171-173); records
        whenever the input requires grad."""
        rank = self.data.ndim
        if dim0 >= rank:
            raise ValueError(f"dim0 {dim0} out of bounds for tensor with rank {rank}")
        if dim1 >= rank:
            raise ValueError(f"dim1 {dim1} out of bounds for tensor with rank {rank}")
        if dim0 == dim1:
            return OTensor(self.data.copy())
        out = OTensor(np.ascontiguousarray(np.swapaxes(self.data, dim0, dim1)))
        if self.requires_grad:
            self._record(out, [self.id], GradFn("transpose", shapes=(self.shape,), dims=(dim0, dim1)))
        return out

    def t(self):
        """transpose.rs:283-291: the last two axes."""
        if self.data.ndim < 2:
            raise ValueError(f"Matrix transpose requires at least 2 dimensions, got {self.data.ndim}")
        return self.transpose(self.data.ndim - 2, self.data.ndim - 1)

    def contiguous(self):
        """transform/contiguous.rs:123-157: a copy; records (identity
        gradient) whenever the input requires grad."""
        out = OTensor(self.data.copy())
        if self.requires_grad:
            self._record(out, [self.id], GradFn("contiguous", shapes=(self.shape,)))
        return out

    def fill(self, value: float) -> None:
        """init/basic.rs:304-326: every element set to value, in place."""
        self.data[...] = np.float32(value)

    def backward(self, grad_output: Optional[np.ndarray] = None) -> None:
        backward(self, grad_output)

    def grad_by_value(self) -> Optional[np.ndarray]:
        if self.grad is not None:
            return self.grad.copy()
        g = _gradients.get(self.id)
        return None if g is None else g.copy()

    def zero_grad(self) -> None:
        self.grad = None

    def value(self) -> float:
        assert self.size() == 1
        return float(self.data.reshape(-1)[0])


def _broadcast(fn):
    """Materialise both operands to the broadcast shape, then the same-shape
    op (ops/broadcasting.rs:299-478: NumPy's rules, axes aligned right)."""

    def apply(a, b):
        shape = np.broadcast_shapes(a.shape, b.shape)
        return fn(np.ascontiguousarray(np.broadcast_to(a, shape)), np.ascontiguousarray(np.broadcast_to(b, shape)))

    return apply


def _reduce_to(g: np.ndarray, shape) -> np.ndarray:
    """reduce_gradient_to_shape (grad_fn/utils.rs:23-60): sum_dims([0]) once
    per leading axis, then sum_dims([i], keepdim) over each axis broadcast
    from size 1, then a reshape -- with the reference's fp32 sums."""
    shape = tuple(shape)
    if g.shape == shape:
        return g
    r = g
    for _ in range(g.ndim - len(shape)):
        r = O.sum_dims(r, [0], False)
    for i, (cur, tgt) in enumerate(zip(list(r.shape), shape)):
        if tgt == 1 and cur > 1:
            r = O.sum_dims(r, [i], True)
    return np.ascontiguousarray(r.reshape(shape))


def _matmul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """The product in f64 rounded once to fp32, with the reference's shape rules
    and messages (numpy's matmul broadcasts batch axes the same way)."""
    if a.ndim == 1 and b.ndim == 1:
        if a.shape[0] != b.shape[0]:
            raise ValueError("Tensors must have same length for dot product")
        return np.array(np.dot(a.astype(np.float64), b.astype(np.float64)), np.float32).reshape(())
    if a.ndim == 1 and b.ndim == 2 and a.shape[0] != b.shape[0]:
        raise ValueError("Vector length must match matrix rows")
    if a.ndim == 2 and b.ndim == 1 and a.shape[1] != b.shape[0]:
        raise ValueError("Matrix columns must match vector length")
    if (a.ndim > 2 or b.ndim > 2) and (a.ndim < 2 or b.ndim < 2):
        raise ValueError("Batched matmul requires at least 2D tensors")
    if a.ndim == 2 and b.ndim == 2:
        return O.gemm_f64(a, b).astype(np.float32)
    return np.ascontiguousarray(np.matmul(a.astype(np.float64), b.astype(np.float64)).astype(np.float32))


def _expand(go: np.ndarray, input_shape, dims, keepdim: bool) -> np.ndarray:
    """apply_reduce_sum_dims (grad_fn/reductions/sum.rs:18-52): each input
    element takes the gradient at its kept coordinates."""
    kd = [1 if k in dims else v for k, v in enumerate(input_shape)]
    return np.ascontiguousarray(np.broadcast_to(go.reshape(kd), input_shape))


def _apply(fn: GradFn, go: np.ndarray) -> list[Optional[np.ndarray]]:
    """GradFn::apply (grad_fn/mod.rs:490-789) for the variants on the path."""
    k = fn.kind
    if k == "add":                                   # grad_fn/ops/add.rs:4-28
        if fn.shapes is None:
            return [go, go]
        return [_reduce_to(go, fn.shapes[0]), _reduce_to(go, fn.shapes[1])]
    if k == "sub":                                   # grad_fn/ops/sub.rs:4-33
        if fn.shapes is None:
            return [go, O.neg(go)]
        return [_reduce_to(go, fn.shapes[0]), O.neg(_reduce_to(go, fn.shapes[1]))]
    if k == "mul":                                   # grad_fn/ops/mul.rs:4-49
        a, b = fn.saved
        if fn.shapes is None:
            return [O.mul(go, b), O.mul(go, a)]
        ab, bb = np.broadcast_arrays(a, b)
        return [_reduce_to(O.mul(go, np.ascontiguousarray(bb)), fn.shapes[0]),
                _reduce_to(O.mul(go, np.ascontiguousarray(ab)), fn.shapes[1])]
    if k == "div":                                   # grad_fn/ops/div.rs:4-49
        a, b = fn.saved
        if fn.shapes is not None:
            ab, bb = np.broadcast_arrays(a, b)
            a, b = np.ascontiguousarray(ab), np.ascontiguousarray(bb)
        ga = O.div(go, b)
        gb = O.neg(O.div(O.mul(go, a), O.mul(b, b)))
        if fn.shapes is None:
            return [ga, gb]
        return [_reduce_to(ga, fn.shapes[0]), _reduce_to(gb, fn.shapes[1])]
    if k == "transpose":                             # grad_fn/transforms/transpose.rs
        return [np.ascontiguousarray(np.swapaxes(go, fn.dims[0], fn.dims[1]))]
    if k == "contiguous":                            # grad_fn/mod.rs:534-537: identity
        return [go]
    if k in ("add_scalar", "sub_scalar"):
        return [go]
    if k == "mul_scalar":
        return [O.mul_scalar(go, fn.scalar)]
    if k == "div_scalar":
        return [O.div_scalar(go, fn.scalar)]
    if k == "relu":                                  # grad_fn/ops/relu.rs:4-17
        return [O.relu_bwd(fn.saved[0], go)]
    if k == "pow":                                   # grad_fn/ops/pow.rs:5-27
        return [O.pow_bwd(fn.saved[0], go, fn.scalar)]
    if k == "matmul":                                # grad_fn/ops/matmul.rs:4-219
        a, b = fn.saved
        if a.ndim == 2 and b.ndim == 2:
            gl = O.gemm_f64(go, b, tb=True).astype(np.float32) if fn.requires[0] else None
            gr = O.gemm_f64(a, go, ta=True).astype(np.float32) if fn.requires[1] else None
            return [gl, gr]
        if a.ndim == 1 and b.ndim == 1:              # go * b, go * a (go has shape [])
            g = np.broadcast_to(go.reshape(()), a.shape)
            return [O.mul(np.ascontiguousarray(g), b) if fn.requires[0] else None,
                    O.mul(np.ascontiguousarray(g), a) if fn.requires[1] else None]
        g64, a64, b64 = (v.astype(np.float64) for v in (go, a, b))
        if a.ndim == 1 and b.ndim == 2:              # go . M^T, outer(v, go)
            return [(b64 @ g64).astype(np.float32) if fn.requires[0] else None,
                    O.mul(*np.broadcast_arrays(a[:, None], go[None, :])) if fn.requires[1] else None]
        if a.ndim == 2 and b.ndim == 1:              # outer(go, v), M^T . go
            return [O.mul(*np.broadcast_arrays(go[:, None], b[None, :])) if fn.requires[0] else None,
                    (a64.T @ g64).astype(np.float32) if fn.requires[1] else None]
        # batched: go . B^T and A^T . go, then reduce_gradient_to_original_shape
        gl = _reduce_to(np.matmul(g64, np.swapaxes(b64, -1, -2)).astype(np.float32), a.shape) if fn.requires[0] else None
        gr = _reduce_to(np.matmul(np.swapaxes(a64, -1, -2), g64).astype(np.float32), b.shape) if fn.requires[1] else None
        return [gl, gr]
    if k == "sum":                                   # grad_fn/reductions/sum.rs:4-16
        shape = fn.shapes[0]
        if go.size == 1:
            return [O.fill(shape, float(go.reshape(-1)[0]))]
        return [O.fill(shape, 1.0)]
    if k == "mean":                                  # grad_fn/reductions/mean.rs:4-30
        shape = fn.shapes[0]
        base = np.float32(1.0) / np.float32(fn.numel) if fn.numel > 0 else np.float32(0.0)
        if go.size == 1:
            return [O.fill(shape, float(base * np.float32(go.reshape(-1)[0])))]
        return [O.fill(shape, float(base))]
    if k in ("exp", "log", "sqrt", "tanh", "sigmoid", "leaky_relu"):
        return [O.unary_bwd(k, fn.saved[0], go, fn.scalar or 0.0)]
    if k == "softmax":                               # grad_fn/ops/softmax.rs:4-38
        return [O.softmax_bwd(fn.saved[0], go, fn.axis)]
    if k == "sum_dims":                              # grad_fn/reductions/sum.rs:18-52
        return [_expand(go, fn.shapes[0], fn.dims, fn.keepdim)]
    if k == "mean_dims":                             # grad_fn/reductions/mean.rs:32-52
        factor = int(np.prod([fn.shapes[0][d] for d in fn.dims], dtype=np.int64))
        scale = np.float32(1.0) / np.float32(factor) if factor > 0 else np.float32(0.0)
        return [O.mul_scalar(_expand(go, fn.shapes[0], fn.dims, fn.keepdim), float(scale))]
    raise NotImplementedError(k)


# Test hook: when set, called as hook(input_id, scale, terms) for every
# gradient a 2-D matmul backward or a row-broadcast add backward produces,
# where scale[i] = sum of |terms| of the sum that produced element i (for
# a^T.go: (|a|^T.|go|)[i, j]; for go.b^T: (|go|.|b|^T)[i, j]; for a bias
# column sum: sum_r |go[r, j]|) and terms is that sum's length.  Any fp32
# evaluation of the sum, in any order, lies within terms * 2^-23 * scale of
# the exact value; a gradient smaller than that has no fp32-determined sign.
GRAD_SCALE_HOOK = None


def _report_scales(fn: GradFn, current: np.ndarray, input_ids, grads) -> None:
    if fn.kind == "matmul" and fn.saved[0].ndim == 2 and fn.saved[1].ndim == 2:
        # matmul records both operands (input_ids = [a, b]); f32 products of
        # the absolute values are ample for a bound
        a, b = (np.abs(v).astype(np.float32) for v in fn.saved)
        g = np.abs(current).astype(np.float32)
        if grads[0] is not None:
            GRAD_SCALE_HOOK(input_ids[0], (g @ b.T).astype(np.float64), b.shape[1])
        if grads[1] is not None:
            GRAD_SCALE_HOOK(input_ids[1], (a.T @ g).astype(np.float64), a.shape[0])
    elif fn.kind == "add" and fn.shapes is not None:  # gradients go to input_ids by position
        for idx, shape in enumerate(fn.shapes):
            if idx < len(input_ids) and len(shape) == 1 and current.ndim == 2 and shape[0] == current.shape[1]:
                GRAD_SCALE_HOOK(input_ids[idx], np.abs(current.astype(np.float64)).sum(axis=0), current.shape[0])


def backward(t: OTensor, grad_output: Optional[np.ndarray] = None) -> None:
    """GradEngine::backward (engine.rs:962-1047)."""
    init = O.fill(t.shape, 1.0) if grad_output is None else np.ascontiguousarray(grad_output, np.float32)
    if t.requires_grad:                                            # utils.rs:735 accumulate_grad
        t.grad = init if t.grad is None else O.add(t.grad, init)
    _gradients[t.id] = init
    work = [t.id]
    while work:
        node = work.pop()
        op = _operations.get(node)
        if op is None:
            continue
        current = _gradients.pop(node, None)
        if current is None:
            continue
        input_ids, fn = op
        grads = _apply(fn, current)
        if GRAD_SCALE_HOOK is not None:
            _report_scales(fn, current, input_ids, grads)
        for idx, iid in enumerate(input_ids):
            if idx < len(grads) and grads[idx] is not None:
                g = grads[idx]
                if iid in _gradients:                              # engine.rs:514-524
                    _gradients[iid] = O.add(_gradients[iid], g)
                else:
                    _gradients[iid] = g
                if iid in _operations:
                    work.append(iid)


@dataclass
class _AdamState:
    m: np.ndarray
    v: np.ndarray
    step: int = 0
    vmax: Optional[np.ndarray] = None


class OAdam:
    """optimizers/adam/mod.rs (AdamConfig of :90-117)."""

    def __init__(self, learning_rate=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
                 amsgrad=False):
        self.lr, self.b1, self.b2, self.eps = learning_rate, beta1, beta2, eps
        self.weight_decay, self.amsgrad = weight_decay, amsgrad
        self.states: dict[int, _AdamState] = {}
        self.step_count = 0

    def add_parameter(self, p: OTensor) -> None:
        assert p.requires_grad, "Parameter must require gradients"
        self.states[p.id] = _AdamState(np.zeros(p.size(), np.float32), np.zeros(p.size(), np.float32))

    def add_parameters(self, ps) -> None:
        for p in ps:
            self.add_parameter(p)

    def step(self, params) -> None:
        self.step_count += 1                                          # :1036-1044
        for p in params:
            assert p.id in self.states, "Parameter must be linked to optimizer before stepping"
            g = p.grad_by_value()
            if g is None:
                warnings.warn(f"Failed to update parameter: Parameter {p.id} has no gradient")
                continue
            st = self.states[p.id]
            st.step += 1
            first = False
            if self.amsgrad and st.vmax is None:
                st.vmax = np.zeros_like(st.m)
                first = True
            flat = p.data.reshape(-1)
            O.adam_step(flat, np.ascontiguousarray(g.reshape(-1)), st.m, st.v, self.step_count,
                        self.lr, self.b1, self.b2, self.eps, self.weight_decay,
                        st.vmax if self.amsgrad else None, first)

    def zero_grad(self, params) -> None:
        for p in params:
            p.zero_grad()
        clear_gradients()
