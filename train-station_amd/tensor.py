"""Python face of train-station's Tensor / gradtrack / Adam API on the MI355X.

Every method is one call into ``libts_gradtrack.so`` (``include/ts_gradtrack.h``),
whose C++ host code launches the gfx950 kernels of ``libts_hip.so``.  Method
names and meaning follow the reference (tensor/core/utils.rs, tensor/ops/*,
tensor/reductions/{sum,mean}.rs, gradtrack/, optimizers/adam/mod.rs); its
panics surface as ``TsError``.
"""
from __future__ import annotations

import contextlib
import ctypes
from typing import Iterable, Optional, Sequence

import numpy as np

from ._ffi import F, SZ, TsError, gradtrack as _G, last_error


def _dims(shape: Sequence[int]):
    shape = [int(d) for d in shape]
    arr = (SZ * max(len(shape), 1))(*shape)
    return arr, len(shape)


def _wrap(handle) -> "Tensor":
    if not handle:
        raise TsError(last_error() or "native call returned no tensor")
    return Tensor(handle)


def _ok(status: int) -> None:
    if status != 0:
        raise TsError(last_error())


def _take_bytes(call) -> bytes:
    """Run a native call that returns a malloc'd buffer through (data, len)."""
    data, n = ctypes.c_void_p(), ctypes.c_size_t()
    _ok(call(ctypes.byref(data), ctypes.byref(n)))
    try:
        return ctypes.string_at(data, n.value)
    finally:
        _G.ts_buffer_free(data)


def _path(path) -> bytes:
    return str(path).encode()


class Tensor:
    """Handle on a device tensor owned by the native host library."""

    __slots__ = ("_h",)

    def __init__(self, handle):
        self._h = ctypes.c_void_p(handle)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _G.ts_tensor_free(h)
            self._h = None

    # -- construction (utils.rs:120-171, init/basic.rs, init/data.rs) -----------
    @staticmethod
    def new(shape: Sequence[int]) -> "Tensor":
        d, r = _dims(shape)
        return _wrap(_G.ts_tensor_new(d, r))

    @staticmethod
    def zeros(shape: Sequence[int]) -> "Tensor":
        d, r = _dims(shape)
        return _wrap(_G.ts_tensor_zeros(d, r))

    @staticmethod
    def ones(shape: Sequence[int]) -> "Tensor":
        d, r = _dims(shape)
        return _wrap(_G.ts_tensor_ones(d, r))

    @staticmethod
    def from_slice(data, shape: Sequence[int]) -> "Tensor":
        a = np.ascontiguousarray(np.asarray(data, dtype=np.float32).reshape(-1))
        d, r = _dims(shape)
        return _wrap(_G.ts_tensor_from_slice(a.ctypes.data_as(F), a.size, d, r))

    @staticmethod
    def randn(shape: Sequence[int], seed: Optional[int] = None) -> "Tensor":
        """Tensor::randn (init/random.rs:231-235), generated on the device."""
        d, r = _dims(shape)
        return _wrap(_G.ts_tensor_randn(d, r, 0 if seed is None else int(seed), seed is not None))

    def fill_randn(self, seed: Optional[int] = None) -> None:
        """fill_randn (random.rs:270-299), in place."""
        _ok(_G.ts_tensor_fill_randn(self._h, 0 if seed is None else int(seed), seed is not None))

    def clone(self) -> "Tensor":
        return _wrap(_G.ts_tensor_clone(self._h))

    # -- metadata -----------------------------------------------------------------
    def id(self) -> int:
        return int(_G.ts_tensor_id(self._h))

    @property
    def shape(self) -> tuple:
        rank = _G.ts_tensor_rank(self._h)
        out = (SZ * max(rank, 1))()
        _G.ts_tensor_dims(self._h, out, rank)
        return tuple(int(out[i]) for i in range(rank))

    def size(self) -> int:
        return int(_G.ts_tensor_size(self._h))

    def device_ptr(self) -> int:
        return int(_G.ts_tensor_device_ptr(self._h) or 0)

    # -- autograd flags (utils.rs:412-450) ------------------------------------------
    def with_requires_grad(self) -> "Tensor":
        _ok(_G.ts_tensor_with_requires_grad(self._h))
        return self

    def set_requires_grad(self, flag: bool) -> None:
        _ok(_G.ts_tensor_set_requires_grad(self._h, int(bool(flag))))

    def requires_grad(self) -> bool:
        return bool(_G.ts_tensor_requires_grad(self._h))

    # -- recorded ops -------------------------------------------------------------------
    def add_tensor(self, other: "Tensor") -> "Tensor":
        return _wrap(_G.ts_tensor_add_tensor(self._h, other._h))

    def sub_tensor(self, other: "Tensor") -> "Tensor":
        return _wrap(_G.ts_tensor_sub_tensor(self._h, other._h))

    def mul_tensor(self, other: "Tensor") -> "Tensor":
        return _wrap(_G.ts_tensor_mul_tensor(self._h, other._h))

    def div_tensor(self, other: "Tensor") -> "Tensor":
        return _wrap(_G.ts_tensor_div_tensor(self._h, other._h))

    def add_scalar(self, s: float) -> "Tensor":
        return _wrap(_G.ts_tensor_add_scalar(self._h, s))

    def sub_scalar(self, s: float) -> "Tensor":
        return _wrap(_G.ts_tensor_sub_scalar(self._h, s))

    def mul_scalar(self, s: float) -> "Tensor":
        return _wrap(_G.ts_tensor_mul_scalar(self._h, s))

    def div_scalar(self, s: float) -> "Tensor":
        return _wrap(_G.ts_tensor_div_scalar(self._h, s))

    def relu(self) -> "Tensor":
        return _wrap(_G.ts_tensor_relu(self._h))

    def pow_scalar(self, e: float) -> "Tensor":
        return _wrap(_G.ts_tensor_pow_scalar(self._h, e))

    def matmul(self, other: "Tensor") -> "Tensor":
        return _wrap(_G.ts_tensor_matmul(self._h, other._h))

    # -- tensor/ops/{exp,log,sqrt,tanh,sigmoid,leaky_relu,softmax}.rs -------------
    def exp(self) -> "Tensor":
        return _wrap(_G.ts_tensor_exp(self._h))

    def log(self) -> "Tensor":
        return _wrap(_G.ts_tensor_log(self._h))

    def sqrt(self) -> "Tensor":
        return _wrap(_G.ts_tensor_sqrt(self._h))

    def tanh(self) -> "Tensor":
        return _wrap(_G.ts_tensor_tanh(self._h))

    def sigmoid(self) -> "Tensor":
        return _wrap(_G.ts_tensor_sigmoid(self._h))

    def leaky_relu(self, negative_slope: float) -> "Tensor":
        return _wrap(_G.ts_tensor_leaky_relu(self._h, negative_slope))

    def softmax(self, dim: int) -> "Tensor":
        return _wrap(_G.ts_tensor_softmax(self._h, dim))

    def sum_dims(self, dims: Sequence[int], keepdim: bool = False) -> "Tensor":
        d, r = _dims(dims)
        return _wrap(_G.ts_tensor_sum_dims(self._h, d, r, int(bool(keepdim))))

    def mean_dims(self, dims: Sequence[int], keepdim: bool = False) -> "Tensor":
        d, r = _dims(dims)
        return _wrap(_G.ts_tensor_mean_dims(self._h, d, r, int(bool(keepdim))))

    # -- transform/{transpose,contiguous}.rs ----------------------------------------
    def transpose(self, dim0: int, dim1: int) -> "Tensor":
        return _wrap(_G.ts_tensor_transpose(self._h, dim0, dim1))

    def t(self) -> "Tensor":
        return _wrap(_G.ts_tensor_t(self._h))

    def contiguous(self) -> "Tensor":
        return _wrap(_G.ts_tensor_contiguous(self._h))

    def is_contiguous(self) -> bool:
        return bool(_G.ts_tensor_is_contiguous(self._h))

    def fill(self, value: float) -> None:
        """Tensor::fill (init/basic.rs:304-326), in place."""
        _ok(_G.ts_tensor_fill(self._h, value))

    def sum(self) -> "Tensor":
        return _wrap(_G.ts_tensor_sum(self._h))

    def mean(self) -> "Tensor":
        return _wrap(_G.ts_tensor_mean(self._h))

    # -- gradients (utils.rs:525-790) --------------------------------------------------
    def backward(self, grad_output: Optional["Tensor"] = None) -> None:
        _ok(_G.ts_tensor_backward(self._h, grad_output._h if grad_output is not None else None))

    def grad(self) -> Optional["Tensor"]:
        """Tensor::grad (utils.rs:491-506): the gradient stored on the tensor
        itself, sharing its buffer; None when there is none, also when only
        the graph's gradient map holds one (use grad_by_value for that)."""
        h = _G.ts_tensor_grad(self._h)
        if not h:
            err = last_error()
            if err:
                raise TsError(err)
            return None
        return Tensor(h)

    def grad_by_value(self) -> Optional["Tensor"]:
        h = _G.ts_tensor_grad_by_value(self._h)
        if not h:
            err = last_error()
            if err:
                raise TsError(err)
            return None
        return Tensor(h)

    def set_grad(self, grad: "Tensor") -> None:
        _ok(_G.ts_tensor_set_grad(self._h, grad._h))

    def zero_grad(self) -> None:
        _ok(_G.ts_tensor_zero_grad(self._h))

    # -- host access ------------------------------------------------------------------------
    def data(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=np.float32)
        _ok(_G.ts_tensor_data(self._h, out.ctypes.data_as(F), out.size))
        return out

    def value(self) -> float:
        v = ctypes.c_float()
        _ok(_G.ts_tensor_value(self._h, ctypes.byref(v)))
        return float(v.value)

    def __repr__(self) -> str:
        return f"Tensor(id={self.id()}, shape={list(self.shape)}, requires_grad={self.requires_grad()})"

    # -- checkpoint (tensor/core/serialization.rs, serialization/core/traits.rs) ----
    def to_binary(self) -> bytes:
        return _take_bytes(lambda d, n: _G.ts_tensor_to_binary(self._h, d, n))

    @staticmethod
    def from_binary(data: bytes) -> "Tensor":
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        return _wrap(_G.ts_tensor_from_binary(buf, len(data)))

    def to_json(self) -> str:
        return _take_bytes(lambda d, n: _G.ts_tensor_to_json(self._h, d, n)).decode()

    @staticmethod
    def from_json(text: str) -> "Tensor":
        b = text.encode()
        return _wrap(_G.ts_tensor_from_json(b, len(b)))

    def save_binary(self, path) -> None:
        _ok(_G.ts_tensor_save_binary(self._h, _path(path)))

    def save_json(self, path) -> None:
        _ok(_G.ts_tensor_save_json(self._h, _path(path)))

    @staticmethod
    def load_binary(path) -> "Tensor":
        return _wrap(_G.ts_tensor_load_binary(_path(path)))

    @staticmethod
    def load_json(path) -> "Tensor":
        return _wrap(_G.ts_tensor_load_json(_path(path)))


def _handles(params: Iterable[Tensor]):
    ps = list(params)
    arr = (ctypes.c_void_p * max(len(ps), 1))(*[p._h.value for p in ps])
    return arr, len(ps)


class Adam:
    """optimizers/adam/mod.rs (AdamConfig defaults: lr 1e-3, betas 0.9/0.999,
    eps 1e-8, weight_decay 0, amsgrad off)."""

    __slots__ = ("_h",)

    def __init__(self, _handle=None):
        h = _handle if _handle is not None else _G.ts_adam_new()
        if not h:
            raise TsError(last_error())
        self._h = ctypes.c_void_p(h)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            _G.ts_adam_free(h)
            self._h = None

    @staticmethod
    def new() -> "Adam":
        return Adam()

    @staticmethod
    def with_config(learning_rate=1e-3, beta1=0.9, beta2=0.999, eps=1e-8, weight_decay=0.0,
                    amsgrad=False) -> "Adam":
        return Adam(_G.ts_adam_with_config(learning_rate, beta1, beta2, eps, weight_decay,
                                           int(bool(amsgrad))))

    @staticmethod
    def with_learning_rate(lr: float) -> "Adam":
        return Adam(_G.ts_adam_with_learning_rate(lr))

    def add_parameter(self, p: Tensor) -> None:
        _ok(_G.ts_adam_add_parameter(self._h, p._h))

    def add_parameters(self, ps: Iterable[Tensor]) -> None:
        for p in ps:
            self.add_parameter(p)

    def step(self, params: Iterable[Tensor]) -> None:
        arr, n = _handles(params)
        _ok(_G.ts_adam_step(self._h, arr, n))

    def zero_grad(self, params: Iterable[Tensor]) -> None:
        arr, n = _handles(params)
        _ok(_G.ts_adam_zero_grad(self._h, arr, n))

    def learning_rate(self) -> float:
        return float(_G.ts_adam_learning_rate(self._h))

    def set_learning_rate(self, lr: float) -> None:
        _G.ts_adam_set_learning_rate(self._h, lr)

    def step_count(self) -> int:
        return int(_G.ts_adam_step_count(self._h))

    def state(self, p: Tensor, which: str) -> np.ndarray:
        out = np.empty(p.size(), dtype=np.float32)
        _ok(_G.ts_adam_state(self._h, p._h, {"m": 0, "v": 1}[which], out.ctypes.data_as(F), out.size))
        return out

    def config(self) -> dict:
        v = (ctypes.c_float * 5)()
        a = ctypes.c_int()
        _ok(_G.ts_adam_config(self._h, v, ctypes.byref(a)))
        return dict(learning_rate=v[0], beta1=v[1], beta2=v[2], eps=v[3], weight_decay=v[4],
                    amsgrad=bool(a.value))

    def parameter_step(self, p: Tensor) -> int:
        return int(_G.ts_adam_parameter_step(self._h, p._h))

    # -- checkpoint (optimizers/adam/serialization.rs) --------------------------------
    def to_binary(self) -> bytes:
        return _take_bytes(lambda d, n: _G.ts_adam_to_binary(self._h, d, n))

    @staticmethod
    def from_binary(data: bytes) -> "Adam":
        buf = ctypes.create_string_buffer(bytes(data), len(data))
        h = _G.ts_adam_from_binary(buf, len(data))
        if not h:
            raise TsError(last_error())
        return Adam(h)

    def to_json(self) -> str:
        return _take_bytes(lambda d, n: _G.ts_adam_to_json(self._h, d, n)).decode()

    @staticmethod
    def from_json(text: str) -> "Adam":
        b = text.encode()
        h = _G.ts_adam_from_json(b, len(b))
        if not h:
            raise TsError(last_error())
        return Adam(h)

    def save_binary(self, path) -> None:
        _ok(_G.ts_adam_save_binary(self._h, _path(path)))

    def save_json(self, path) -> None:
        _ok(_G.ts_adam_save_json(self._h, _path(path)))

    @staticmethod
    def load_binary(path) -> "Adam":
        h = _G.ts_adam_load_binary(_path(path))
        if not h:
            raise TsError(last_error())
        return Adam(h)

    @staticmethod
    def load_json(path) -> "Adam":
        h = _G.ts_adam_load_json(_path(path))
        if not h:
            raise TsError(last_error())
        return Adam(h)

    def relink_parameters(self, params: Iterable[Tensor]) -> None:
        """adam/mod.rs:396-454: map saved states onto live parameters by position."""
        arr, n = _handles(params)
        _ok(_G.ts_adam_relink_parameters(self._h, arr, n))

    def saved_parameter_count(self) -> int:
        return int(_G.ts_adam_saved_parameter_count(self._h))


def adam_config_to_binary(config: dict) -> bytes:
    """AdamConfig::to_binary (adam/serialization.rs:40-62)."""
    v = (ctypes.c_float * 5)(*[config[k] for k in _CONFIG_KEYS])
    return _take_bytes(lambda d, n: _G.ts_adam_config_to_binary(v, int(bool(config["amsgrad"])), d, n))


def adam_config_to_json(config: dict) -> str:
    v = (ctypes.c_float * 5)(*[config[k] for k in _CONFIG_KEYS])
    return _take_bytes(lambda d, n: _G.ts_adam_config_to_json(v, int(bool(config["amsgrad"])), d, n)).decode()


def adam_config_from_binary(data: bytes) -> dict:
    v, a = (ctypes.c_float * 5)(), ctypes.c_int()
    buf = ctypes.create_string_buffer(bytes(data), len(data))
    _ok(_G.ts_adam_config_from_binary(buf, len(data), v, ctypes.byref(a)))
    return dict(zip(_CONFIG_KEYS, list(v)), amsgrad=bool(a.value))


def adam_config_from_json(text: str) -> dict:
    v, a = (ctypes.c_float * 5)(), ctypes.c_int()
    b = text.encode()
    _ok(_G.ts_adam_config_from_json(b, len(b), v, ctypes.byref(a)))
    return dict(zip(_CONFIG_KEYS, list(v)), amsgrad=bool(a.value))


_CONFIG_KEYS = ("learning_rate", "beta1", "beta2", "eps", "weight_decay")


class NoGradTrack:
    """gradtrack/no_grad_track.rs:80-130 as a context manager."""

    def __enter__(self):
        _G.ts_no_grad_push()
        return self

    def __exit__(self, *exc):
        _G.ts_no_grad_pop()
        return False


def is_grad_enabled() -> bool:
    return bool(_G.ts_is_grad_enabled())


def set_grad_enabled(enabled: bool) -> None:
    """no_grad_track.rs:188-199: replaces the innermost gradient state."""
    _G.ts_set_grad_enabled(int(bool(enabled)))


def with_no_grad(f):
    """no_grad_track.rs:229-235: runs f() with gradient tracking disabled."""
    with NoGradTrack():
        return f()


def clear_gradients() -> None:
    _G.ts_clear_gradients()


def set_fusion(on: bool) -> None:
    """Fuse a 2-D matmul with a following row-bias add and relu (and, in
    backward, the dX product with relu's gradient) into one kernel; results
    are bit-identical either way.  On by default."""
    _G.ts_fusion_enable(1 if on else 0)


def fusion_enabled() -> bool:
    return bool(_G.ts_fusion_enabled())


class StepGraph:
    """One recorded training step (include/ts_gradtrack.h, ts_step_graph_*):
    the work issued inside ``with StepGraph.record() as g:`` is recorded as a
    HIP graph, not run (and not counted); ``g.replay(n)`` runs it n times,
    each replay's Adam steps taking the step counts that follow the
    optimizer's count at that moment, as eager steps would.  The recording
    starts with no gradients held and should end with ``zero_grad``.  Inside
    the recording nothing may read the device or upload host data; results are
    read after a replay."""

    def __init__(self) -> None:
        self._h = None

    @staticmethod
    @contextlib.contextmanager
    def record():
        g = StepGraph()
        _ok(_G.ts_step_graph_begin())
        try:
            yield g
        except BaseException:
            _G.ts_step_graph_abort()
            raise
        h = _G.ts_step_graph_end()
        if not h:
            raise TsError(last_error() or "recording the step failed")
        g._h = h

    def replay(self, times: int = 1) -> None:
        if not self._h:
            raise TsError("the step graph holds no recording")
        _ok(_G.ts_step_graph_replay(self._h, int(times)))

    def free(self) -> None:
        if self._h:
            _G.ts_step_graph_free(self._h)
            self._h = None

    def __del__(self) -> None:
        try:
            self.free()
        except Exception:
            pass


def recording() -> bool:
    return bool(_G.ts_step_graph_recording())


def synchronize() -> None:
    _ok(_G.ts_synchronize())


def stream() -> int:
    return int(_G.ts_stream() or 0)


class Profile:
    """Device-event timing of every kernel the host library launches, by class."""

    GEMM, ELEMENTWISE, REDUCTION, ADAM = 0, 1, 2, 3

    @staticmethod
    def enable(on: bool = True, classes: Optional[Sequence[int]] = None) -> None:
        """Time launches of `classes` (default: all); the others record no events."""
        mask = 0xFFFFFFFF if classes is None else sum(1 << int(k) for k in classes)
        _G.ts_profile_classes(mask)
        _G.ts_profile_enable(int(bool(on)))

    @staticmethod
    def reset() -> None:
        _G.ts_profile_reset()

    @staticmethod
    def read(kernel_class: int):
        ms, work, n = ctypes.c_double(), ctypes.c_double(), ctypes.c_uint64()
        _ok(_G.ts_profile_read(kernel_class, ctypes.byref(ms), ctypes.byref(work), ctypes.byref(n)))
        return {"ms": ms.value, "work": work.value, "launches": int(n.value)}


def pool_stats() -> dict:
    return {"live_bytes": int(_G.ts_pool_live_bytes()), "cached_bytes": int(_G.ts_pool_cached_bytes())}


def empty_cache() -> None:
    _G.ts_pool_empty_cache()
