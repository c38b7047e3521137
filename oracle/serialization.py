"""CPU restatement of train-station's serialization format (test infrastructure).

TEST INFRASTRUCTURE ONLY: imported by ``tests/`` as the checker of the
product's checkpoint code; the product never imports it.

Restates, from the reference's sources (paths under train-station/src/):

* the FieldValue tree (serialization/core/types.rs) -- here ``FV(kind, value)``;
* the binary format "TS_B" v1: header (binary/header.rs:41-53, :76-106,
  :120-215), primitives (binary/writer.rs, binary/reader.rs incl. its size
  limits), values (binary/structs.rs:90-460);
* the JSON format: writer (json/structs.rs:32-184, json/escape.rs), reader
  (json/structs.rs:186-310 on top of a standard JSON parse);
* Tensor / Shape / Device fields (tensor/core/serialization.rs:128-248) and
  Adam / AdamConfig / parameter state fields (optimizers/adam/serialization.rs).

Object members come from Rust HashMaps, whose iteration order is random per
process; writers here take the member order from the caller (``shuffle``
reorders them the way the reference might).
"""
from __future__ import annotations

import json
import random
import struct
from dataclasses import dataclass
from typing import Any

import numpy as np

KINDS = ["Bool", "I8", "I16", "I32", "I64", "U8", "U16", "U32", "U64", "Usize", "F32", "F64",
         "String", "Bytes", "JsonObject", "BinaryObject", "Array", "Optional", "Object", "Enum"]
TAG = {k: i for i, k in enumerate(KINDS)}

MAGIC = 0x54535F42       # binary/types.rs:13
VERSION = 1              # binary/types.rs:20
OBJECT_TYPES = {0x1001: "Tensor", 0x1002: "Adam", 0x1003: "AdamConfig", 0x1004: "Shape",
                0x1005: "ParameterState"}


class FormatError(ValueError):
    pass


@dataclass
class FV:
    """FieldValue.  value: bool / int / float (F32 held as np.float32) / str /
    bytes / list[FV] (Array) / FV | None (Optional) / dict[str, FV] (Object) /
    (variant, FV | None) (Enum)."""
    kind: str
    value: Any


def usize(v: int) -> FV:
    return FV("Usize", int(v))


def f32(v) -> FV:
    return FV("F32", np.float32(v))


def array_f32(values) -> FV:
    return FV("Array", [FV("F32", np.float32(x)) for x in np.asarray(values, np.float32).reshape(-1)])


def array_usize(values) -> FV:
    return FV("Array", [usize(x) for x in values])


def enum_unit(variant: str) -> FV:
    return FV("Enum", (variant, None))


def obj(pairs, shuffle: random.Random | None = None) -> FV:
    items = list(pairs.items() if isinstance(pairs, dict) else pairs)
    if shuffle is not None:
        shuffle.shuffle(items)
    return FV("Object", dict(items))


# ---- binary ---------------------------------------------------------------------------

def _w_string(out: bytearray, s: str) -> None:  # writer.rs write_string: u32 length + UTF-8
    b = s.encode()
    out += struct.pack("<I", len(b)) + b


def write_value(out: bytearray, v: FV) -> None:
    """binary/structs.rs:147-290"""
    out.append(TAG[v.kind])
    k, x = v.kind, v.value
    if k == "Bool":
        out.append(1 if x else 0)
    elif k in ("I8", "U8"):
        out += struct.pack("<b" if k == "I8" else "<B", x)
    elif k in ("I16", "U16"):
        out += struct.pack("<h" if k == "I16" else "<H", x)
    elif k in ("I32", "U32"):
        out += struct.pack("<i" if k == "I32" else "<I", x)
    elif k in ("I64", "U64", "Usize"):
        out += struct.pack("<q" if k == "I64" else "<Q", x)
    elif k == "F32":
        out += np.float32(x).tobytes()
    elif k == "F64":
        out += struct.pack("<d", x)
    elif k in ("String", "JsonObject"):
        _w_string(out, x)
    elif k in ("Bytes", "BinaryObject"):
        out += struct.pack("<Q", len(x)) + bytes(x)
    elif k == "Array":
        out += struct.pack("<Q", len(x))
        for e in x:
            write_value(out, e)
    elif k == "Optional":
        out.append(0 if x is None else 1)
        if x is not None:
            write_value(out, x)
    elif k == "Object":
        out += struct.pack("<Q", len(x))
        for key, e in x.items():
            _w_string(out, key)
            write_value(out, e)
    elif k == "Enum":
        variant, data = x
        _w_string(out, variant)
        out.append(0 if data is None else 1)
        if data is not None:
            write_value(out, data)
    else:
        raise FormatError(f"unknown kind {k}")


def write_binary(fields) -> bytes:
    """StructSerializer::to_binary: header with the Tensor object type for every
    struct (binary/structs.rs:90-120), then the field count and fields."""
    fields = list(fields.items() if isinstance(fields, dict) else fields)
    body = bytearray()
    body += struct.pack("<Q", len(fields))
    for name, v in fields:
        _w_string(body, name)
        write_value(body, v)
    header = struct.pack("<IIIQI", MAGIC, VERSION, 0, len(body), 0x1001)
    return bytes(header) + bytes(body)


class _Reader:
    def __init__(self, data: bytes):
        self.d, self.p = data, 0

    def take(self, n: int) -> bytes:
        if len(self.d) - self.p < n:
            raise FormatError("failed to fill whole buffer")
        b = self.d[self.p:self.p + n]
        self.p += n
        return b

    def unpack(self, fmt: str):
        return struct.unpack(fmt, self.take(struct.calcsize(fmt)))[0]

    def boolean(self) -> bool:  # reader.rs read_bool
        b = self.unpack("<B")
        if b > 1:
            raise FormatError(f"Invalid boolean value: {b}")
        return b == 1

    def string(self) -> str:  # reader.rs read_string: at most 1,000,000 bytes, UTF-8
        n = self.unpack("<I")
        if n > 1_000_000:
            raise FormatError(f"String length {n} exceeds maximum allowed")
        try:
            return self.take(n).decode("utf-8")
        except UnicodeDecodeError as e:
            raise FormatError(f"Invalid UTF-8 string: {e}") from None

    def vec_u8(self) -> bytes:  # read_vec_u8: at most 100,000,000 bytes
        n = self.unpack("<Q")
        if n > 100_000_000:
            raise FormatError(f"Collection length {n} exceeds maximum allowed")
        return self.take(n)


def read_value(r: _Reader) -> FV:
    """binary/structs.rs:349-460"""
    tag = r.unpack("<B")
    if tag >= len(KINDS):
        raise FormatError(f"Unknown type tag: {tag}")
    k = KINDS[tag]
    if k == "Bool":
        return FV(k, r.boolean())
    fmt = {"I8": "<b", "U8": "<B", "I16": "<h", "U16": "<H", "I32": "<i", "U32": "<I", "I64": "<q",
           "U64": "<Q", "Usize": "<Q", "F64": "<d"}
    if k in fmt:
        return FV(k, r.unpack(fmt[k]))
    if k == "F32":
        return FV(k, np.frombuffer(r.take(4), np.float32)[0])
    if k in ("String", "JsonObject"):
        return FV(k, r.string())
    if k in ("Bytes", "BinaryObject"):
        return FV(k, r.vec_u8())
    if k == "Array":
        n = r.unpack("<Q")
        return FV(k, [read_value(r) for _ in range(n)])
    if k == "Optional":
        return FV(k, read_value(r) if r.boolean() else None)
    if k == "Object":
        n = r.unpack("<Q")
        d = {}
        for _ in range(n):
            key = r.string()
            d[key] = read_value(r)
        return FV(k, d)
    variant = r.string()
    return FV(k, (variant, read_value(r) if r.boolean() else None))


def read_binary(data: bytes) -> dict:
    """StructDeserializer::from_binary (binary/header.rs:76-106, :178-215;
    binary/structs.rs:293-312)."""
    r = _Reader(bytes(data))
    magic = r.unpack("<I")
    if magic != MAGIC:
        raise FormatError(f"Invalid magic number: expected 0x{MAGIC:08X}, found 0x{magic:08X}")
    version = r.unpack("<I")
    if version != VERSION:
        raise FormatError(f"Version mismatch: expected {VERSION}, found {version}")
    r.unpack("<I")  # checksum, not validated
    length = r.unpack("<Q")
    otype = r.unpack("<I")
    if otype not in OBJECT_TYPES:
        raise FormatError(f"Unknown object type: 0x{otype:08X}")
    if otype != 0x1001:
        raise FormatError(f"Object type mismatch: expected Tensor, found {OBJECT_TYPES[otype]}")
    if r.p + length > len(r.d):
        raise FormatError("Data length mismatch")
    n = r.unpack("<Q")
    fields = {}
    for _ in range(n):
        name = r.string()
        fields[name] = read_value(r)
    return fields


# ---- JSON -----------------------------------------------------------------------------

def rust_display(x, f32: bool = True) -> str:
    """Rust's Display of a float: shortest round-trip digits in fixed notation
    (numpy's Dragon4 'unique' positional formatting gives the same digits)."""
    v = np.float32(x) if f32 else np.float64(x)
    if np.isnan(v):
        return "NaN"
    if np.isinf(v):
        return "-inf" if v < 0 else "inf"
    if v == 0:
        return "-0" if np.signbit(v) else "0"
    return np.format_float_positional(v, unique=True, trim="-")


def json_float(x, f32: bool = True) -> str:
    """json/structs.rs:80-95: '.0' after integral values (fract() == 0)."""
    v = np.float32(x) if f32 else np.float64(x)
    s = rust_display(v, f32)
    if np.isfinite(v) and float(v) == float(np.trunc(v)):
        s += ".0"
    return s


def escape_string(s: str) -> str:
    """json/escape.rs escape_string"""
    out = []
    for ch in s:
        o = ord(ch)
        if ch == '"':
            out.append('\\"')
        elif ch == "\\":
            out.append("\\\\")
        elif o == 8:
            out.append("\\b")
        elif o == 12:
            out.append("\\f")
        elif ch == "\n":
            out.append("\\n")
        elif ch == "\r":
            out.append("\\r")
        elif ch == "\t":
            out.append("\\t")
        elif o < 0x20 or 0x7F <= o <= 0x9F:
            out.append(f"\\u{o:04x}")
        else:
            out.append(ch)
    return "".join(out)


def value_json(v: FV) -> str:
    """json/structs.rs:67-184"""
    k, x = v.kind, v.value
    if k == "Bool":
        return "true" if x else "false"
    if k in ("I8", "I16", "I32", "I64", "U8", "U16", "U32", "U64", "Usize"):
        return str(int(x))
    if k == "F32":
        return json_float(x, True)
    if k == "F64":
        return json_float(x, False)
    if k == "String":
        return '"' + escape_string(x) + '"'
    if k in ("Bytes", "BinaryObject"):
        return '"' + bytes(x).hex() + '"'
    if k == "JsonObject":
        return x
    if k == "Array":
        return "[" + ",".join(value_json(e) for e in x) + "]"
    if k == "Optional":
        return "null" if x is None else value_json(x)
    if k == "Object":
        return "{" + ",".join(f'"{escape_string(key)}":{value_json(e)}' for key, e in x.items()) + "}"
    variant, data = x
    return '{"variant":"' + escape_string(variant) + '","data":' + ("null" if data is None else value_json(data)) + "}"


def to_json(fields) -> str:
    """json/structs.rs:32-43 (top-level names are not escaped)"""
    fields = list(fields.items() if isinstance(fields, dict) else fields)
    return "{" + ",".join(f'"{name}":{value_json(v)}' for name, v in fields) + "}"


def number_fv(n: float) -> FV:
    """json/structs.rs:232-256.  Integral values: i64 (saturating), then the
    narrowest signed type -- the usize branch compares with `usize::MAX as
    i64` = -1 and never applies.  Others: F64."""
    if n == np.trunc(n):
        if n >= 2.0 ** 63:
            i = 2 ** 63 - 1
        elif n <= -(2.0 ** 63):
            i = -(2 ** 63)
        else:
            i = int(n)
        for kind, lo, hi in (("I8", -128, 127), ("I16", -32768, 32767),
                             ("I32", -2 ** 31, 2 ** 31 - 1)):
            if lo <= i <= hi:
                return FV(kind, i)
        return FV("I64", i)
    return FV("F64", float(n))


def _from_py(x) -> FV:
    if x is None:
        return FV("Optional", None)
    if isinstance(x, bool):
        return FV("Bool", x)
    if isinstance(x, float):
        return number_fv(x)
    if isinstance(x, str):
        h = x[2:]
        if x.startswith("0x") and len(x) > 2 and len(h) % 2 == 0 and all(c in "0123456789abcdefABCDEF" for c in h):
            return FV("Bytes", bytes.fromhex(h))
        return FV("String", x)
    if isinstance(x, list):
        return FV("Array", [_from_py(e) for e in x])
    if isinstance(x, dict):
        if len(x) == 2 and "variant" in x and "data" in x:
            if not isinstance(x["variant"], str):
                raise FormatError("Enum variant must be a string")
            data = None if x["data"] is None else _from_py(x["data"])
            return FV("Enum", (x["variant"], data))
        return FV("Object", {k: _from_py(e) for k, e in x.items()})
    raise FormatError(f"unexpected JSON value {x!r}")


def _no_constant(name):
    raise FormatError(f"invalid JSON token {name}")


def from_json(text: str) -> dict:
    """json/structs.rs:186-200: the root must be an object; numbers are read
    as f64 (every number, as the reference's parser does)."""
    root = json.loads(text, parse_int=float, parse_float=float, parse_constant=_no_constant)
    if not isinstance(root, dict):
        raise FormatError("Expected JSON object at root")
    return {k: _from_py(v) for k, v in root.items()}


# ---- FieldValue accessors (core/types.rs:525-1263) -------------------------------------

_INTS = ("I8", "I16", "I32", "I64", "U8", "U16", "U32", "U64", "Usize")


def as_f32(v: FV) -> np.float32:
    if v.kind in ("F32", "F64") or v.kind in _INTS:
        return np.float32(v.value)
    raise FormatError(f"Expected f32, found {v.kind}")


def as_usize(v: FV) -> int:
    if v.kind in _INTS:
        if v.value < 0:
            raise FormatError(f"Cannot convert negative {v.kind} {v.value} to usize")
        return int(v.value)
    raise FormatError(f"Expected usize, found {v.kind}")


def as_bool(v: FV) -> bool:
    if v.kind != "Bool":
        raise FormatError(f"Expected bool, found {v.kind}")
    return bool(v.value)


# ---- Tensor / Adam fields -----------------------------------------------------------------

def contiguous_strides(dims):
    s, stride = [], 1
    for d in reversed(dims):
        s.append(stride)
        stride *= d
    return list(reversed(s))


def tensor_fields(data, dims, requires_grad=False, device=("Cpu", 0), shuffle=None):
    """Tensor::to_serializer (tensor/core/serialization.rs:181-199)"""
    dims = [int(d) for d in dims]
    shape = obj([("dims", array_usize(dims)), ("size", usize(int(np.prod(dims, dtype=np.int64)) if dims else 1)),
                 ("strides", array_usize(contiguous_strides(dims))), ("layout", enum_unit("Contiguous"))], shuffle)
    dev = obj([("type", enum_unit(device[0])), ("index", usize(device[1]))], shuffle)
    return [("data", array_f32(data)), ("shape", shape), ("device", dev),
            ("requires_grad", FV("Bool", bool(requires_grad)))]


def tensor_from_fields(fields: dict):
    """Tensor::from_deserializer (serialization.rs:201-248) -> (data, dims, requires_grad)"""
    def need(name):
        if name not in fields:
            raise FormatError(f"Validation failed for field '{name}': Field not found")
        return fields[name]
    data_fv = need("data")
    if data_fv.kind != "Array":
        raise FormatError("Expected Vec<f32>")
    data = np.array([as_f32(e) for e in data_fv.value], dtype=np.float32)
    shape = need("shape")
    if shape.kind != "Object":
        raise FormatError("Expected object for shape")
    s = shape.value
    dims = [as_usize(e) for e in s["dims"].value]
    size = as_usize(s["size"])
    strides = [as_usize(e) for e in s["strides"].value]
    if s["layout"].kind != "Enum" or s["layout"].value[0] not in ("Contiguous", "Strided", "View"):
        raise FormatError("bad layout")
    if size != int(np.prod(dims, dtype=np.int64)):
        raise FormatError(f"Shape size {size} doesn't match computed size")
    if len(dims) != len(strides):
        raise FormatError("Dimensions and strides must have same length")
    dev = need("device")
    if dev.value["type"].value[0] not in ("Cpu", "Cuda"):
        raise FormatError("Unknown device type variant")
    as_usize(dev.value["index"])
    rg = as_bool(need("requires_grad"))
    if data.size != size:
        raise FormatError(f"Data length {data.size} doesn't match shape size {size}")
    if strides != contiguous_strides(dims):
        raise FormatError("Reconstructed tensor shape doesn't match serialized shape")
    return data, dims, rg


def tensor_from_fv(v: FV):
    """Tensor::from_field_value (serialization.rs:251-288)"""
    if v.kind == "BinaryObject":
        return tensor_from_fields(read_binary(v.value))
    if v.kind == "JsonObject":
        return tensor_from_fields(from_json(v.value))
    if v.kind == "Object":
        return tensor_from_fields(v.value)
    raise FormatError("Expected binary object, JSON object, or structured object for tensor field")


CONFIG_KEYS = ("learning_rate", "beta1", "beta2", "eps", "weight_decay")


def config_fields(cfg: dict, shuffle=None):
    """AdamConfig::to_serializer (adam/serialization.rs:40-50)"""
    pairs = [(k, f32(cfg[k])) for k in CONFIG_KEYS] + [("amsgrad", FV("Bool", bool(cfg["amsgrad"])))]
    return pairs


def config_from_fields(fields: dict) -> dict:
    cfg = {k: float(as_f32(fields[k])) for k in CONFIG_KEYS}
    cfg["amsgrad"] = as_bool(fields["amsgrad"])
    return cfg


def adam_fields(config: dict, states: dict, step_count: int, insertion_order, nested: str = "json",
                shuffle=None):
    """Adam::to_serializer (adam/serialization.rs:140-160).  states: id ->
    dict(m, v, v_hat_max (or None), step, dims).  The reference nests each
    tensor as its JSON text (impls.rs:416-428), `nested="json"`."""
    def tensor_fv(arr, dims):
        fl = tensor_fields(arr, dims, False, shuffle=shuffle)
        if nested == "json":
            return FV("JsonObject", to_json(fl))
        if nested == "binary":
            return FV("BinaryObject", write_binary(fl))
        return obj(fl)
    st = []
    for pid, s in states.items():
        vm = FV("Optional", None if s.get("v_hat_max") is None else tensor_fv(s["v_hat_max"], s["dims"]))
        st.append((str(pid), obj([("m", tensor_fv(s["m"], s["dims"])), ("v", tensor_fv(s["v"], s["dims"])),
                                  ("v_hat_max", vm), ("step", usize(s["step"]))], shuffle)))
    return [("config", obj(config_fields(config), shuffle)), ("states", obj(st, shuffle)),
            ("step_count", usize(step_count)), ("insertion_order", array_usize(insertion_order))]


def adam_from_fields(fields: dict) -> dict:
    """Adam::from_deserializer (adam/serialization.rs:162-190)"""
    cfg = config_from_fields(fields["config"].value)
    states = {}
    for key, sv in fields["states"].value.items():
        if not key.lstrip("+").isdigit():
            raise FormatError(f"Invalid key '{key}' in parameter states map")
        s = sv.value
        m, dims, _ = tensor_from_fv(s["m"])
        v, _, _ = tensor_from_fv(s["v"])
        vm = s["v_hat_max"]
        vhat = None
        if vm.kind == "Optional":
            if vm.value is not None:
                vhat = tensor_from_fv(vm.value)[0]
        else:
            vhat = tensor_from_fv(vm)[0]
        states[int(key)] = dict(m=m, v=v, v_hat_max=vhat, step=as_usize(s["step"]), dims=dims)
    order = [as_usize(e) for e in fields["insertion_order"].value]
    return dict(config=cfg, states=states, step_count=as_usize(fields["step_count"]), insertion_order=order)
