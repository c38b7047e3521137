"""Pins of the serialization restatement (oracle/serialization.py) and, on the
CPU, of the product's format core through AdamConfig, which needs no device.

Facts used, none taken from the restatement itself:
* the reference's own format tests: header layout and errors
  (binary/header.rs tests), primitive byte counts (binary/writer.rs tests),
  the tagged value bytes (binary/structs.rs tests), JSON number reading
  (json/structs.rs tests), Adam config round trips (adam/serialization.rs tests);
* the byte layout implied by Rust's to_le_bytes and u32 string lengths,
  assembled by hand with struct;
* Rust's float Display (shortest round-trip digits, fixed notation) on
  values whose text is known, and its integer cast rules.
"""
from __future__ import annotations

import random
import struct

import numpy as np
import pytest

from oracle import serialization as S


def test_header_layout_known_bytes():
    b = S.write_binary([("x", S.FV("Bool", True))])
    # magic 0x54535F42 little-endian = "B_ST", version 1, checksum 0,
    # data length (u64), object type 0x1001
    assert b[:4] == b"B_ST" and struct.unpack("<I", b[:4])[0] == 0x54535F42
    magic, version, checksum, length, otype = struct.unpack("<IIIQI", b[:24])
    assert (version, checksum, otype) == (1, 0, 0x1001)
    assert length == len(b) - 24
    # body: field count u64, name (u32 len + bytes), tag 0, value 1
    assert b[24:] == struct.pack("<Q", 1) + struct.pack("<I", 1) + b"x" + bytes([0, 1])


def test_header_errors_as_reference_tests():
    good = S.write_binary([("x", S.usize(3))])
    bad_magic = struct.pack("<I", 0xDEADBEEF) + good[4:]
    with pytest.raises(S.FormatError, match="magic"):
        S.read_binary(bad_magic)
    bad_version = good[:4] + struct.pack("<I", 999) + good[8:]
    with pytest.raises(S.FormatError, match="Version"):
        S.read_binary(bad_version)
    bad_type = good[:20] + struct.pack("<I", 0x9999)
    with pytest.raises(S.FormatError, match="Unknown object type"):
        S.read_binary(bad_type + good[24:])
    with pytest.raises(S.FormatError):
        S.read_binary(good[:-1])  # truncated


def test_primitive_byte_counts_from_writer_tests():
    # writer.rs test_basic_types_writing: u8, u16, u32, u64, f32, bool, "Hello, World!"
    out = bytearray()
    out += struct.pack("<BHIQ", 42, 1234, 0x12345678, 0x123456789ABCDEF0)
    out += np.float32(np.pi).tobytes() + bytes([1])
    S._w_string(out, "Hello, World!")
    assert len(out) == 1 + 2 + 4 + 8 + 4 + 1 + 4 + 13


def test_tagged_values_known_bytes():
    # binary/structs.rs test_read_field_value_binary: tag 0 bool, tag 3 i32, tag 12 string
    raw = bytes([0, 1]) + bytes([3]) + struct.pack("<i", 42) + bytes([12]) + struct.pack("<I", 5) + b"hello"
    r = S._Reader(raw)
    assert S.read_value(r) == S.FV("Bool", True)
    assert S.read_value(r) == S.FV("I32", 42)
    assert S.read_value(r) == S.FV("String", "hello")
    out = bytearray()
    for v in (S.FV("Bool", True), S.FV("I32", 42), S.FV("String", "hello")):
        S.write_value(out, v)
    assert bytes(out) == raw
    # an F32 is tag 10 + 4 little-endian bytes; an Array is tag 16 + u64 count
    out = bytearray()
    S.write_value(out, S.array_f32([1.0, -2.5]))
    assert bytes(out) == bytes([16]) + struct.pack("<Q", 2) + bytes([10]) + struct.pack("<f", 1.0) + \
        bytes([10]) + struct.pack("<f", -2.5)


def test_reader_limits():
    long = bytes([12]) + struct.pack("<I", 1_000_001) + b"a" * 1_000_001
    with pytest.raises(S.FormatError, match="exceeds maximum"):
        S.read_value(S._Reader(long))
    with pytest.raises(S.FormatError, match="Invalid boolean"):
        S.read_value(S._Reader(bytes([0, 2])))
    with pytest.raises(S.FormatError, match="Unknown type tag"):
        S.read_value(S._Reader(bytes([20])))


@pytest.mark.parametrize("x,text", [
    (0.1, "0.1"), (1.0, "1.0"), (-3.0, "-3.0"), (1e-7, "0.0000001"), (0.5, "0.5"),
    (123456790.0, "123456790.0"), (16777216.0, "16777216.0"),
    (3.4028235e38, "340282350000000000000000000000000000000.0"),
    (1.17549435e-38, "0.000000000000000000000000000000000000011754944"),
    (1e-45, "0.000000000000000000000000000000000000000000001"),
    (-0.0, "-0.0"), (float("nan"), "NaN"), (float("inf"), "inf"), (float("-inf"), "-inf"),
    (2.5e-5, "0.000025"), (1234.5, "1234.5"),
])
def test_json_float_text(x, text):
    # Rust's Display + the ".0" rule of json/structs.rs:80-87
    assert S.json_float(x) == text


def test_json_numbers_as_the_reference_reads_them():
    f = S.from_json('{"a": 42, "b": 300, "c": 70000, "d": 1e10, "e": 1.5, "f": -0.0, "g": 1e30, "h": -7}')
    assert f["a"] == S.FV("I8", 42)            # the usize branch never applies
    assert f["b"].kind == "I16" and f["c"].kind == "I32" and f["d"].kind == "I64"
    assert f["e"] == S.FV("F64", 1.5)
    assert f["f"] == S.FV("I8", 0)             # -0.0 loses its sign
    assert f["g"] == S.FV("I64", 2 ** 63 - 1)  # saturating cast
    assert f["h"] == S.FV("I8", -7)
    assert S.as_usize(f["a"]) == 42            # json/structs.rs test_json_number_parsing
    assert [S.as_usize(v) for v in S.from_json('{"values": [1, 2, 3]}')["values"].value] == [1, 2, 3]
    with pytest.raises(S.FormatError):
        S.as_usize(f["h"])
    with pytest.raises(S.FormatError):
        S.from_json('{"x": NaN}')
    with pytest.raises(S.FormatError):
        S.from_json("[1, 2]")  # root must be an object


def test_json_enum_and_bytes_rules():
    f = S.from_json('{"e": {"variant": "Cpu", "data": null}, "o": {"variant": "X", "data": 1, "z": 2},'
                    ' "b": "0x4865", "s": "0x486"}')
    assert f["e"] == S.FV("Enum", ("Cpu", None))
    assert f["o"].kind == "Object"
    assert f["b"] == S.FV("Bytes", b"He")
    assert f["s"] == S.FV("String", "0x486")


def test_escape_rules():
    assert S.escape_string('a"b\\c\n\t\x08\x0c\r\x01\x7f\x85é') == 'a\\"b\\\\c\\n\\t\\b\\f\\r\\u0001\\u007f\\u0085é'


def test_tensor_fields_round_trip_both_formats():
    rng = random.Random(3)
    data = np.array([0.0, -0.0, 1.5, -2.25, 3.4028235e38, 1e-45, 0.1], np.float32)
    for shuffle in (None, rng):
        fl = S.tensor_fields(data, [7], True, shuffle=shuffle)
        d, dims, rg = S.tensor_from_fields(S.read_binary(S.write_binary(fl)))
        assert d.tobytes() == data.tobytes() and dims == [7] and rg
        d, dims, rg = S.tensor_from_fields(S.from_json(S.to_json(fl)))
        want = data.copy()
        want[1] = 0.0  # JSON reads -0.0 as the integer 0
        want[4] = np.float32(2.0 ** 63)  # integral values >= 2^63 saturate to i64::MAX
        assert d.tobytes() == want.tobytes()


def test_tensor_validation_errors():
    fl = dict(S.tensor_fields(np.zeros(6, np.float32), [2, 3]))
    bad = dict(fl)
    bad["data"] = S.array_f32(np.zeros(5, np.float32))
    with pytest.raises(S.FormatError, match="Data length 5"):
        S.tensor_from_fields(bad)
    bad = dict(fl)
    del bad["requires_grad"]
    with pytest.raises(S.FormatError, match="Field not found"):
        S.tensor_from_fields(bad)


# ---- the product's format core on the CPU (AdamConfig needs no device) --------------------

CFG = dict(learning_rate=2e-3, beta1=0.85, beta2=0.995, eps=1e-9, weight_decay=5e-4, amsgrad=False)


def _product():
    import train_station_amd as T
    return T


def test_product_config_binary_matches_oracle_bytes():
    T = _product()
    got = T.adam_config_to_binary(CFG)
    assert got == S.write_binary(S.config_fields(CFG))
    back = T.adam_config_from_binary(got)
    for k in S.CONFIG_KEYS:
        assert np.float32(back[k]) == np.float32(CFG[k])
    assert back["amsgrad"] is False


def test_product_config_json_matches_oracle_text():
    T = _product()
    cfg = dict(CFG, amsgrad=True, learning_rate=1.0, weight_decay=0.0)
    got = T.adam_config_to_json(cfg)
    assert got == S.to_json(S.config_fields(cfg))
    assert '"learning_rate":1.0' in got and '"weight_decay":0.0' in got
    back = T.adam_config_from_json(got)
    assert back["amsgrad"] is True and np.float32(back["beta2"]) == np.float32(0.995)


def test_product_reads_reference_style_config():
    T = _product()
    rng = random.Random(11)
    # member order shuffled, whitespace, integers where floats were written
    text = S.to_json(S.config_fields(dict(CFG, learning_rate=3.0)))
    d = S.from_json(text)
    items = list(d.items())
    rng.shuffle(items)
    text = "{\n  " + ",\n  ".join(f'"{k}" : {S.value_json(v)}' for k, v in items) + "\n}"
    back = T.adam_config_from_json(text.replace("3.0", "3"))
    assert back["learning_rate"] == 3.0 and np.float32(back["eps"]) == np.float32(1e-9)
    b = S.write_binary(list(reversed(S.config_fields(CFG))))
    back = T.adam_config_from_binary(b)
    assert np.float32(back["weight_decay"]) == np.float32(5e-4)


@pytest.mark.parametrize("text,msg", [
    ('{"learning_rate": 1.0}', "Field not found"),
    ('{"learning_rate": 1.0, "beta1": 0.9, "beta2": 0.9, "eps": 1e-8, "weight_decay": 0.0, "amsgrad": 1}',
     "Expected bool"),
    ('{"learning_rate": "x", "beta1": 0.9, "beta2": 0.9, "eps": 1e-8, "weight_decay": 0.0, "amsgrad": true}',
     "Expected f32"),
    ('{"learning_rate": 1.0,}', "JSON"),
    ('[1]', "object at root"),
])
def test_product_config_errors(text, msg):
    T = _product()
    with pytest.raises(T.TsError, match=msg):
        T.adam_config_from_json(text)


def test_product_binary_errors():
    T = _product()
    good = T.adam_config_to_binary(CFG)
    with pytest.raises(T.TsError, match="magic"):
        T.adam_config_from_binary(struct.pack("<I", 0xDEADBEEF) + good[4:])
    with pytest.raises(T.TsError, match="Version"):
        T.adam_config_from_binary(good[:4] + struct.pack("<I", 999) + good[8:])
    with pytest.raises(T.TsError, match="end of data|Data length"):
        T.adam_config_from_binary(good[:-3])


def test_product_formats_consecutive_floats_independently():
    # a long value followed by short ones in one document: each float's text
    # must not depend on the one before it
    T = _product()
    cfg = dict(learning_rate=3.4028235e38, beta1=0.1, beta2=1e-45, eps=-1e-40, weight_decay=1.0, amsgrad=False)
    assert T.adam_config_to_json(cfg) == S.to_json(S.config_fields(cfg))
    for big, small in ((1.2345678e-30, 2.0), (-123456.79, 0.5), (3.4028235e38, 1e-7)):
        cfg = dict(learning_rate=big, beta1=small, beta2=big, eps=small, weight_decay=small, amsgrad=True)
        assert T.adam_config_to_json(cfg) == S.to_json(S.config_fields(cfg))
