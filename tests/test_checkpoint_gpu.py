"""Checkpoint / resume of device tensors and Adam state in the reference's
formats, checked against the format restatement (oracle/serialization.py).

* Tensor: the product's binary bytes and JSON text equal the restatement's for
  the same values (the product writes object members in the reference's
  declaration order); files written the reference's way -- members in any
  order, other numeric tags, whitespace -- load to the values the
  restatement reads.
* Adam: the restatement reads the product's checkpoints back to the
  optimizer's live state; a run checkpointed after k steps, reloaded,
  relinked and continued is bit-identical to the uninterrupted run; a
  checkpoint written the reference's way (nested tensors as JSON text)
  resumes the same way.
"""
from __future__ import annotations

import random
import struct
import time

import numpy as np
import pytest

from conftest import assert_bits_equal
from oracle import serialization as S

pytestmark = pytest.mark.gpu

SHAPES = [[], [0], [1], [7], [2, 3], [3, 5, 7], [300, 257]]


def T():
    import train_station_amd as mod
    return mod


def _values(shape, seed):
    n = int(np.prod(shape, dtype=np.int64)) if shape else 1
    rng = np.random.default_rng(seed)
    a = rng.standard_normal(n).astype(np.float32)
    special = np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, -1e-40, 3.4028235e38, 0.1, 1.0, -5.0],
                       np.float32)
    k = min(n, special.size)
    a[:k] = special[:k]
    return a


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)) or "scalar")
def test_tensor_binary_bytes_match_restatement(shape):
    for rg in (False, True):
        a = _values(shape, 1)
        t = T().Tensor.from_slice(a, shape)
        if rg:
            t.with_requires_grad()
        got = t.to_binary()
        want = S.write_binary(S.tensor_fields(a, shape, rg))
        assert got == want, (shape, rg)
        back = T().Tensor.from_binary(got)
        assert list(back.shape) == shape and back.requires_grad() == rg
        assert_bits_equal(back.data().reshape(-1), a)


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)) or "scalar")
def test_tensor_json_text_matches_restatement(shape):
    a = _values(shape, 2)
    t = T().Tensor.from_slice(a, shape)
    got = t.to_json()
    assert got == S.to_json(S.tensor_fields(a, shape, False))
    finite = np.isfinite(a)
    if finite.all():
        back = T().Tensor.from_json(got)
        want, _, _ = S.tensor_from_fields(S.from_json(got))
        assert_bits_equal(back.data().reshape(-1), want)


def test_tensor_nan_bits_survive_binary():
    a = np.array([1.0, 2.0, 3.0, 4.0, 5.0], np.float32)
    a.view(np.uint32)[2] = 0x7FC12345  # a NaN with a payload
    t = T().Tensor.from_slice(a, [5])
    back = T().Tensor.from_binary(t.to_binary())
    assert back.data().view(np.uint32)[2] == 0x7FC12345


def test_tensor_reads_reference_style_binary():
    rng = random.Random(5)
    a = _values([4, 9], 3)
    for trial in range(4):
        fl = S.tensor_fields(a, [4, 9], trial % 2 == 1, device=("Cuda", 3) if trial == 3 else ("Cpu", 0),
                             shuffle=rng)
        if trial >= 2:
            fl = list(reversed(fl))  # top-level order is not significant to the reader
        if trial == 2:
            # elements of other numeric types read through FieldValue::as_f32
            fl = [(k, S.FV("Array", [S.FV("I32", 7), S.FV("F64", 0.25)] + v.value[2:]) if k == "data" else v)
                  for k, v in fl]
        raw = S.write_binary(fl)
        want, dims, rg = S.tensor_from_fields(S.read_binary(raw))
        t = T().Tensor.from_binary(raw)
        assert list(t.shape) == dims and t.requires_grad() == rg
        assert_bits_equal(t.data().reshape(-1), want)


def test_tensor_reads_reference_style_json():
    rng = random.Random(8)
    a = np.array([[1.0, -0.0, 2.5], [1e30, -7.0, 0.125]], np.float32)
    fl = S.tensor_fields(a, [2, 3], True, shuffle=rng)
    text = S.to_json(list(reversed(fl)))
    text = text.replace(",", " ,\n ").replace(":", " : ")
    want, dims, rg = S.tensor_from_fields(S.from_json(text))
    assert want[1] == 0.0 and not np.signbit(want[1])  # -0.0 comes back as the integer 0
    assert want[3] == np.float32(2.0 ** 63)            # 1e30 saturates as an i64
    t = T().Tensor.from_json(text)
    assert list(t.shape) == dims and t.requires_grad() == rg
    assert_bits_equal(t.data().reshape(-1), want)


def test_tensor_files(tmp_path):
    a = _values([33, 17], 4)
    t = T().Tensor.from_slice(a, [33, 17]).with_requires_grad()
    t.save_binary(tmp_path / "t.bin")
    assert (tmp_path / "t.bin").read_bytes() == S.write_binary(S.tensor_fields(a, [33, 17], True))
    b = T().Tensor.load_binary(tmp_path / "t.bin")
    assert_bits_equal(b.data().reshape(-1), a)
    assert b.requires_grad()
    # JSON: the writer prints infinities as `inf`, which the reader (like the
    # reference's, json/parser.rs) does not accept
    t.save_json(tmp_path / "inf.json")
    with pytest.raises(T().TsError, match="Unexpected character 'i'"):
        T().Tensor.load_json(tmp_path / "inf.json")
    f = np.where(np.isfinite(a), a, np.float32(7.0)).astype(np.float32)
    T().Tensor.from_slice(f, [33, 17]).save_json(tmp_path / "t.json")
    j = T().Tensor.load_json(tmp_path / "t.json")
    want, _, _ = S.tensor_from_fields(S.from_json((tmp_path / "t.json").read_text()))
    assert_bits_equal(j.data().reshape(-1), want)
    with pytest.raises(T().TsError, match="cannot open"):
        T().Tensor.load_binary(tmp_path / "missing.bin")


def test_tensor_load_errors():
    Tm = T()
    good = S.write_binary(S.tensor_fields(np.arange(6, dtype=np.float32), [2, 3]))
    with pytest.raises(Tm.TsError, match="magic"):
        Tm.Tensor.from_binary(struct.pack("<I", 0xDEADBEEF) + good[4:])
    with pytest.raises(Tm.TsError):
        Tm.Tensor.from_binary(good[:-5])
    fl = dict(S.tensor_fields(np.arange(6, dtype=np.float32), [2, 3]))
    fl["data"] = S.array_f32(np.arange(5, dtype=np.float32))
    with pytest.raises(Tm.TsError, match="Data length 5 doesn't match shape size 6"):
        Tm.Tensor.from_binary(S.write_binary(fl))
    fl = dict(S.tensor_fields(np.arange(6, dtype=np.float32), [2, 3]))
    del fl["device"]
    with pytest.raises(Tm.TsError, match="'device': Field not found"):
        Tm.Tensor.from_binary(S.write_binary(fl))
    fl = dict(S.tensor_fields(np.arange(6, dtype=np.float32), [2, 3]))
    fl["shape"].value["strides"] = S.array_usize([1, 2])
    with pytest.raises(Tm.TsError, match="Reconstructed tensor shape"):
        Tm.Tensor.from_binary(S.write_binary(fl))
    fl = dict(S.tensor_fields(np.arange(6, dtype=np.float32), [2, 3]))
    fl["shape"].value["size"] = S.usize(7)
    with pytest.raises(Tm.TsError, match="Shape size 7 doesn't match computed size 6"):
        Tm.Tensor.from_json(S.to_json(fl))


# ---- Adam ---------------------------------------------------------------------------------

def _mlp(seed=0, widths=(32, 48, 8), batch=64):
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((batch, widths[0])).astype(np.float32)
    t = rng.standard_normal((batch, widths[-1])).astype(np.float32)
    ws = [(rng.standard_normal((widths[i], widths[i + 1])) / np.sqrt(widths[i])).astype(np.float32)
          for i in range(len(widths) - 1)]
    bs = [np.zeros(widths[i + 1], np.float32) for i in range(len(widths) - 1)]
    return x, t, ws, bs


def _params(ws, bs):
    Tm = T()
    ps = []
    for w, b in zip(ws, bs):
        ps.append(Tm.Tensor.from_slice(w, w.shape).with_requires_grad())
        ps.append(Tm.Tensor.from_slice(b, b.shape).with_requires_grad())
    return ps


def _step(opt, ps, x, t):
    Tm = T()
    h = Tm.Tensor.from_slice(x, x.shape)
    for i in range(0, len(ps), 2):
        h = h.matmul(ps[i]).add_tensor(ps[i + 1])
        if i + 2 < len(ps):
            h = h.relu()
    loss = h.sub_tensor(Tm.Tensor.from_slice(t, t.shape)).pow_scalar(2.0).mean()
    loss.backward()
    opt.step(ps)
    opt.zero_grad(ps)


def _new_opt(amsgrad):
    return T().Adam.with_config(learning_rate=1e-2, weight_decay=1e-3 if amsgrad else 0.0,
                                amsgrad=amsgrad)


@pytest.mark.parametrize("amsgrad", [False, True])
@pytest.mark.parametrize("fmt", ["binary", "json"])
def test_resume_is_bit_identical(tmp_path, amsgrad, fmt):
    x, t, ws, bs = _mlp(1)
    # uninterrupted: 7 steps
    ps = _params(ws, bs)
    opt = _new_opt(amsgrad)
    opt.add_parameters(ps)
    for _ in range(7):
        _step(opt, ps, x, t)
    want = [p.data() for p in ps]
    # checkpointed after 3 steps, reloaded into fresh objects, 4 more steps
    ps = _params(ws, bs)
    opt = _new_opt(amsgrad)
    opt.add_parameters(ps)
    for _ in range(3):
        _step(opt, ps, x, t)
    ext = "bin" if fmt == "binary" else "json"
    for i, p in enumerate(ps):
        getattr(p, f"save_{fmt}")(tmp_path / f"p{i}.{ext}")
    getattr(opt, f"save_{fmt}")(tmp_path / f"adam.{ext}")
    del opt, ps
    ps2 = [getattr(T().Tensor, f"load_{fmt}")(tmp_path / f"p{i}.{ext}") for i in range(4)]
    assert all(p.requires_grad() for p in ps2)
    opt2 = getattr(T().Adam, f"load_{fmt}")(tmp_path / f"adam.{ext}")
    assert opt2.saved_parameter_count() == 4 and opt2.step_count() == 3
    assert opt2.config()["amsgrad"] == amsgrad
    probe = getattr(T().Adam, f"load_{fmt}")(tmp_path / f"adam.{ext}")
    with pytest.raises(T().TsError, match="must be linked"):
        probe.step(ps2)  # the saved states are still under the old ids (adam/mod.rs:1033-1037)
    opt2.relink_parameters(ps2)
    assert [opt2.parameter_step(p) for p in ps2] == [3, 3, 3, 3]
    for _ in range(4):
        _step(opt2, ps2, x, t)
    for p, w in zip(ps2, want):
        assert_bits_equal(p.data(), w)


@pytest.mark.parametrize("amsgrad", [False, True])
def test_adam_checkpoint_read_by_restatement(amsgrad):
    x, t, ws, bs = _mlp(2)
    ps = _params(ws, bs)
    opt = _new_opt(amsgrad)
    opt.add_parameters(ps)
    for _ in range(2):
        _step(opt, ps, x, t)
    for raw, how in ((opt.to_binary(), "binary"), (opt.to_json(), "json")):
        fields = S.read_binary(raw) if how == "binary" else S.from_json(raw)
        st = S.adam_from_fields(fields)
        assert st["step_count"] == 2
        assert st["insertion_order"] == [p.id() for p in ps]
        assert st["config"]["amsgrad"] == amsgrad
        assert np.float32(st["config"]["learning_rate"]) == np.float32(1e-2)
        for p in ps:
            s = st["states"][p.id()]
            assert s["step"] == 2 and s["dims"] == list(p.shape)
            assert_bits_equal(s["m"], opt.state(p, "m"))
            assert_bits_equal(s["v"], opt.state(p, "v"))
            assert (s["v_hat_max"] is not None) == amsgrad
    # the product's JSON equals the restatement's text for the same state
    exact = S.adam_from_fields(S.read_binary(opt.to_binary()))["states"]
    states = {p.id(): dict(m=opt.state(p, "m"), v=opt.state(p, "v"), step=2, dims=list(p.shape),
                           v_hat_max=exact[p.id()]["v_hat_max"]) for p in ps}
    cfg = opt.config()
    want = S.to_json(S.adam_fields(cfg, states, 2, [p.id() for p in ps], nested="json"))
    assert opt.to_json() == want


def test_adam_resumes_from_reference_style_checkpoint():
    # the reference nests m / v as JSON text inside its binary checkpoint and
    # orders members arbitrarily; such a file resumes exactly
    x, t, ws, bs = _mlp(3)
    ps = _params(ws, bs)
    opt = _new_opt(False)
    opt.add_parameters(ps)
    for _ in range(3):
        _step(opt, ps, x, t)
    rng = random.Random(1)
    states = {p.id(): dict(m=opt.state(p, "m"), v=opt.state(p, "v"), v_hat_max=None, step=3,
                           dims=list(p.shape)) for p in ps}
    raw = S.write_binary(S.adam_fields(opt.config(), states, 3, [p.id() for p in ps], nested="json",
                                       shuffle=rng))
    snap = [p.data() for p in ps]
    ps2 = [T().Tensor.from_slice(a, p.shape).with_requires_grad() for a, p in zip(snap, ps)]
    opt2 = T().Adam.from_binary(raw)
    opt2.relink_parameters(ps2)
    _step(opt, ps, x, t)
    _step(opt2, ps2, x, t)
    for a, b in zip(ps, ps2):
        assert_bits_equal(b.data(), a.data())


def test_relink_errors():
    Tm = T()
    x, t, ws, bs = _mlp(4)
    ps = _params(ws, bs)
    opt = _new_opt(False)
    opt.add_parameters(ps)
    _step(opt, ps, x, t)
    raw = opt.to_binary()
    o = Tm.Adam.from_binary(raw)
    with pytest.raises(Tm.TsError, match="Parameter count mismatch: expected 4 parameters, got 3"):
        o.relink_parameters(ps[:3])
    swapped = [ps[1], ps[0], ps[2], ps[3]]
    with pytest.raises(Tm.TsError, match="Shape mismatch for parameter at position 0"):
        o.relink_parameters(swapped)
    plain = [Tm.Tensor.from_slice(p.data(), p.shape) for p in ps]
    with pytest.raises(Tm.TsError, match="Parameter at index 0 must require gradients"):
        o.relink_parameters(plain)
    o.relink_parameters(ps)
    assert o.saved_parameter_count() == 4


def test_large_checkpoint_round_trip(tmp_path):
    # a config-5 weight (4096 x 4096) and its Adam state: the nested binary
    # objects stay under the reference reader's 10^8-byte limit
    Tm = T()
    n = 4096
    w = Tm.Tensor.randn([n, n], seed=5).with_requires_grad()
    opt = Tm.Adam.new()
    opt.add_parameter(w)
    g = Tm.Tensor.randn([n, n], seed=6)
    w.set_grad(g)
    opt.step([w])
    t0 = time.perf_counter()
    w.save_binary(tmp_path / "w.bin")
    t1 = time.perf_counter()
    opt.save_binary(tmp_path / "adam.bin")
    t2 = time.perf_counter()
    w2 = Tm.Tensor.load_binary(tmp_path / "w.bin")
    t3 = time.perf_counter()
    o2 = Tm.Adam.load_binary(tmp_path / "adam.bin")
    t4 = time.perf_counter()
    mb = 4 * n * n / 1e6
    print(f"checkpoint {n}x{n}: tensor save {mb / (t1 - t0):.0f} MB/s, load {mb / (t3 - t2):.0f} MB/s; "
          f"adam save {2 * mb / (t2 - t1):.0f} MB/s, load {2 * mb / (t4 - t3):.0f} MB/s", flush=True)
    assert_bits_equal(w2.data(), w.data())
    o2.relink_parameters([w2])
    assert_bits_equal(o2.state(w2, "m"), opt.state(w, "m"))
    assert_bits_equal(o2.state(w2, "v"), opt.state(w, "v"))
    raw = (tmp_path / "adam.bin").read_bytes()
    hdr = S._Reader(raw)
    assert hdr.unpack("<I") == S.MAGIC
