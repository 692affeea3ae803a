"""Archive format and checkpoint resume, host side (no GPU).

The archive format and the checkpoint layout are the reference's
(serialization.py, training/checkpoint.py); `golden/checkpoint_reference.nt`
was written by the reference's own save_checkpoint, and the exception texts
in golden.json come from its save/load.
"""

from __future__ import annotations

import json
import math
import struct
import zipfile
from pathlib import Path

import numpy as np
import pytest

import namitorch_amd as nt
from namitorch_amd import checkpoint as ck
from namitorch_amd import serialization as ser

GOLDEN = Path(__file__).resolve().parent / "golden"


def _golden():
    return json.loads((GOLDEN / "golden.json").read_text())


def _zip_entries(path):
    with zipfile.ZipFile(path) as archive:
        return {info.filename: (info.compress_type, archive.read(info.filename)) for info in archive.infolist()}


def test_roundtrip_preserves_types_and_bits(tmp_path):
    rng = np.random.default_rng(5)
    f32 = rng.standard_normal((3, 5)).astype(np.float32)
    f32[0, :4] = [np.inf, -np.inf, -0.0, np.float32(1e-45)]
    bf = nt.tensor((f32.view(np.uint32) & np.uint32(0xFFFF0000)).view(np.float32), dtype=nt.bfloat16)
    obj = {
        "none": None, "flag": True, "count": 7, "name": "adamw",
        "floats": [0.1, -0.0, math.inf, -math.inf, 5e-324, 1.7976931348623157e308],
        "nan": math.nan,
        "tuple": (1, (2.5, "x")),
        "w32": nt.tensor(f32, requires_grad=True),
        "w16": nt.tensor(f32.astype(np.float16)),
        "w64": nt.tensor(f32.astype(np.float64)),
        "i32": nt.tensor(np.arange(6, dtype=np.int32)),
        "mask": nt.tensor(np.array([True, False])),
        "bf16": bf,
        "raw": np.arange(12, dtype=np.uint16).reshape(3, 4),
    }
    path = tmp_path / "state.nt"
    ser.save(obj, path)
    back = ser.load(path)
    assert list(back) == list(obj)
    assert back["none"] is None and back["flag"] is True and back["count"] == 7 and back["name"] == "adamw"
    assert [struct.pack("<d", v) for v in back["floats"]] == [struct.pack("<d", v) for v in obj["floats"]]
    assert math.isnan(back["nan"])
    assert back["tuple"] == (1, (2.5, "x")) and isinstance(back["tuple"], tuple) and isinstance(back["tuple"][1], tuple)
    for key in ("w32", "w16", "w64", "i32", "mask"):
        assert isinstance(back[key], nt.Tensor) and back[key].dtype is obj[key].dtype
        assert back[key].bits().tobytes() == obj[key].bits().tobytes()
    assert back["w32"].requires_grad and not back["w16"].requires_grad
    # bfloat16 travels as its exact float32 widening.
    assert back["bf16"].dtype is nt.float32
    assert back["bf16"].numpy().tobytes() == bf.numpy().tobytes()
    assert isinstance(back["raw"], np.ndarray) and back["raw"].dtype == np.uint16
    assert np.array_equal(back["raw"], obj["raw"])


def test_archive_layout_is_the_reference_format(tmp_path):
    path = tmp_path / "layout.nt"
    ser.save({"a": nt.tensor(np.ones(3, np.float32)), "b": [np.zeros((2, 2), np.int64)], "c": 0.5}, path)
    entries = _zip_entries(path)
    assert list(entries) == ["metadata.json", "arrays.npz"]
    assert all(kind == zipfile.ZIP_STORED for kind, _ in entries.values())
    raw = entries["metadata.json"][1]
    metadata = json.loads(raw)
    assert raw == json.dumps(metadata, ensure_ascii=True, separators=(",", ":")).encode()
    assert metadata["format_version"] == 1
    assert metadata["arrays"] == [{"id": "a0", "dtype": "<f4", "shape": [3], "nbytes": 12},
                                  {"id": "a1", "dtype": "<i8", "shape": [2, 2], "nbytes": 32}]
    assert metadata["tree"] == {"type": "dict", "items": [
        ["a", {"type": "tensor", "id": "a0", "requires_grad": False}],
        ["b", {"type": "list", "items": [{"type": "ndarray", "id": "a1"}]}],
        ["c", {"type": "float", "value": "0x1.0000000000000p-1"}]]}
    inner_path = tmp_path / "inner.npz"
    inner_path.write_bytes(entries["arrays.npz"][1])
    with zipfile.ZipFile(inner_path) as inner:
        assert [info.filename for info in inner.infolist()] == ["a0.npy", "a1.npy"]
        assert all(info.compress_type == zipfile.ZIP_STORED for info in inner.infolist())
        assert inner.read("a0.npy")[:8] == b"\x93NUMPY\x01\x00"


def test_error_texts_match_reference(tmp_path):
    expected = _golden()["serialization_errors"]
    cyclic = []
    cyclic.append(cyclic)
    cases = {
        "save_complex": lambda: ser.save({"x": np.zeros(2, dtype=np.complex128)}, tmp_path / "e.nt"),
        "save_cycle": lambda: ser.save(cyclic, tmp_path / "e.nt"),
        "save_int_key": lambda: ser.save({1: 2}, tmp_path / "e.nt"),
        "save_object": lambda: ser.save({"x": object()}, tmp_path / "e.nt"),
        "load_max_bytes_type": lambda: ser.load(tmp_path / "ok.nt", max_array_bytes=-1),
    }
    (tmp_path / "garbage.nt").write_bytes(b"not a zip archive")
    cases["load_garbage"] = lambda: ser.load(tmp_path / "garbage.nt")
    ser.save({"a": np.arange(4, dtype=np.int32)}, tmp_path / "ok.nt")
    cases["load_max_bytes"] = lambda: ser.load(tmp_path / "ok.nt", max_array_bytes=8)
    assert set(cases) == set(expected)
    for name, action in cases.items():
        with pytest.raises(Exception) as caught:
            action()
        assert [type(caught.value).__name__, str(caught.value)] == expected[name], name
    assert not list(tmp_path.glob(".e.nt.*"))   # failed saves leave no staging files


def _rewrite(src: Path, dst: Path, edit_metadata=None, compress=False, extra=None):
    entries = _zip_entries(src)
    metadata = json.loads(entries["metadata.json"][1])
    if edit_metadata is not None:
        edit_metadata(metadata)
    with zipfile.ZipFile(dst, "w") as out:
        kind = zipfile.ZIP_DEFLATED if compress else zipfile.ZIP_STORED
        out.writestr("metadata.json", json.dumps(metadata, separators=(",", ":")), compress_type=kind)
        out.writestr("arrays.npz", entries["arrays.npz"][1], compress_type=zipfile.ZIP_STORED)
        if extra:
            out.writestr(extra, b"")


@pytest.mark.parametrize("case, message", [
    ("compressed", "uncompressed and unencrypted"),
    ("extra_entry", "duplicate, missing or unexpected entries"),
    ("noncanonical_float", "canonical hexadecimal"),
    ("bad_version", "format_version"),
    ("unknown_node", "Unknown archive tree node type"),
    ("unreferenced", "unreferenced arrays"),
    ("nbytes", "nbytes does not match"),
    ("dtype_spelling", "canonical NumPy dtype string"),
])
def test_load_rejects_malformed_archives(tmp_path, case, message):
    good = tmp_path / "good.nt"
    ser.save({"x": nt.tensor(np.ones(4, np.float32)), "y": 0.5, "z": [1]}, good)
    bad = tmp_path / "bad.nt"
    edits = {
        "noncanonical_float": lambda m: m["tree"]["items"][1][1].update(value="0x1.0p-1"),
        "bad_version": lambda m: m.update(format_version=2),
        "unknown_node": lambda m: m["tree"]["items"][2][1].update(type="set"),
        "unreferenced": lambda m: m["tree"]["items"].pop(0),
        "nbytes": lambda m: m["arrays"][0].update(nbytes=15),
        "dtype_spelling": lambda m: m["arrays"][0].update(dtype="float32"),
    }
    _rewrite(good, bad, edit_metadata=edits.get(case), compress=case == "compressed",
             extra="junk" if case == "extra_entry" else None)
    with pytest.raises(ser.SerializationError, match=message):
        ser.load(bad)


def test_pack_unpack_optimizer_keys():
    packed = {"version": 1, "state": {"0": {"step": 1}, "12": {}}}
    assert ck.unpack_optimizer(packed)["state"] == {0: {"step": 1}, 12: {}}
    for key in ("01", "-1", "a", "1.0", "٣"):
        with pytest.raises(ser.SerializationError):
            ck.unpack_optimizer({"state": {key: {}}})
    with pytest.raises(ser.SerializationError):
        ck.unpack_optimizer({"state": []})


def _tiny_named(device="cpu"):
    weight = nt.Parameter(nt.tensor(np.zeros((40, 48), np.float32), device=device))
    bias = nt.Parameter(nt.tensor(np.zeros(40, np.float32), device=device))
    return {"weight": weight, "bias": bias}


def _tiny_optimizer(named, **extra):
    return nt.optim.AdamW([{"params": [named["weight"]], "weight_decay": 0.1},
                           {"params": [named["bias"]], "weight_decay": 0.0}],
                          lr=1e-3, betas=(0.9, 0.95), eps=1e-8, **extra)


def test_reference_checkpoint_loads_on_host():
    """The reference's own checkpoint restores into this package's AdamW and
    GradScaler (host tensors: validation and state only, no compute)."""
    archive = ser.load(GOLDEN / "checkpoint_reference.nt")
    assert archive["optimizer_type"] == ck.optimizer_type(_tiny_optimizer(_tiny_named()))
    named = _tiny_named()
    optimizer = _tiny_optimizer(named)
    scaler = nt.amp.GradScaler(init_scale=1024.0, growth_interval=2)
    info = ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", named, optimizer, scaler=scaler)
    assert (info["step"], info["epoch"], info["config"]) == (3, 0, {"case": "amp-adamw"})
    assert scaler.state_dict() == {"version": 1, "scale": 512.0, "growth_factor": 2.0, "backoff_factor": 0.5,
                                   "growth_interval": 2, "enabled": True, "growth_tracker": 1}
    for index, name in enumerate(("weight", "bias")):
        parameter = named[name]
        assert parameter.numpy().tobytes() == archive["model"][name].numpy().tobytes()
        state = optimizer.state[id(parameter)]
        saved = archive["optimizer"]["state"][str(index)]
        assert state["step"] == saved["step"] == 2
        for buffer in ("exp_avg", "exp_avg_sq"):
            assert state[buffer].numpy().tobytes() == saved[buffer].numpy().tobytes()
    assert [group["weight_decay"] for group in optimizer.param_groups] == [0.1, 0.0]


def test_checkpoint_mismatches_are_rejected_before_anything_changes(tmp_path):
    named = _tiny_named()
    optimizer = _tiny_optimizer(named)
    swapped = nt.optim.AdamW([{"params": [named["bias"]]}, {"params": [named["weight"]]}])
    before = optimizer.state_dict()
    with pytest.raises(ValueError, match="parameter names or group order"):
        ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", named, swapped)
    with pytest.raises(ValueError, match="optimizer type"):
        ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", named, nt.optim.Adam(list(named.values())))
    with pytest.raises(RuntimeError, match="missing"):
        ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", {"weight": named["weight"]}, None)
    assert not named["weight"].numpy().any() and optimizer.state_dict() == before


def test_checkpoint_written_here_has_the_reference_layout(tmp_path):
    named = _tiny_named()
    optimizer = _tiny_optimizer(named)
    ck.load_checkpoint(GOLDEN / "checkpoint_reference.nt", named, optimizer)
    scaler = nt.amp.GradScaler()
    path = tmp_path / "mine.nt"
    ck.save_checkpoint(path, named, optimizer, scaler=scaler, step=3, config={"case": "amp-adamw"})
    mine = ser.load(path)
    reference = ser.load(GOLDEN / "checkpoint_reference.nt")
    assert set(mine) == set(reference)
    for key in ("checkpoint_version", "optimizer_type", "optimizer_parameter_names", "step", "epoch",
                "cumulative_tokens", "config", "scheduler"):
        assert mine[key] == reference[key], key
    assert set(mine["rng"]) == {"default", "generators"}
    assert set(mine["rng"]["default"]) == set(reference["rng"]["default"])
    ours, theirs = mine["optimizer"], reference["optimizer"]
    assert ours["defaults"] == theirs["defaults"] and ours["param_groups"] == theirs["param_groups"]
    assert ours["param_shapes"] == theirs["param_shapes"]
    for key, values in theirs["state"].items():
        assert ours["state"][key]["step"] == values["step"]
        for buffer in ("exp_avg", "exp_avg_sq"):
            assert ours["state"][key][buffer].numpy().tobytes() == values[buffer].numpy().tobytes()


def _same_tree(a, b, where="checkpoint"):
    """Equal archive trees: the same keys, values and types; Tensors and
    arrays with the same dtype, shape and bytes."""
    if isinstance(a, nt.Tensor) or isinstance(b, nt.Tensor):
        assert isinstance(a, nt.Tensor) and isinstance(b, nt.Tensor), where
        assert a.dtype is b.dtype and a.shape == b.shape, where
        assert a.numpy().tobytes() == b.numpy().tobytes(), where
    elif isinstance(a, np.ndarray) or isinstance(b, np.ndarray):
        assert isinstance(a, np.ndarray) and isinstance(b, np.ndarray), where
        assert a.dtype == b.dtype and a.shape == b.shape and a.tobytes() == b.tobytes(), where
    elif isinstance(a, dict):
        assert isinstance(b, dict) and set(a) == set(b), where
        for key in a:
            _same_tree(a[key], b[key], f"{where}[{key!r}]")
    elif isinstance(a, (list, tuple)):
        assert type(a) is type(b) and len(a) == len(b), where
        for index, (x, y) in enumerate(zip(a, b)):
            _same_tree(x, y, f"{where}[{index}]")
    else:
        assert type(a) is type(b) and a == b, (where, a, b)


def test_checkpoint_written_here_restores_in_the_reference(tmp_path):
    """The format's other direction.  checkpoint_package.nt was written by
    this package's save_checkpoint from package_state.build's seeded state,
    and the reference's load_checkpoint (training/checkpoint.py:131-174)
    restored it (tests/golden/make_golden.py, package_checkpoint_case): the
    parameters, moments, step counts, group options, schedule and scaler it
    restored are exactly the saved state, and the writer still writes that
    file's contents for that state."""
    import json
    import sys
    sys.path.insert(0, str(GOLDEN))
    import package_state
    named, optimizer, scheduler, scaler = package_state.build(nt)
    path = tmp_path / "again.nt"
    ck.save_checkpoint(path, named, optimizer, scheduler, scaler=scaler, **package_state.SAVE)
    _same_tree(ser.load(path), ser.load(GOLDEN / "checkpoint_package.nt"))
    restored = np.load(GOLDEN / "package_checkpoint.npz")
    record = json.loads((GOLDEN / "package_checkpoint.json").read_text())
    for name in ("weight", "bias"):
        parameter = named[name]
        state = optimizer.state[id(parameter)]
        assert restored[name].tobytes() == parameter.numpy().tobytes()
        for buffer in ("exp_avg", "exp_avg_sq"):
            assert restored[f"{name}_{buffer}"].tobytes() == state[buffer].numpy().tobytes(), (name, buffer)
        assert int(restored[f"{name}_step"]) == state["step"] == 7
    saved = package_state.SAVE
    assert record["info"] == {"step": saved["step"], "epoch": saved["epoch"], "config": saved["config"],
                              "cumulative_tokens": saved["cumulative_tokens"]}
    assert record["load_result"] == "LoadStateDictResult(missing_keys=[], unexpected_keys=[])"
    groups = [{key: (list(value) if isinstance(value, tuple) else value) for key, value in group.items()
               if key != "params"} for group in optimizer.param_groups]
    assert record["param_groups"] == groups
    assert record["scheduler"] == json.loads(json.dumps(scheduler.state_dict()))
    assert record["last_lr"] == scheduler.get_last_lr()
    assert record["scaler"] == scaler.state_dict() and record["scale"] == scaler.get_scale() == 2048.0
