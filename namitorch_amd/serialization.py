"""NamiTorch archive format (``.nt``): reader and writer.

Byte-compatible with ``namitorch/serialization.py:14-257`` so that optimizer
and GradScaler state written here loads in the reference and vice versa:

* an uncompressed zip holding ``metadata.json`` and ``arrays.npz`` (itself an
  uncompressed zip of NPY 1.0 files ``a0.npy``, ``a1.npy`` ... in order of
  first appearance);
* ``metadata.json`` = ``{"format_version": 1, "tree": node, "arrays":
  [{"id", "dtype", "shape", "nbytes"}]}``, compact ASCII JSON, at most 16 MiB;
* tree nodes ``none``, ``bool``/``int``/``str`` (value), ``float`` (value as
  ``float.hex()``), ``list``/``tuple`` (items), ``dict`` (items as
  ``[key, node]`` pairs, string keys), ``tensor`` (id, requires_grad) and
  ``ndarray`` (id);
* array dtypes limited to bool, signed/unsigned integers of 1/2/4/8 bytes and
  float16/32/64, written with their canonical NumPy dtype string.

bfloat16 has no archive dtype (the whitelist above).  A bfloat16 Tensor is
written as its exact float32 widening (``<f4``); the reference reads it as
float32 and an optimizer loading it narrows it back to its state dtype,
which is exact because every value came from bfloat16.

Device tensors are copied to the host when written; tensors read back are
host (CPU) Tensors, as in the reference, and the optimizer moves them to the
parameter's device in ``load_state_dict``.  The writer stages the archive in
a temporary file next to the destination, fsyncs it and renames it over the
destination, so a crash never leaves a torn archive.
"""

from __future__ import annotations

import json
import math
import os
import tempfile
import zipfile
from pathlib import Path

import numpy as np

from .dtype import from_numpy_dtype
from .tensor import Tensor

FORMAT_VERSION = 1
MAX_DEPTH = 128
MAX_METADATA_BYTES = 16 * 1024 * 1024
_ARRAY_KINDS = {"b": (1,), "i": (1, 2, 4, 8), "u": (1, 2, 4, 8), "f": (2, 4, 8)}
_SCALAR_TYPES = {"bool": bool, "int": int, "str": str, "float": str}


class SerializationError(ValueError):
    """An archive (or an object to archive) violates the format."""

    __slots__ = ()


def archive_dtype(text) -> np.dtype:
    """The NumPy dtype for an archive dtype string; rejects anything outside
    the whitelist or in a non-canonical spelling (serialization.py:23-33)."""
    if not isinstance(text, str):
        raise SerializationError("Array dtype must be a string.")
    dtype = np.dtype(text)
    if (dtype.kind not in _ARRAY_KINDS or dtype.itemsize not in _ARRAY_KINDS[dtype.kind]
            or dtype.fields is not None or dtype.subdtype is not None):
        raise SerializationError(f"Unsupported archive array dtype {text!r}; object and complex arrays are forbidden.")
    if dtype.str != text:
        raise SerializationError("Array dtype must use its canonical NumPy dtype string.")
    return dtype


# ---- writing ------------------------------------------------------------------------------
class _Writer:
    """Turns an object tree into metadata nodes plus the list of arrays to store."""

    def __init__(self):
        self.arrays: list[tuple[str, np.ndarray]] = []
        self._open: set[int] = set()

    def _add_array(self, array: np.ndarray) -> str:
        if array.dtype.metadata is not None:
            raise SerializationError("Array dtypes with custom metadata are unsupported.")
        archive_dtype(array.dtype.str)
        identifier = f"a{len(self.arrays)}"
        self.arrays.append((identifier, array))
        return identifier

    def node(self, value, depth: int = 0) -> dict:
        if depth > MAX_DEPTH:
            raise SerializationError(f"Archive nesting exceeds {MAX_DEPTH} levels.")
        if value is None:
            return {"type": "none"}
        kind = type(value)
        if kind is bool or kind is int or kind is str:
            return {"type": kind.__name__, "value": value}
        if kind is float:
            return {"type": "float", "value": value.hex()}
        if isinstance(value, Tensor):
            # Device tensors come to the host here; bfloat16 widens exactly to float32.
            node = {"type": "tensor", "id": self._add_array(value.numpy())}
            node["requires_grad"] = value.requires_grad
            return node
        if isinstance(value, np.ndarray):
            return {"type": "ndarray", "id": self._add_array(value)}
        if not isinstance(value, (list, tuple, dict)):
            raise TypeError(f"Cannot serialize {type(value).__name__}; only primitive containers, Tensor and ndarray are supported.")
        identity = id(value)
        if identity in self._open:
            raise SerializationError("Cannot serialize cyclic containers.")
        self._open.add(identity)
        try:
            if isinstance(value, dict):
                if any(type(key) is not str for key in value):
                    raise TypeError("Archive dictionaries require string keys.")
                return {"type": "dict", "items": [[key, self.node(item, depth + 1)] for key, item in value.items()]}
            return {"type": "tuple" if isinstance(value, tuple) else "list",
                    "items": [self.node(item, depth + 1) for item in value]}
        finally:
            self._open.discard(identity)


def save(obj, path) -> None:
    """Write `obj` (nested None/bool/int/float/str/list/tuple/dict with
    string keys, Tensor and ndarray leaves) as an archive at `path`."""
    writer = _Writer()
    tree = writer.node(obj)
    metadata = {
        "format_version": FORMAT_VERSION,
        "tree": tree,
        "arrays": [{"id": identifier, "dtype": array.dtype.str, "shape": list(array.shape), "nbytes": array.nbytes}
                   for identifier, array in writer.arrays],
    }
    encoded = json.dumps(metadata, ensure_ascii=True, allow_nan=False, separators=(",", ":")).encode("utf-8")
    if len(encoded) > MAX_METADATA_BYTES:
        raise SerializationError("Archive metadata exceeds the 16 MiB format limit.")
    destination = Path(path)
    staged = None
    try:
        with tempfile.NamedTemporaryFile(mode="w+b", dir=destination.parent, prefix=f".{destination.name}.",
                                         suffix=".tmp", delete=False) as stream:
            staged = Path(stream.name)
            with zipfile.ZipFile(stream, "w", compression=zipfile.ZIP_STORED, allowZip64=True) as outer:
                outer.writestr("metadata.json", encoded)
                with outer.open("arrays.npz", "w", force_zip64=True) as payload:
                    with zipfile.ZipFile(payload, "w", compression=zipfile.ZIP_STORED, allowZip64=True) as inner:
                        for identifier, array in writer.arrays:
                            with inner.open(f"{identifier}.npy", "w", force_zip64=True) as entry:
                                np.lib.format.write_array(entry, np.ascontiguousarray(array), version=(1, 0),
                                                          allow_pickle=False)
            stream.flush()
            os.fsync(stream.fileno())
        os.replace(staged, destination)
        staged = None
    finally:
        if staged is not None:
            staged.unlink(missing_ok=True)


# ---- reading ------------------------------------------------------------------------------
def _unique_pairs(pairs):
    result = {}
    for key, value in pairs:
        if key in result:
            raise SerializationError(f"Duplicate JSON field {key!r}.")
        result[key] = value
    return result


def _reject_constant(value):
    raise SerializationError(f"Nonstandard JSON constant {value!r} is forbidden.")


def _expect_fields(value, expected: set, what: str) -> None:
    if type(value) is not dict or set(value) != expected:
        raise SerializationError(f"Invalid {what} fields; expected {sorted(expected)}.")


def _check_entries(archive: zipfile.ZipFile, expected: set) -> None:
    entries = archive.infolist()
    names = [entry.filename for entry in entries]
    if len(names) != len(set(names)) or set(names) != expected:
        raise SerializationError("Archive contains duplicate, missing or unexpected entries.")
    for entry in entries:
        if entry.compress_type != zipfile.ZIP_STORED or entry.flag_bits & 1:
            raise SerializationError("Archive entries must be uncompressed and unencrypted.")


def _array_table(records, max_array_bytes) -> dict:
    if type(records) is not list:
        raise SerializationError("Array records must be a list.")
    limit = np.iinfo(np.intp).max
    table = {}
    total = 0
    for position, record in enumerate(records):
        _expect_fields(record, {"id", "dtype", "shape", "nbytes"}, "array record")
        if record["id"] != f"a{position}":
            raise SerializationError("Array IDs must be unique consecutive identifiers.")
        dtype = archive_dtype(record["dtype"])
        shape = record["shape"]
        if type(shape) is not list or any(type(size) is not int or not 0 <= size <= limit for size in shape):
            raise SerializationError("Array shape must contain nonnegative platform-sized integers.")
        nbytes = math.prod(shape) * dtype.itemsize
        if type(record["nbytes"]) is not int or record["nbytes"] != nbytes or nbytes > limit:
            raise SerializationError("Array nbytes does not match its shape and dtype or exceeds the platform limit.")
        total += nbytes
        if max_array_bytes is not None and total > max_array_bytes:
            raise SerializationError("Archive arrays exceed max_array_bytes.")
        table[record["id"]] = (dtype, tuple(shape), nbytes)
    return table


class _Reader:
    def __init__(self, inner: zipfile.ZipFile, table: dict):
        self.inner = inner
        self.table = table
        self.used: set[str] = set()

    def _array(self, identifier: str) -> np.ndarray:
        dtype, shape, nbytes = self.table[identifier]
        entry = self.inner.getinfo(f"{identifier}.npy")
        with self.inner.open(entry) as stream:
            if np.lib.format.read_magic(stream) != (1, 0):
                raise SerializationError("Only NPY version 1.0 is supported by this archive format.")
            header_shape, fortran, header_dtype = np.lib.format.read_array_header_1_0(stream)
            if header_shape != shape or header_dtype != dtype or fortran:
                raise SerializationError(f"NPY header disagrees with metadata for {identifier!r}.")
            if entry.file_size - stream.tell() != nbytes:
                raise SerializationError(f"Invalid array payload size for {identifier!r}.")
            stream.seek(0)
            return np.lib.format.read_array(stream, allow_pickle=False)

    def value(self, node, depth: int = 0):
        if depth > MAX_DEPTH:
            raise SerializationError(f"Archive nesting exceeds {MAX_DEPTH} levels.")
        if type(node) is not dict or type(node.get("type")) is not str:
            raise SerializationError("Every tree node must have a string type tag.")
        kind = node["type"]
        if kind == "none":
            _expect_fields(node, {"type"}, "none node")
            return None
        if kind in _SCALAR_TYPES:
            _expect_fields(node, {"type", "value"}, "scalar node")
            raw = node["value"]
            if type(raw) is not _SCALAR_TYPES[kind]:
                raise SerializationError(f"Invalid scalar value for type {kind!r}.")
            if kind != "float":
                return raw
            number = float.fromhex(raw)
            if number.hex() != raw:
                raise SerializationError("Float values must use canonical hexadecimal strings.")
            return number
        if kind in ("list", "tuple", "dict"):
            _expect_fields(node, {"type", "items"}, "container node")
            items = node["items"]
            if type(items) is not list:
                raise SerializationError("Container items must be a list.")
            if kind == "dict":
                result = {}
                for pair in items:
                    if type(pair) is not list or len(pair) != 2 or type(pair[0]) is not str or pair[0] in result:
                        raise SerializationError("Dictionary entries must have unique string keys.")
                    result[pair[0]] = self.value(pair[1], depth + 1)
                return result
            values = [self.value(item, depth + 1) for item in items]
            return tuple(values) if kind == "tuple" else values
        if kind in ("tensor", "ndarray"):
            _expect_fields(node, {"type", "id", "requires_grad"} if kind == "tensor" else {"type", "id"}, "array node")
            identifier = node["id"]
            if type(identifier) is not str or identifier not in self.table or identifier in self.used:
                raise SerializationError("Array reference must name a unique existing array ID.")
            self.used.add(identifier)
            if kind == "ndarray":
                return self._array(identifier)
            dtype = from_numpy_dtype(self.table[identifier][0])
            requires_grad = node["requires_grad"]
            if type(requires_grad) is not bool or (requires_grad and not dtype.can_require_grad):
                raise SerializationError("Invalid requires_grad flag for serialized Tensor dtype.")
            return Tensor(self._array(identifier), dtype=dtype, requires_grad=requires_grad)
        raise SerializationError(f"Unknown archive tree node type {kind!r}.")


def load(path, *, max_array_bytes=None):
    """Read an archive written by `save` (or by the reference); tensors come
    back as host Tensors.  `max_array_bytes` bounds the total array payload."""
    if max_array_bytes is not None and (type(max_array_bytes) is not int or max_array_bytes < 0):
        raise TypeError("max_array_bytes must be a nonnegative Python integer or None.")
    try:
        with zipfile.ZipFile(path, "r") as outer:
            _check_entries(outer, {"metadata.json", "arrays.npz"})
            if outer.getinfo("metadata.json").file_size > MAX_METADATA_BYTES:
                raise SerializationError("Archive metadata exceeds the 16 MiB format limit.")
            metadata = json.loads(outer.read("metadata.json"), object_pairs_hook=_unique_pairs,
                                  parse_constant=_reject_constant)
            _expect_fields(metadata, {"format_version", "tree", "arrays"}, "metadata")
            if type(metadata["format_version"]) is not int or metadata["format_version"] != FORMAT_VERSION:
                raise SerializationError("Unsupported archive format_version.")
            table = _array_table(metadata["arrays"], max_array_bytes)
            with outer.open("arrays.npz") as payload, zipfile.ZipFile(payload, "r") as inner:
                _check_entries(inner, {f"{identifier}.npy" for identifier in table})
                reader = _Reader(inner, table)
                result = reader.value(metadata["tree"])
                if reader.used != set(table):
                    raise SerializationError("Archive contains unreferenced arrays.")
                return result
    except SerializationError:
        raise
    except (zipfile.BadZipFile, ValueError, TypeError, KeyError, EOFError, OverflowError, RecursionError) as error:
        raise SerializationError(f"Invalid NamiTorch archive: {error}") from error


__all__ = ["FORMAT_VERSION", "SerializationError", "archive_dtype", "save", "load"]
