"""safetensors headers, validated before any payload byte is read.

File layout: an unsigned 64-bit little-endian header length ``N``; ``N`` bytes of
UTF-8 JSON mapping each tensor name to ``{"dtype", "shape", "data_offsets"}`` (plus
an optional ``"__metadata__"`` object of strings); then the payload, which
``data_offsets = [begin, end)`` index relative to its first byte (``8 + N``).

Behaviour follows the reference's ``python/ayaka/model_loader/st.py:30-331``: every
field is untrusted, so the parser refuses (with :class:`CheckpointCorruptError`)
a header length of 0, above 64 MiB or past the end of the file; non-UTF-8 or
non-object JSON; a tensor name given twice (``json`` would silently keep the last);
an unknown dtype token; a shape that is not a list of non-negative ints; offsets
that are not two non-negative ints in order; a byte range whose length disagrees
with ``dtype x shape``; a range past the end of the file; and two tensors claiming
overlapping bytes. Sub-byte tokens (``I4``, ``U4``, ``F4``) are well-formed but have
no unpacking path here: :class:`UnsupportedWeightFormatError`.
"""

from __future__ import annotations

import json
import math
import struct
from dataclasses import dataclass
from pathlib import Path
from typing import Any

from ayaka.exceptions import CheckpointCorruptError, UnsupportedWeightFormatError
from ayaka.types import DType

__all__ = [
    "SafetensorsHeader",
    "TensorEntry",
    "parse_safetensors_header",
    "read_safetensors_header",
]

#: safetensors dtype token -> DType, for every type stored whole bytes per element.
_TOKENS: dict[str, DType] = {d.safetensors_token: d for d in DType if not d.sub_byte}
_SUB_BYTE_TOKENS = frozenset({"I4", "U4", "F4"})
_HEADER_LIMIT = 64 << 20
_U64_MAX = (1 << 64) - 1


@dataclass(frozen=True, slots=True)
class TensorEntry:
    """One tensor of one file: where its bytes are and how to view them."""

    tensor_key: str
    file_uri: str
    dtype: DType
    shape: tuple[int, ...]
    byte_offset: int  # absolute, from the start of the file
    nbytes: int

    @property
    def end_offset(self) -> int:
        return self.byte_offset + self.nbytes

    @property
    def numel(self) -> int:
        return math.prod(self.shape) if self.shape else 1


@dataclass(frozen=True, slots=True)
class SafetensorsHeader:
    """A validated header: entries sorted by file position, metadata as sorted pairs."""

    file_uri: str
    data_start: int
    file_size: int
    entries: tuple[TensorEntry, ...] = ()
    metadata: tuple[tuple[str, str], ...] = ()

    @property
    def tensor_keys(self) -> frozenset[str]:
        return frozenset(e.tensor_key for e in self.entries)

    @property
    def payload_bytes(self) -> int:
        return sum(e.nbytes for e in self.entries)


def _pairs_without_repeats(pairs: list[tuple[str, Any]]) -> dict[str, Any]:
    """``object_pairs_hook`` that keeps repeated keys visible: a repeated key at any
    level is recorded under a marker the caller checks at the top level."""
    out: dict[str, Any] = {}
    repeats: list[str] = []
    for key, value in pairs:
        if key in out:
            repeats.append(key)
        out[key] = value
    if repeats:
        out[_REPEATS] = repeats
    return out


_REPEATS = "\x00repeated-keys"  # cannot occur as a JSON key of a real header


def _dtype_of(token: object, key: str) -> DType:
    if not isinstance(token, str):
        raise CheckpointCorruptError(f"{key}: dtype is {type(token).__name__}, not a string")
    dtype = _TOKENS.get(token)
    if dtype is not None:
        return dtype
    if token in _SUB_BYTE_TOKENS:
        raise UnsupportedWeightFormatError(f"{key}: sub-byte dtype {token} has no unpacking path")
    raise CheckpointCorruptError(f"{key}: unknown safetensors dtype {token!r}; known: {sorted(_TOKENS)}")


def _is_int(v: object) -> bool:
    return isinstance(v, int) and not isinstance(v, bool)


def _shape_of(raw: object, key: str) -> tuple[int, ...]:
    if not isinstance(raw, list) or not all(_is_int(d) for d in raw):
        raise CheckpointCorruptError(f"{key}: shape must be a list of ints, got {raw!r}")
    shape = tuple(int(d) for d in raw)
    if any(d < 0 for d in shape):
        raise CheckpointCorruptError(f"{key}: negative dim in shape {shape}")
    if (math.prod(shape) if shape else 1) > _U64_MAX:
        raise CheckpointCorruptError(f"{key}: shape {shape} overflows a 64-bit element count")
    return shape


def _range_of(raw: object, key: str) -> tuple[int, int]:
    if not isinstance(raw, list) or len(raw) != 2:
        raise CheckpointCorruptError(f"{key}: data_offsets must be [begin, end], got {raw!r}")
    begin, end = raw
    if not (_is_int(begin) and _is_int(end)):
        raise CheckpointCorruptError(f"{key}: data_offsets must be integers, got {raw!r}")
    if begin < 0 or end < 0:
        raise CheckpointCorruptError(f"{key}: negative data_offset in {raw!r}")
    if begin > end:
        raise CheckpointCorruptError(f"{key}: data_offsets [{begin}, {end}) run backwards")
    if end > _U64_MAX:
        raise CheckpointCorruptError(f"{key}: data_offset {end} overflows u64")
    return int(begin), int(end)


def parse_safetensors_header(raw_header: bytes, *, file_uri: str, data_start: int, file_size: int) -> SafetensorsHeader:
    """Validate the JSON header of ``file_uri`` (whose payload starts at ``data_start``
    and which is ``file_size`` bytes long) and return its entries."""
    try:
        text = raw_header.decode("utf-8")
    except UnicodeDecodeError as exc:
        raise CheckpointCorruptError(f"{file_uri}: header is not valid UTF-8") from exc
    try:
        header = json.loads(text, object_pairs_hook=_pairs_without_repeats)
    except json.JSONDecodeError as exc:
        raise CheckpointCorruptError(f"{file_uri}: header is not valid JSON: {exc}") from exc
    if not isinstance(header, dict):
        raise CheckpointCorruptError(f"{file_uri}: header is {type(header).__name__}, not an object")
    repeated = header.pop(_REPEATS, None)
    if repeated:
        raise CheckpointCorruptError(
            f"{file_uri}: duplicate tensor keys in header: {sorted(set(repeated))} (a JSON parser keeps only the last)")

    metadata: tuple[tuple[str, str], ...] = ()
    meta = header.pop("__metadata__", None)
    if isinstance(meta, dict):
        meta.pop(_REPEATS, None)
        metadata = tuple(sorted((str(k), str(v)) for k, v in meta.items()))

    entries = []
    for key, spec in header.items():
        if not isinstance(spec, dict):
            raise CheckpointCorruptError(f"{file_uri}: entry {key!r} is not an object")
        dtype = _dtype_of(spec.get("dtype"), key)
        shape = _shape_of(spec.get("shape"), key)
        begin, end = _range_of(spec.get("data_offsets"), key)
        need = dtype.nbytes(math.prod(shape) if shape else 1)
        if end - begin != need:
            raise CheckpointCorruptError(
                f"{file_uri}: entry {key!r} has {end - begin} bytes in data_offsets, "
                f"but shape {shape} and dtype {dtype.label} require {need}")
        offset = data_start + begin
        if offset + need > file_size:
            raise CheckpointCorruptError(
                f"{file_uri}: entry {key!r} ends at {offset + need}, beyond the file size of {file_size}")
        entries.append(TensorEntry(key, file_uri, dtype, shape, offset, need))
    entries.sort(key=lambda e: (e.byte_offset, e.end_offset))
    for before, after in zip(entries, entries[1:]):
        if after.byte_offset < before.end_offset:
            raise CheckpointCorruptError(
                f"{file_uri}: {before.tensor_key} [{before.byte_offset}:{before.end_offset}) overlaps "
                f"{after.tensor_key} [{after.byte_offset}:{after.end_offset})")
    return SafetensorsHeader(file_uri, data_start, file_size, tuple(entries), metadata)


def read_safetensors_header(path: str | Path) -> SafetensorsHeader:
    """Read and validate the header of one file (reads its first ``8 + N`` bytes only)."""
    p = Path(path)
    try:
        size = p.stat().st_size
    except OSError as exc:
        raise CheckpointCorruptError(f"{p}: cannot stat: {exc}") from exc
    if size < 8:
        raise CheckpointCorruptError(f"{p}: {size} B is too small to hold a header length")
    try:
        with p.open("rb") as fh:
            (length,) = struct.unpack("<Q", fh.read(8))
            if length == 0:
                raise CheckpointCorruptError(f"{p}: header length is 0")
            if length > _HEADER_LIMIT:
                raise CheckpointCorruptError(
                    f"{p}: header claims {length} B (limit {_HEADER_LIMIT}); refusing to allocate on it")
            if 8 + length > size:
                raise CheckpointCorruptError(f"{p}: header claims {length} B but the file is {size} B")
            raw = fh.read(length)
    except OSError as exc:
        raise CheckpointCorruptError(f"{p}: cannot read header: {exc}") from exc
    if len(raw) != length:
        raise CheckpointCorruptError(f"{p}: header truncated, read {len(raw)} of {length} B")
    return parse_safetensors_header(raw, file_uri=str(p), data_start=8 + length, file_size=size)
