"""Checkpoint tensors from safetensors files into host memory or HBM.

:class:`CheckpointReader` indexes a checkpoint (a directory with
``model.safetensors.index.json``, one ``model.safetensors``, any ``*.safetensors``
files, or a single file; reference ``model_loader/source.py:18-251``), validating
every header first (``ayaka.model_loader.st``) and refusing a tensor name that two
shards both claim.

Payloads are read with ``preadv`` straight into the destination's bytes. For a GPU
destination they go through two pinned staging buffers: the host reads chunk
``i + 1`` from disk while chunk ``i`` is copied to HBM on the current stream, so a
multi-GB FP8 weight never exists as a full host copy. :meth:`read_into` fills an
existing tensor (a row slice of a packed ``[N, K]`` weight, say) with no
intermediate device tensor. A short read is a :class:`CheckpointCorruptError`.
"""

from __future__ import annotations

import json
import os
from collections.abc import Iterable, Mapping
from pathlib import Path
from typing import Any

import torch

from ayaka.exceptions import CheckpointCorruptError, UnsupportedWeightFormatError
from ayaka.model_loader.st import SafetensorsHeader, TensorEntry, read_safetensors_header

__all__ = ["CheckpointReader", "INDEX_FILENAME", "SINGLE_FILENAME", "checkpoint_files"]

INDEX_FILENAME = "model.safetensors.index.json"
SINGLE_FILENAME = "model.safetensors"
CONFIG_FILENAME = "config.json"
_STAGING_BYTES = 64 << 20


def checkpoint_files(path: str | os.PathLike[str]) -> tuple[Path, ...]:
    """The safetensors files of a checkpoint: the shards its index names, else
    ``model.safetensors``, else every ``*.safetensors`` in the directory; a file path
    is itself."""
    root = Path(path)
    if root.is_file():
        if root.suffix != ".safetensors":
            raise CheckpointCorruptError(f"{root}: not a .safetensors file")
        return (root,)
    if not root.is_dir():
        raise CheckpointCorruptError(f"{root}: no such checkpoint file or directory")
    index = root / INDEX_FILENAME
    if index.is_file():
        try:
            weight_map = json.loads(index.read_text())["weight_map"]
        except (OSError, ValueError, KeyError, TypeError) as exc:
            raise CheckpointCorruptError(f"{index}: unreadable shard index: {exc}") from exc
        if not isinstance(weight_map, dict) or not all(isinstance(v, str) for v in weight_map.values()):
            raise CheckpointCorruptError(f"{index}: weight_map must map tensor names to file names")
        names = sorted(set(weight_map.values()))
        for name in names:
            if Path(name).name != name:
                raise CheckpointCorruptError(f"{index}: shard {name!r} is not a file in the checkpoint directory")
            if not (root / name).is_file():
                raise CheckpointCorruptError(f"{index}: shard {name!r} is missing")
        return tuple(root / n for n in names)
    if (root / SINGLE_FILENAME).is_file():
        return (root / SINGLE_FILENAME,)
    shards = tuple(sorted(root.glob("*.safetensors")))
    if not shards:
        raise CheckpointCorruptError(
            f"no safetensors checkpoint in {root}: expected {INDEX_FILENAME}, {SINGLE_FILENAME} or *.safetensors")
    return shards


def _read_exact(fd: int, view: memoryview, offset: int, label: str) -> None:
    done = 0
    while done < len(view):
        got = os.preadv(fd, [view[done:]], offset + done)
        if got <= 0:
            raise CheckpointCorruptError(f"{label}: payload truncated at byte {offset + done}")
        done += got


class CheckpointReader:
    """Validated index over a checkpoint's tensors, with host and HBM readers.

    Use as a context manager (or call :meth:`close`) to release file descriptors and
    the pinned staging buffers.
    """

    def __init__(self, path: str | os.PathLike[str], *, staging_bytes: int = _STAGING_BYTES) -> None:
        self.path = Path(path)
        self.headers: tuple[SafetensorsHeader, ...] = tuple(read_safetensors_header(f) for f in checkpoint_files(path))
        entries: dict[str, TensorEntry] = {}
        for header in self.headers:
            for entry in header.entries:
                other = entries.get(entry.tensor_key)
                if other is not None:
                    raise CheckpointCorruptError(
                        f"tensor {entry.tensor_key!r} is stored in both {other.file_uri} and {entry.file_uri}")
                entries[entry.tensor_key] = entry
        self._entries = entries
        self._fds: dict[str, int] = {}
        self._staging_bytes = max(1 << 20, int(staging_bytes))
        self._staging: list[torch.Tensor] = []
        self._events: list[Any] = []

    # ------------------------------------------------------------------ index
    def keys(self) -> Iterable[str]:
        return self._entries.keys()

    def __contains__(self, key: object) -> bool:
        return key in self._entries

    def entry(self, key: str) -> TensorEntry:
        try:
            return self._entries[key]
        except KeyError:
            raise KeyError(f"checkpoint {self.path} has no tensor {key!r}") from None

    @property
    def config(self) -> Mapping[str, Any]:
        """``config.json`` beside the checkpoint files, or ``{}`` if there is none."""
        root = self.path if self.path.is_dir() else self.path.parent
        cfg = root / CONFIG_FILENAME
        if not cfg.is_file():
            return {}
        try:
            value = json.loads(cfg.read_text())
        except (OSError, ValueError) as exc:
            raise CheckpointCorruptError(f"{cfg}: unreadable config: {exc}") from exc
        if not isinstance(value, dict):
            raise CheckpointCorruptError(f"{cfg}: config is not a JSON object")
        return value

    # ------------------------------------------------------------------ reads
    def read(self, key: str, device: torch.device | str | None = None) -> torch.Tensor:
        """A new tensor holding ``key`` (its checkpoint dtype and shape) on ``device``."""
        entry = self.entry(key)
        if entry.dtype.torch_name is None:
            raise UnsupportedWeightFormatError(f"{key}: {entry.dtype.label} has no torch dtype")
        out = torch.empty(entry.shape, dtype=entry.dtype.torch_dtype, device=device or "cpu")
        self.read_into(key, out)
        return out

    def read_into(self, key: str, destination: torch.Tensor) -> None:
        """Fill ``destination`` (contiguous, exactly the tensor's byte size; its dtype
        may differ only as a same-size reinterpretation) with ``key``'s bytes."""
        entry = self.entry(key)
        if not destination.is_contiguous():
            raise ValueError(f"{key}: destination must be contiguous")
        size = destination.numel() * destination.element_size()
        if size != entry.nbytes:
            raise ValueError(f"{key}: destination holds {size} B, the checkpoint tensor {entry.nbytes} B")
        if entry.nbytes == 0:
            return
        raw = destination.reshape(-1).view(torch.uint8)
        fd = self._fd(entry.file_uri)
        if raw.device.type == "cpu":
            _read_exact(fd, memoryview(raw.numpy()), entry.byte_offset, key)
            return
        with torch.cuda.device(raw.device):  # the copies and their events on that device's stream
            self._stream_to_device(fd, entry, raw)

    def _fd(self, file_uri: str) -> int:
        fd = self._fds.get(file_uri)
        if fd is None:
            try:
                fd = os.open(file_uri, os.O_RDONLY)
            except OSError as exc:
                raise CheckpointCorruptError(f"{file_uri}: cannot open: {exc}") from exc
            self._fds[file_uri] = fd
        return fd

    def _stream_to_device(self, fd: int, entry: TensorEntry, raw: torch.Tensor) -> None:
        if not self._staging:
            self._staging = [torch.empty(self._staging_bytes, dtype=torch.uint8, pin_memory=True) for _ in range(2)]
            self._events = [None, None]
        chunk = self._staging_bytes
        for i, start in enumerate(range(0, entry.nbytes, chunk)):
            slot = i % 2
            if self._events[slot] is not None:
                self._events[slot].synchronize()  # the copy that last used this buffer is done
            n = min(chunk, entry.nbytes - start)
            buf = self._staging[slot][:n]
            _read_exact(fd, memoryview(buf.numpy()), entry.byte_offset + start, entry.tensor_key)
            raw[start:start + n].copy_(buf, non_blocking=True)
            event = torch.cuda.Event()
            event.record()
            self._events[slot] = event

    def close(self) -> None:
        for event in self._events:
            if event is not None:
                event.synchronize()
        self._events = []
        self._staging = []
        for fd in self._fds.values():
            os.close(fd)
        self._fds = {}

    def __enter__(self) -> "CheckpointReader":
        return self

    def __exit__(self, *exc: object) -> None:
        self.close()
