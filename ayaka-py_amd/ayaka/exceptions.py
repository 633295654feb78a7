"""Checkpoint-loading errors (the loader subset of the reference's
``ayaka/exceptions.py:12-60``: same class names and hierarchy)."""

from __future__ import annotations


class ModelLoadError(RuntimeError):
    """Loading a checkpoint failed; the model is not usable."""


class CheckpointCorruptError(ModelLoadError):
    """A checkpoint file is malformed or inconsistent with itself (bad header, byte
    ranges that overlap or run past the file, a dtype/shape that disagrees with the
    byte count, a payload that cannot be read in full)."""


class UnsupportedWeightFormatError(ModelLoadError):
    """A well-formed checkpoint stores a format this package has no path for
    (sub-byte dtypes, a tensor whose dtype the target parameter cannot take)."""


__all__ = ["CheckpointCorruptError", "ModelLoadError", "UnsupportedWeightFormatError"]
