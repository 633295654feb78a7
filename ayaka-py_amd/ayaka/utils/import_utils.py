"""Capability errors (semantics of the reference's ``ayaka/utils/import_utils.py:19-26``)."""

from __future__ import annotations


class CapabilityError(ImportError):
    """A kernel, library or device capability the caller asked for is unavailable."""

    def __init__(self, capability: str, *, detail: str, remedy: str) -> None:
        self.capability = capability
        self.detail = detail
        self.remedy = remedy
        super().__init__(f"capability {capability!r} unavailable: {detail}. Remedy: {remedy}")
