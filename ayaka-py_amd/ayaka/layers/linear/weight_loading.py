"""Weight-loader helpers (reference ``ayaka/layers/linear/weight_loading.py:15-21``)."""

from __future__ import annotations

from typing import Any

from torch.nn import Parameter


class WeightLoadError(ValueError):
    """A checkpoint tensor does not fit the parameter it is loaded into."""


def set_weight_attrs(parameter: Parameter, attrs: dict[str, Any]) -> None:
    """Attach loader metadata (e.g. ``weight_loader``) to a parameter."""
    for name, value in attrs.items():
        setattr(parameter, name, value)
