"""Shared validation for operator-owned configuration dataclasses.

Same contract as spark_mlx_llm/ops/base.py:13-53: keyword-only fields whose
metadata["choices"] drive both validation and CLI choices.
"""

from collections.abc import Mapping
from dataclasses import dataclass, fields

__all__ = ["OperatorConfig"]


@dataclass(kw_only=True)
class OperatorConfig:
    """Keyword-only fields can also be inherited by a model's flat config."""

    def __post_init__(self):
        self.validate()

    @classmethod
    def from_dict(cls, values: Mapping):
        """Extract this operator's fields from a checkpoint/model config."""
        return cls(**{f.name: values[f.name] for f in fields(cls) if f.name in values})

    @classmethod
    def choices(cls, name: str) -> tuple:
        item = next(f for f in fields(cls) if f.name == name)
        return item.metadata["choices"]

    @classmethod
    def validate_values(cls, values: Mapping):
        """Validate supplied fields without filling missing values."""
        for item in fields(cls):
            if item.name not in values:
                continue
            value = values[item.name]
            if type(item.default) is bool and type(value) is not bool:
                raise ValueError(f"{item.name} must be a boolean, got {value!r}")
            choices = item.metadata.get("choices")
            if choices is not None and value not in choices:
                raise ValueError(f"{item.name} must be one of {choices}, got {value!r}")

    def validate(self):
        self.validate_values({f.name: getattr(self, f.name) for f in fields(self)})
