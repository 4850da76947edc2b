"""Config dataclasses owned by the operators (linear, SDPA, ...).

The contract callers rely on (spark_mlx_llm/ops/base.py:13-53): every field is
keyword-only, a field may list its legal values in ``metadata["choices"]``,
boolean fields accept only real bools, and a model's flat config can be
filtered down to one operator's fields. The messages of the ValueErrors are
part of that contract, since configuration front ends surface them verbatim.
"""

from collections.abc import Mapping
from dataclasses import Field, dataclass, fields

__all__ = ["OperatorConfig"]


def _check_field(spec: Field, value) -> None:
    """Raise ValueError when ``value`` is not legal for the field ``spec``."""
    if isinstance(spec.default, bool) and type(value) is not bool:
        raise ValueError(f"{spec.name} must be a boolean, got {value!r}")
    legal = spec.metadata.get("choices")
    if legal is not None and value not in legal:
        raise ValueError(f"{spec.name} must be one of {legal}, got {value!r}")


@dataclass(kw_only=True)
class OperatorConfig:
    """Base of the operator configs; subclasses declare keyword-only fields,
    which a model config that inherits them can also carry."""

    def __post_init__(self):
        self.validate()

    @classmethod
    def _field(cls, name: str) -> Field:
        for spec in fields(cls):
            if spec.name == name:
                return spec
        raise KeyError(name)

    @classmethod
    def from_dict(cls, values: Mapping):
        """Build the config from the subset of ``values`` that names its fields
        (a checkpoint or model config may hold many other keys)."""
        own = {spec.name for spec in fields(cls)}
        return cls(**{key: values[key] for key in own if key in values})

    @classmethod
    def choices(cls, name: str) -> tuple:
        """Legal values of field ``name``, shared by validation and CLI flags."""
        return cls._field(name).metadata["choices"]

    @classmethod
    def validate_values(cls, values: Mapping):
        """Check only the fields present in ``values``; absent fields are left
        to their defaults, so a partial checkpoint config validates."""
        for spec in fields(cls):
            if spec.name in values:
                _check_field(spec, values[spec.name])

    def validate(self):
        self.validate_values(vars(self))
