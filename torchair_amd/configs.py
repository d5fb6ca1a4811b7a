"""CompilerConfig: the option tree of python/torchair/configs/compiler_config.py:24-60.

Options are typed values; assigning to a leaf validates it (e.g. ``config.mode = "reduce-overhead"``).
Only the options that change this backend's behaviour are modelled; GE-only option groups
are accepted as free-form namespaces and reported once as having no effect.
"""
from __future__ import annotations

import warnings
from typing import Any, Iterator, Tuple

INT64_MAX = 2 ** 63 - 1


class OptionValue:
    """A typed option with an optional list of allowed values."""

    def __init__(self, default, optional=None):
        self._default = default
        self._optional = optional
        self._value = default

    def __bool__(self):
        return bool(self._value)

    @property
    def default(self):
        return self._default

    @property
    def optional(self):
        return self._optional

    @property
    def value(self):
        return self._value

    @value.setter
    def value(self, v):
        if isinstance(self._optional, (list, tuple)) and v not in self._optional:
            raise ValueError(f"Value {v!r} (type: {type(v)}) not in optional list {self._optional!r}.")
        self._value = v


class IntRangeValue(OptionValue):
    def __init__(self, default, lo, hi):
        super().__init__(default)
        self._lo, self._hi = lo, hi

    @property
    def value(self):
        return self._value

    @value.setter
    def value(self, v):
        if not isinstance(v, int) or isinstance(v, bool):
            raise ValueError(f"Please set integer type, but got {type(v)}")
        if v < self._lo or v > self._hi:
            raise ValueError(f"Please set value in [{self._lo}, {self._hi}], {v} is out of range.")
        self._value = v


class NpuBaseConfig:
    """Attribute assignment on a leaf option goes through the option's validator."""

    def __setattr__(self, name, value):
        cur = self.__dict__.get(name)
        if isinstance(cur, OptionValue) and not isinstance(value, OptionValue):
            cur.value = value
            return
        object.__setattr__(self, name, value)

    def leaves(self, prefix: str = "") -> Iterator[Tuple[str, Any]]:
        for k, v in self.__dict__.items():
            if k.startswith("_"):
                continue
            path = f"{prefix}{k}"
            if isinstance(v, OptionValue):
                yield path, v.value
            elif isinstance(v, NpuBaseConfig):
                yield from v.leaves(path + ".")


class _AclGraphDebugConfig(NpuBaseConfig):
    def __init__(self):
        self.enable_output_clone = OptionValue(False, [True, False])
        self.static_capture_size_limit = IntRangeValue(64, 1, INT64_MAX)
        self.clone_input = OptionValue(True, [True, False])


class _DebugConfig(NpuBaseConfig):
    def __init__(self):
        self.run_eagerly = OptionValue(False, [True, False])
        self.aclgraph = _AclGraphDebugConfig()


class _AclGraphConfig(NpuBaseConfig):
    def __init__(self):
        self.use_custom_pool = None


class _ExperimentalConfig(NpuBaseConfig):
    def __init__(self):
        self.frozen_parameter = OptionValue(False, [True, False])
        # FX fusion passes before lowering (python/torchair/configs/experimental_config.py:29)
        self.pattern_fusion_pass = OptionValue(True, [True, False])


class _Opaque(NpuBaseConfig):
    """GE-only option group: values are stored and ignored."""

    def __init__(self, name):
        object.__setattr__(self, "_name", name)


class CompilerConfig(NpuBaseConfig):
    """Set CompilerConfig configuration."""

    def __init__(self):
        self.debug = _DebugConfig()
        self.aclgraph_config = _AclGraphConfig()
        self.experimental_config = _ExperimentalConfig()
        self.ge_config = _Opaque("ge_config")
        self.fusion_config = _Opaque("fusion_config")
        self.dump_config = _Opaque("dump_config")
        self.export = _Opaque("export")
        self.inference_config = _Opaque("inference_config")
        self.mode = OptionValue("max-autotune", ["max-autotune", "reduce-overhead", "npugraph_ex"])

    def __eq__(self, other):
        return isinstance(other, CompilerConfig) and dict(self.leaves()) == dict(other.leaves())

    def as_dict(self):
        return dict(self.leaves())


def check_config_support(config: CompilerConfig) -> None:
    """Warns once about GE-only option groups that were set (they have no effect here)."""
    set_groups = [g for g in ("ge_config", "fusion_config", "dump_config", "export", "inference_config")
                  if len(vars(getattr(config, g))) > 1]
    if set_groups:
        warnings.warn("The following torchair config groups have no effect on the ROCm backend: "
                      + ", ".join(set_groups), UserWarning)
