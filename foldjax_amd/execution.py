"""The neutral ``triangle_kernel`` knob with the ``"hip"`` value.

Mirrors the reference's vocabulary for the knob every port spells
differently (``src/foldjax/execution.py:33-45``): one neutral name, and per
port a table that translates it to the port's own option name and value
(``src/foldjax/backends/boltz2.py:160-170``, ``backends/protenix.py:179-189``,
``backends/openfold3.py:167-171``), with ``translate``'s rules
(``execution.py:95-135``): a value outside the knob's vocabulary, or one the
port cannot express, is an error, never a silently dropped argument.

This package adds ``"hip"`` to the vocabulary and maps ``"auto"`` -- "the
fastest path this build can actually run" -- to ``"hip"`` explicitly: the
package runs on ROCm only, so there is nothing to probe. ``"cueq"`` and
``"xla"`` keep their native translations; the port mirrors then refuse them
with the reference's selector errors (they are JAX backends).
"""

from __future__ import annotations

from typing import Any

#: Neutral knob -> the values it accepts (the reference's plus "hip").
KNOBS: dict[str, tuple[str, ...]] = {
    "triangle_kernel": ("auto", "cueq", "xla", "hip"),
}

#: Old spellings of the knob that the reference keeps working
#: (``execution.py:50-57``).
ALIASES: dict[str, str] = {
    "triangle_backend": "triangle_kernel",
    "trunk_triangle_attention_backend": "triangle_kernel",
}

#: Per port: neutral knob -> (native option name, {neutral value: native value}).
EXECUTION_OPTIONS: dict[str, dict[str, tuple[str, dict[str, str]]]] = {
    "boltz2": {
        "triangle_kernel": ("triangle_backend", {"auto": "hip", "hip": "hip", "cueq": "cueq", "xla": "xla"}),
    },
    "protenix": {
        "triangle_kernel": (
            "trunk_triangle_attention_backend",
            {"auto": "hip", "hip": "hip", "cueq": "cueq_jit", "xla": "xla_jit"},
        ),
    },
    "openfold3": {
        "triangle_kernel": ("triangle_kernel", {"auto": "hip", "hip": "hip", "cueq": "cueq", "xla": "xla"}),
    },
}


def normalize(options: dict[str, Any], *, native: set[str]) -> dict[str, Any]:
    """Rewrite alias keys to the neutral name (``execution.py:64-92``);
    ``native`` names the options this port takes directly, which are kept."""
    out: dict[str, Any] = {}
    for key, value in options.items():
        neutral = ALIASES.get(key)
        if neutral is None or key in native:
            out[key] = value
            continue
        if neutral in options:
            raise ValueError(
                f"{key!r} and {neutral!r} were both set; {key!r} is the old "
                f"name for {neutral!r}, so pass one of them"
            )
        out[neutral] = value
    return out


def translate(options: dict[str, Any], model: str) -> dict[str, Any]:
    """Neutral knobs -> the port's own option names and values
    (``execution.py:95-135``)."""
    try:
        table = EXECUTION_OPTIONS[model]
    except KeyError:
        raise ValueError(f"unknown model {model!r}; expected one of {tuple(EXECUTION_OPTIONS)}") from None
    out = dict(options)
    for knob, value in list(options.items()):
        if knob not in KNOBS:
            continue
        entry = table.get(knob)
        if entry is None:
            raise ValueError(f"{model} does not support {knob}")
        native_name, values = entry
        allowed = KNOBS[knob]
        if value not in allowed:
            raise ValueError(f"{knob} must be one of {allowed}, got {value!r}")
        native_value = values.get(value)
        if native_value is None:
            raise ValueError(f"{model} does not support {knob}={value!r}; it takes {tuple(values)}")
        del out[knob]
        if native_name in out and native_name != knob:
            raise ValueError(
                f"{knob} and the native option {native_name!r} were both set for {model}; pass one of them"
            )
        out[native_name] = native_value
    return out


def triangle_kernel(model: str, value: str = "auto") -> str:
    """The native triangle selector value for ``triangle_kernel=value`` on
    ``model`` (``"auto"`` -> ``"hip"``)."""
    return translate({"triangle_kernel": value}, model)[EXECUTION_OPTIONS[model]["triangle_kernel"][0]]
