"""RoPE base resolution, shared by the torch path and the HIP tables.

Same precedence as the reference ``src/nanovllm/rope_config.py:25-92``:
a top-level ``rope_theta`` wins, then one nested in ``rope_scaling`` /
``rope_parameters``, then Qwen3's default 1e6. Scaled RoPE variants are
rejected rather than silently ignored.
"""

from __future__ import annotations

from typing import Any

QWEN3_DEFAULT_ROPE_THETA = 1_000_000.0
_THETA_KEYS = ("rope_theta", "rope_parameters")


def _get(config: Any, key: str):
    if isinstance(config, dict):
        return config.get(key)
    return getattr(config, key, None)


def _number(value: Any) -> float | None:
    if isinstance(value, bool) or not isinstance(value, (int, float)):
        return None
    return float(value)


def resolve_rope_theta(config: Any, default: float = QWEN3_DEFAULT_ROPE_THETA) -> float:
    for key in _THETA_KEYS:
        value = _number(_get(config, key))
        if value is not None:
            return value
    nested = _get(config, "rope_scaling") or _get(config, "rope_parameters")
    if isinstance(nested, dict):
        for key in _THETA_KEYS:
            value = _number(nested.get(key))
            if value is not None:
                return value
    return float(default)


def resolve_rope_type(config: Any) -> str | None:
    nested = _get(config, "rope_scaling") or _get(config, "rope_parameters")
    if not isinstance(nested, dict):
        return None
    kind = nested.get("rope_type") or nested.get("type")
    return None if kind is None else str(kind)


def assert_supported_rope_type(config: Any) -> None:
    kind = resolve_rope_type(config)
    if kind is None or kind.lower() == "default":
        return
    raise NotImplementedError(
        f"rope_type={kind!r} is not supported: only unscaled RoPE is "
        "implemented (torch path and HIP cos/sin tables alike)."
    )
