"""Plugin configuration read from the OSCAR_ASCEND_* environment variables.

The variable names, their defaults and their accepted ranges are the reference's
deployment interface (oscar_ascend/config.py:35-103): an environment written for the
reference selects the same behaviour here.  The knobs are declared once, as rows of
``KNOBS`` (variable, attribute, parser, default); ``OscarConfig.from_env`` parses
every row, then checks the combinations this backend supports.

Parsing rules (the reference's): an unset, blank or unparsable number falls back to
the default; window sizes and the workspace budget are clamped at zero; clip ratios
must lie in [0, 1]; only per-vector quantization (group size 0) and the streaming
attention mode exist.
"""
from __future__ import annotations

import os
from dataclasses import dataclass, field
from typing import Callable, NamedTuple

from .format import BITS, D_DEFAULT, LEVELS, SLOT_SIZE

MIB = 1 << 20


def _number(kind: type) -> Callable[[str | None, object], object]:
    def parse(raw: str | None, default):
        if raw is None or not raw.strip():
            return default
        try:
            return kind(raw)
        except ValueError:
            return default
    return parse


def _at_least_zero(raw: str | None, default):
    return max(0, _number(int)(raw, default))


def _text(raw: str | None, default):
    return default if raw is None else raw


def _switch(raw: str | None, default):
    return default if raw is None else raw != "0"


class Knob(NamedTuple):
    env: str
    attr: str
    parse: Callable[[str | None, object], object]
    default: object


KNOBS: tuple[Knob, ...] = (
    Knob("OSCAR_ASCEND_K_CLIP_RATIO", "k_clip_ratio", _number(float), 0.0),
    Knob("OSCAR_ASCEND_V_CLIP_RATIO", "v_clip_ratio", _number(float), 0.0),
    Knob("OSCAR_ASCEND_K_ROTATION_PATH", "k_rotation_path", _text, ""),
    Knob("OSCAR_ASCEND_V_ROTATION_PATH", "v_rotation_path", _text, ""),
    Knob("OSCAR_ASCEND_SINK_TOKENS", "sink_tokens", _at_least_zero, 64),
    Knob("OSCAR_ASCEND_RECENT_TOKENS", "recent_tokens", _at_least_zero, 256),
    Knob("OSCAR_ASCEND_STAGING_TOKENS", "staging_tokens", _at_least_zero, 8192),
    Knob("OSCAR_ASCEND_GROUP_SIZE", "group_size", _number(int), 0),
    Knob("OSCAR_ASCEND_ATTENTION_MODE", "attention_mode", _text, "streaming"),
    Knob("OSCAR_ASCEND_STREAM_WORKSPACE_MIB", "stream_workspace_mib", _at_least_zero, 32),
    Knob("OSCAR_ASCEND_VERBOSE", "verbose", _switch, True),
    Knob("OSCAR_ASCEND_ENABLE", "enable", _text, "auto"),
)


@dataclass
class OscarConfig:
    """One FULL-attention impl's settings (defaults = the reference's)."""

    head_dim: int = D_DEFAULT
    k_clip_ratio: float = 0.0
    v_clip_ratio: float = 0.0
    k_rotation_path: str = ""
    v_rotation_path: str = ""
    sink_tokens: int = 64
    recent_tokens: int = 256
    staging_tokens: int = 8192
    group_size: int = 0
    attention_mode: str = "streaming"
    stream_workspace_mib: int = 32
    verbose: bool = True
    enable: str = "auto"
    extra: dict = field(default_factory=dict)

    # ---- derived quantities
    @property
    def window_enabled(self) -> bool:
        """The FP32 sink/recent window exists when it has room and something to hold."""
        return self.staging_tokens > 0 and (self.sink_tokens > 0 or self.recent_tokens > 0)

    @property
    def stream_workspace_bytes(self) -> int:
        return self.stream_workspace_mib * MIB

    @property
    def levels(self) -> int:
        return LEVELS

    @property
    def data_bytes(self) -> int:
        """Packed code bytes per vector (64 at D = 256)."""
        return -(-self.head_dim * BITS // 8)

    @property
    def slot_bytes(self) -> int:
        """Logical slot: 96 K bytes (meta, padding, codes) + 64 V code bytes."""
        return SLOT_SIZE

    @property
    def num_groups(self) -> int:
        return 1 if self.group_size == 0 else -(-self.head_dim // self.group_size)

    # ---- construction
    @classmethod
    def from_env(cls, head_dim: int | None = None, environ=None) -> "OscarConfig":
        env = os.environ if environ is None else environ
        values = {k.attr: k.parse(env.get(k.env), k.default) for k in KNOBS}
        if head_dim is None:
            head_dim = _number(int)(env.get("OSCAR_ASCEND_HEAD_DIM"), D_DEFAULT)
        cfg = cls(head_dim=head_dim, **values)
        cfg.extra["enable"] = cfg.enable
        cfg.validate()
        return cfg

    def validate(self) -> None:
        problems = []
        if self.attention_mode not in ("streaming", "native"):
            problems.append("OSCAR_ASCEND_ATTENTION_MODE must be streaming or native")
        elif self.attention_mode == "native":
            # the reference's dense-history A/B mode is not part of this backend
            problems.append("OSCAR_ASCEND_ATTENTION_MODE=native (dense history) is not provided "
                            "on MI355X; use streaming")
        for name, ratio in (("K", self.k_clip_ratio), ("V", self.v_clip_ratio)):
            if not 0.0 <= ratio <= 1.0:  # NaN fails too
                problems.append(f"OSCAR {name} clip ratio {ratio!r} must be finite and in [0, 1]")
        if self.group_size != 0:
            problems.append("Only per-vector OSCAR quantization (GROUP_SIZE=0) is supported")
        if problems:
            raise ValueError("; ".join(problems))
