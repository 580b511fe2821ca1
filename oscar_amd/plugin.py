"""vllm.general_plugins entry point (mirror of oscar_ascend/plugin.py:73-267).

``load_plugin()`` (no arguments, idempotent) wraps
``vllm.model_executor.layers.attention.attention.Attention.__init__``; after a
layer is constructed, FULL decoder layers of hybrid models have their
``impl.__class__`` swapped to ``OscarAttentionBackendImpl`` (class surgery that
is rolled back if setup raises).  MTP draft layers, non-decoder layers, sliding
windows and attention sinks are left on the native path.

Entry point to register (pyproject):
    [project.entry-points."vllm.general_plugins"]
    oscar_amd = "oscar_amd.plugin:load_plugin"
"""
from __future__ import annotations

import os

_HEARTBEAT: dict = {"loaded": 0, "layers": [], "errors": []}
_PATCHED = False
_SKIP_REASONS_LOGGED: set = set()


def install_impl(impl, target_class):
    """plugin.py:60-70: commit class surgery only if setup succeeds; restore otherwise."""
    old_class, old_state = impl.__class__, impl.__dict__.copy()
    try:
        impl.__class__ = target_class
        impl._oscar_setup()
    except Exception:
        impl.__class__ = old_class
        impl.__dict__.clear()
        impl.__dict__.update(old_state)
        raise


def _is_hybrid_config(model_config) -> bool:
    """plugin.py:202-214: registry flag, or any non-attention entry in layer_types."""
    if getattr(model_config, "is_hybrid", False):
        return True
    hf = getattr(model_config, "hf_text_config", None) or getattr(model_config, "hf_config", None)
    layer_types = getattr(hf, "layer_types", None) or []
    return any(lt != "attention" for lt in layer_types)


def _should_oscar(layer, impl, model_config=None) -> bool:
    """plugin.py:220-253: FULL decoder attention of a hybrid model, never an MTP draft."""
    layer_name = getattr(layer, "layer_name", "") or ""
    if ".mtp." in layer_name or layer_name.startswith("mtp."):
        if "mtp-draft" not in _SKIP_REASONS_LOGGED:
            _SKIP_REASONS_LOGGED.add("mtp-draft")
            print(f"[oscar-amd][SKIP] {layer_name}: mtp-draft (draft KV stays bf16)")
        return False
    try:
        if model_config is None:
            from vllm.config import get_current_vllm_config

            model_config = get_current_vllm_config().model_config
        reasons = []
        if not _is_hybrid_config(model_config):
            reasons.append("not-hybrid")
        at = getattr(impl, "attn_type", "decoder")
        if str(getattr(at, "value", at)) != "decoder":
            reasons.append(f"attn_type={at!r}")
        if getattr(impl, "sliding_window", None) is not None:
            reasons.append("sliding-window")
        if getattr(impl, "sinks", None) is not None:
            reasons.append("sinks")
        if reasons:
            key = ",".join(reasons)
            if key not in _SKIP_REASONS_LOGGED:
                _SKIP_REASONS_LOGGED.add(key)
                print(f"[oscar-amd][SKIP] {layer_name}: {key}")
            return False
        return True
    except Exception as e:  # pragma: no cover - reported, layer stays native
        print(f"[oscar-amd][SKIP] _should_oscar failed: {e}")
        return False


def _patch_attention_class(attention_cls, target_class=None) -> None:
    """Wrap ``attention_cls.__init__`` with the OSCAR after-hook."""
    orig_init = attention_cls.__init__

    def _patched_init(self, *args, **kwargs):
        orig_init(self, *args, **kwargs)
        impl = getattr(self, "impl", None)
        if impl is None or not _should_oscar(self, impl):
            return None
        try:
            from .backend import OscarAttentionBackendImpl

            install_impl(impl, target_class or OscarAttentionBackendImpl)
            _HEARTBEAT["loaded"] += 1
            _HEARTBEAT["layers"].append(
                f"{getattr(self, 'layer_name', '?')}:heads={impl.num_heads}/kv={impl.num_kv_heads}"
                f"/d={impl.head_size}")
        except Exception as e:
            _HEARTBEAT["errors"].append(str(e))
            raise RuntimeError(f"[oscar-amd] injection failed: {getattr(self, 'layer_name', '?')}: {e}") from e
        return None

    attention_cls.__init__ = _patched_init


def load_plugin() -> None:
    """plugin.py:73-181: idempotent; OSCAR_ASCEND_ENABLE=0 disables the surgery."""
    global _PATCHED
    if _PATCHED:
        return
    if os.environ.get("OSCAR_ASCEND_ENABLE", "auto") == "0":
        print("[oscar-amd] OSCAR_ASCEND_ENABLE=0: native attention path kept")
        _PATCHED = True
        return
    try:
        from vllm.model_executor.layers.attention.attention import Attention
    except Exception as e:
        _HEARTBEAT["errors"].append(f"attention import: {e}")
        print(f"[oscar-amd] Attention not found, plugin inactive: {e}")
        _PATCHED = True
        return
    _patch_attention_class(Attention)
    _PATCHED = True
    print("[oscar-amd] plugin installed: Attention.__init__ after-hook")


def heartbeat() -> dict:
    return dict(_HEARTBEAT)
