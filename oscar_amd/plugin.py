"""vllm.general_plugins entry point (mirror of oscar_ascend/plugin.py:73-267).

``load_plugin()`` (no arguments, idempotent) wraps
``vllm.model_executor.layers.attention.attention.Attention.__init__``; after a
layer is constructed, FULL decoder layers of hybrid models have their
``impl.__class__`` swapped to ``OscarAttentionBackendImpl`` (class surgery that
is rolled back if setup raises).  Non-decoder layers, sliding windows and attention
sinks are left on the native path; MTP draft layers stay native too, in front of a
bf16 shadow of the int8 pool (``oscar_amd.mtp_shadow``).  The worker hooks of
``oscar_amd.integration`` (memory budget, cache initialization, READY manifest) are
installed alongside when the worker classes import.

Entry point to register (pyproject):
    [project.entry-points."vllm.general_plugins"]
    oscar_amd = "oscar_amd.plugin:load_plugin"
"""
from __future__ import annotations

import os

_HEARTBEAT: dict = {"loaded": 0, "layers": [], "shadow_layers": [], "errors": []}
_PATCHED = False
_SKIP_REASONS_LOGGED: set = set()


def install_impl(impl, target_class):
    """Move ``impl`` onto ``target_class`` and run its setup as one transaction: if setup
    raises, the object gets its original class and attribute dict back and the error
    propagates (the reference's rollback contract, plugin.py:60-70)."""
    original_class, original_state = type(impl), dict(vars(impl))
    impl.__class__ = target_class
    try:
        impl._oscar_setup()
    except BaseException:
        impl.__class__ = original_class
        vars(impl).clear()
        vars(impl).update(original_state)
        raise


def hybrid_model(model_config) -> bool:
    """True for models that mix attention with other layer kinds: the registry's
    ``is_hybrid`` flag, or a ``layer_types`` list naming anything but "attention"."""
    if getattr(model_config, "is_hybrid", False):
        return True
    text_cfg = getattr(model_config, "hf_text_config", None) or getattr(model_config, "hf_config", None)
    kinds = set(getattr(text_cfg, "layer_types", None) or ())
    return bool(kinds - {"attention"})


def _is_mtp_draft(layer_name: str) -> bool:
    return layer_name.startswith("mtp.") or ".mtp." in layer_name


def skip_reasons(layer, impl, model_config) -> list[str]:
    """Why a layer keeps the native impl (empty list: OSCAR takes it).  OSCAR takes only
    FULL decoder self-attention of hybrid models (plugin.py:220-253); MTP draft layers
    keep bf16 KV, and are turned down before the model config is consulted."""
    if _is_mtp_draft(getattr(layer, "layer_name", "") or ""):
        return ["mtp-draft"]
    reasons = [] if hybrid_model(model_config) else ["not-hybrid"]
    kind = getattr(impl, "attn_type", "decoder")
    if str(getattr(kind, "value", kind)) != "decoder":  # AttentionType is a str enum
        reasons.append(f"attn_type={kind!r}")
    for attr, label in (("sliding_window", "sliding-window"), ("sinks", "sinks")):
        if getattr(impl, attr, None) is not None:
            reasons.append(label)
    return reasons


def _should_oscar(layer, impl, model_config=None) -> bool:
    """skip_reasons() with the live vLLM model config; each distinct reason is logged once."""
    name = getattr(layer, "layer_name", "") or ""
    try:
        if model_config is None and not _is_mtp_draft(name):
            from vllm.config import get_current_vllm_config

            model_config = get_current_vllm_config().model_config
        reasons = skip_reasons(layer, impl, model_config)
    except Exception as e:  # pragma: no cover - reported, the layer stays native
        reasons = [f"routing check failed: {e}"]
    if reasons:
        key = ",".join(reasons)
        if key not in _SKIP_REASONS_LOGGED:
            _SKIP_REASONS_LOGGED.add(key)
            print(f"[oscar-amd][SKIP] {name or '?'}: {key}")
    return not reasons


def _wants_shadow(layer, model_config=None) -> bool:
    """MTP draft layers of models whose FULL layers OSCAR takes get the bf16 shadow pool
    (their native attention cannot use the int8 pool geometry)."""
    if not _is_mtp_draft(getattr(layer, "layer_name", "") or ""):
        return False
    try:
        if model_config is None:
            from vllm.config import get_current_vllm_config

            model_config = get_current_vllm_config().model_config
        return hybrid_model(model_config)
    except Exception as e:  # pragma: no cover - reported, the layer stays native
        _HEARTBEAT["errors"].append(f"shadow routing: {e}")
        return False


def _patch_attention_class(attention_cls, target_class=None) -> None:
    """Wrap ``attention_cls.__init__`` with the OSCAR after-hook."""
    orig_init = attention_cls.__init__

    def _patched_init(self, *args, **kwargs):
        orig_init(self, *args, **kwargs)
        impl = getattr(self, "impl", None)
        if impl is None:
            return None
        if _wants_shadow(self):
            from .mtp_shadow import install_shadow

            install_shadow(impl)  # native bf16 attention on a bf16 shadow of the int8 pool
            _HEARTBEAT["shadow_layers"].append(getattr(self, "layer_name", "?"))
            return None
        if not _should_oscar(self, impl):
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
    try:
        from .integration import install_runner_hooks

        install_runner_hooks()
        print("[oscar-amd] worker hooks installed: memory budget, cache initialization, READY manifest")
    except Exception as e:  # a worker without these seams keeps lazy arenas
        _HEARTBEAT["errors"].append(f"worker hooks: {e}")
        print(f"[oscar-amd] worker hooks not installed: {e}")


def heartbeat() -> dict:
    return dict(_HEARTBEAT)
