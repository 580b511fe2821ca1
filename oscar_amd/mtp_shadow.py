"""bf16 shadow KV pool for MTP draft layers (the role of oscar_ascend/mtp_shadow.py:29-61).

Under OSCAR's pool geometry the engine's KV tensors are int8 views with D-byte slots
for every attention layer.  MTP draft layers stay on the native bf16 attention
(quantized draft KV lowers the acceptance rate), and the native path cannot write bf16
K/V into an int8 pool.  Their impl therefore keeps its native class with one change:
at forward time a non-bf16 ``kv_cache`` is replaced by a bf16 pool of the same logical
shape, allocated once per layer.  The shadow shares the main pool's block-id space,
so slot_mapping and block tables apply unchanged; a bf16 pool (the legacy 2D-byte
geometry) is used as it is.  Building the shadow is not optional: a failure raises,
since a native write into the int8 pool would corrupt it silently.
"""
from __future__ import annotations

import torch

_CLASSES: dict[type, type] = {}


def _pair(kv_cache):
    """(K, V) of a (K, V) pair or a stacked [2, ...] tensor; None for anything else."""
    if isinstance(kv_cache, (tuple, list, torch.Tensor)) and len(kv_cache) >= 2 and kv_cache[0] is not None:
        return kv_cache[0], kv_cache[1]
    return None


class _ShadowKV:
    """Mixin placed before the native impl class (see :func:`shadow_impl_class`)."""

    _oscar_shadow = True

    def _shadow_kv(self, kv_cache):
        """The layer's bf16 (K, V): the pool itself when it is bf16, else zero-filled
        bf16 tensors of the pool's logical shape, created on the first call."""
        cached = getattr(self, "_oscar_shadow_kv", None)
        if cached is not None:
            return cached
        pair = _pair(kv_cache)
        if pair is None:
            raise ValueError("MTP shadow pool: kv_cache is not a (K, V) pair")
        k, v = pair
        if k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16:
            return k, v
        self._oscar_shadow_kv = (torch.zeros(k.shape, dtype=torch.bfloat16, device=k.device),
                                 torch.zeros(v.shape, dtype=torch.bfloat16, device=v.device))
        gib = (k.numel() + v.numel()) * 2 / 2 ** 30
        print(f"[oscar-amd] MTP shadow pool: shape={tuple(k.shape)} bf16 x2 ({gib:.2f} GiB, "
              "block ids shared with the main pool)")
        return self._oscar_shadow_kv

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
        pair = _pair(kv_cache)
        if pair is not None and pair[0].dtype != torch.bfloat16:
            kv_cache = self._shadow_kv(kv_cache)
        return super().forward(layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs)


def shadow_impl_class(native_cls: type) -> type:
    """The native impl class with the shadow pool in front of its forward (one class
    per native class)."""
    if getattr(native_cls, "_oscar_shadow", False):
        return native_cls
    cls = _CLASSES.get(native_cls)
    if cls is None:
        cls = type(f"MTPShadow{native_cls.__name__}", (_ShadowKV, native_cls), {})
        _CLASSES[native_cls] = cls
    return cls


def install_shadow(impl) -> None:
    impl.__class__ = shadow_impl_class(type(impl))


def is_shadow_impl(impl) -> bool:
    return impl is not None and getattr(type(impl), "_oscar_shadow", False)
