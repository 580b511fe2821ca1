"""bf16 shadow KV pool for MTP draft layers (the role of oscar_ascend/mtp_shadow.py:29-61).

Under OSCAR's pool geometry the engine's KV tensors are int8 views with D-byte slots
for every attention layer.  MTP draft layers stay on the native bf16 attention
(quantized draft KV lowers the acceptance rate), and the native path cannot write bf16
K/V into an int8 pool.  Their impl therefore keeps its native class with one change:
every entry point that receives ``kv_cache`` (``forward`` and ``do_kv_cache_update``)
is handed a bf16 pool of the same logical shape and the same container type (a (K, V)
pair stays a pair, a stacked ``[2, ...]`` tensor stays stacked), allocated once per
layer.  The shadow shares the main pool's block-id space, so slot_mapping and block
tables apply unchanged; a bf16 pool (the legacy 2D-byte geometry) is used as it is.
Building the shadow is not optional: a failure raises, since a native write into the
int8 pool would corrupt it silently.
"""
from __future__ import annotations

import torch

_CLASSES: dict[type, type] = {}


def _halves(kv_cache):
    """(K, V) views of a (K, V) pair or of a stacked [2, ...] tensor; None otherwise."""
    if isinstance(kv_cache, torch.Tensor):
        return (kv_cache[0], kv_cache[1]) if kv_cache.ndim >= 1 and kv_cache.shape[0] == 2 else None
    if isinstance(kv_cache, (tuple, list)) and len(kv_cache) >= 2 and kv_cache[0] is not None:
        return kv_cache[0], kv_cache[1]
    return None


def _needs_shadow(kv_cache) -> bool:
    halves = _halves(kv_cache)
    return halves is not None and not all(t.dtype == torch.bfloat16 for t in halves)


class _ShadowKV:
    """Mixin placed before the native impl class (see :func:`shadow_impl_class`)."""

    _oscar_shadow = True

    def _shadow_kv(self, kv_cache):
        """The pool this layer's native code must see: ``kv_cache`` itself when it is
        already bf16, else a zero-filled bf16 twin in the same container type, built on
        the first call and reused (one per layer)."""
        if not _needs_shadow(kv_cache):
            if _halves(kv_cache) is None:
                raise ValueError("MTP shadow pool: kv_cache is neither a (K, V) pair nor a stacked [2, ...] tensor")
            return kv_cache
        twin = self.__dict__.get("_oscar_shadow_kv")
        if twin is None:
            if isinstance(kv_cache, torch.Tensor):
                twin = torch.zeros(kv_cache.shape, dtype=torch.bfloat16, device=kv_cache.device)
            else:
                k, v = _halves(kv_cache)
                twin = (torch.zeros(k.shape, dtype=torch.bfloat16, device=k.device),
                        torch.zeros(v.shape, dtype=torch.bfloat16, device=v.device))
            self._oscar_shadow_kv = twin
            nbytes = sum(t.numel() for t in _halves(twin)) * 2
            print(f"[oscar-amd] MTP shadow pool: {tuple(_halves(twin)[0].shape)} bf16 K and V "
                  f"({nbytes / 2 ** 30:.2f} GiB), block ids shared with the main pool")
        return twin

    def forward(self, layer, query, key, value, kv_cache, attn_metadata, *args, **kwargs):
        return super().forward(layer, query, key, value, self._shadow_kv(kv_cache), attn_metadata,
                               *args, **kwargs)


class _ShadowKVUpdate(_ShadowKV):
    """The mixin for native impls that also write K/V outside forward."""

    def do_kv_cache_update(self, layer, key, value, kv_cache, slot_mapping, *args, **kwargs):
        # the draft's bf16 K/V go to the shadow, never into the int8 pool
        return super().do_kv_cache_update(layer, key, value, self._shadow_kv(kv_cache), slot_mapping,
                                          *args, **kwargs)


def shadow_impl_class(native_cls: type) -> type:
    """The native impl class with the shadow pool in front of each of its entry points
    that take ``kv_cache`` (one class per native class; ``do_kv_cache_update`` only
    where the native class has it)."""
    if getattr(native_cls, "_oscar_shadow", False):
        return native_cls
    cls = _CLASSES.get(native_cls)
    if cls is None:
        mixin = _ShadowKVUpdate if callable(getattr(native_cls, "do_kv_cache_update", None)) else _ShadowKV
        cls = type(f"MTPShadow{native_cls.__name__}", (mixin, native_cls), {})
        _CLASSES[native_cls] = cls
    return cls


def shadow_halves(kv_cache):
    """(K, V) of a pool or shadow in either container type."""
    halves = _halves(kv_cache)
    if halves is None:
        raise ValueError("MTP shadow pool: kv_cache is neither a (K, V) pair nor a stacked [2, ...] tensor")
    return halves


def install_shadow(impl) -> None:
    impl.__class__ = shadow_impl_class(type(impl))


def is_shadow_impl(impl) -> bool:
    return impl is not None and getattr(type(impl), "_oscar_shadow", False)
