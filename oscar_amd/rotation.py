"""Per-layer K/V rotations from a calibration checkpoint.

The checkpoint layouts are files users already have, so they are read as the
reference reads them (oscar_ascend/rotation.py:44-129, writer gen_rotations.py:228-239):

* ``{"format_version": 2, "objective": ..., "layers": {id: {"rotation": R, "rotation_v": Rv, ...}}}``
* ``{"layers": {id: R}}`` or ``{id: R}`` or ``{id: {"rotation": R, ...}}``
* a stacked ``[num_layers, D, D]`` tensor.

Layer ids may be ints, digit strings or module names (``...layers.11...``).  Every
layout is normalised into one table ``{layer index: {"k": R, "v": Rv or R}}``; an
empty path or a missing layer gives the identity (or an error with ``strict``).
Files are opened with ``torch.load(weights_only=True)``: nothing in them is executed.
"""
from __future__ import annotations

import re
from functools import lru_cache

import torch

_DECODER_LAYER = re.compile(r"\.layers\.(\d+)\.")
_NUMBER = re.compile(r"\d+")


def layer_index_from_name(name: str) -> int | None:
    """Decoder-layer index of a vLLM layer name: the number of ``.layers.<i>.``, else the
    last number in the name, else None (rotation.py:18-24 contract)."""
    hit = _DECODER_LAYER.search(name)
    if hit is not None:
        return int(hit.group(1))
    numbers = _NUMBER.findall(name)
    return int(numbers[-1]) if numbers else None


def _layer_key(key) -> int | None:
    """A checkpoint key as a layer index: ints as they are, digit strings parsed, module
    names by the layer-name rule; anything else is not a layer."""
    if isinstance(key, int):
        return key
    if not isinstance(key, str):
        return None
    try:
        return int(key)
    except ValueError:
        return layer_index_from_name(key)


def _matrices(value) -> dict | None:
    """One layer's matrices {"k": R, "v": Rv (R when absent)} from a bare matrix or a
    dict entry holding "rotation" (and optionally "rotation_v"); None if neither."""
    if torch.is_tensor(value):
        r = value.float().contiguous()
        return {"k": r, "v": r}
    if isinstance(value, dict) and torch.is_tensor(value.get("rotation")):
        rk = value["rotation"].float().contiguous()
        rv = value.get("rotation_v")
        return {"k": rk, "v": rv.float().contiguous() if torch.is_tensor(rv) else rk}
    return None


def _is_current_recipe(obj) -> bool:
    return (isinstance(obj, dict) and obj.get("format_version", 0) >= 2
            and "r_h_pbr" in str(obj.get("objective", "")))


@lru_cache(maxsize=8)
def load_rotation_table(path: str) -> dict[int, dict[str, torch.Tensor]]:
    """The checkpoint at ``path`` as {layer index: {"k": R, "v": Rv}} (CPU fp32, cached)."""
    obj = torch.load(path, map_location="cpu", weights_only=True)
    if torch.is_tensor(obj) and obj.dim() == 3:
        return {i: _matrices(obj[i]) for i in range(obj.shape[0])}
    if not isinstance(obj, dict):
        raise ValueError(f"Unrecognized OSCAR rotation checkpoint structure at {path!r}: {type(obj)}")
    if not _is_current_recipe(obj):
        print(f"[oscar-amd] rotation checkpoint {path!r} does not declare the format_version >= 2 "
              "U@H@P_br recipe; per-vector INT2 accuracy degrades")
    entries = obj["layers"] if "layers" in obj else obj
    table: dict[int, dict[str, torch.Tensor]] = {}
    for key, value in entries.items():
        index, mats = _layer_key(key), _matrices(value)
        if index is not None and mats is not None:
            table[index] = mats
    return table


def _check(r: torch.Tensor, head_dim: int, where: str, strict: bool) -> None:
    if tuple(r.shape) != (head_dim, head_dim):
        raise ValueError(f"OSCAR rotation for {where} has shape {tuple(r.shape)}, "
                         f"expected ({head_dim}, {head_dim}).")
    if strict:
        eye = torch.eye(head_dim)
        if not bool(torch.isfinite(r).all()) or not torch.allclose(r @ r.t(), eye, atol=1e-3, rtol=1e-3):
            raise ValueError(f"OSCAR rotation for {where} is not finite/orthogonal")


def get_layer_rotation(path: str, layer_name: str, head_dim: int, device,
                       dtype: torch.dtype = torch.float32, mode: str = "k",
                       strict: bool = False) -> torch.Tensor:
    """[D, D] rotation of ``layer_name`` (x_rot = x @ R): mode "k" or "v" (R_v, falling
    back to R).  No path, or (non-strict) no entry for the layer -> identity."""
    identity = torch.eye(head_dim, device=device, dtype=dtype)
    if not path:
        return identity
    index = layer_index_from_name(layer_name)
    mats = load_rotation_table(path).get(index) if index is not None else None
    if mats is None:
        if strict:
            raise ValueError(f"Rotation checkpoint {path!r} is missing layer {layer_name}")
        return identity
    r = mats["v" if mode == "v" else "k"]
    _check(r, head_dim, f"layer {index} of {path!r}", strict)
    return r.to(device=device, dtype=dtype).contiguous()
