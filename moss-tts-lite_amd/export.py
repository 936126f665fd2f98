"""Reads the reference's standalone GPTQ export directories (moss_tts_lite/export.py).

What a directory holds (the on-disk format, moss_tts_lite/export.py:29-32, 55, 424-438):
- ``meta.json`` with ``"format": "moss_tts_lite.standalone-gptq"``, the preset name, the
  weight file's name, per-preset group sizes and bf16 keeps, and ``tool.torch``, the
  torch build that wrote the file;
- one safetensors file (``quantized.safetensors`` unless ``weight_file.name`` says
  otherwise). Its tensors named ``layers.{i}.{linear}.q`` are int4 weights in torch's tiled
  int4 layout (``aten._convert_weight_to_int4pack(pre, 8)``), ``layers.{i}.{linear}.qsz``
  their bf16 ``[K/g, N, 2]`` scales and zeros, and every other tensor is a plain weight.

:func:`read_standalone` returns the reference reader's tuple ``(meta, weights, state,
group_size_map, bf16_keep)``. There ``state[layer][linear] = {"packed", "qsz"}`` holds the
tensors as stored. :class:`moss_tts_lite_amd.gptq.W4Dispatch` turns each ``packed`` into
the strip layout on the GPU (``ops.int4pack_from_torch_tiles``).

torch's tiled layout is not the same on every backend, and the package reads the ROCm one
only. A directory whose ``tool.torch`` does not name a ROCm build is refused with
``ValueError`` rather than decoded into wrong weights.

Only json and safetensors touch the files, so nothing in them is executed.
"""
from __future__ import annotations

import json
import os
import re

import torch

from .gptq import LIN_NAMES

__all__ = ["FORMAT_TAG", "META_FILE", "Q_FILE", "is_standalone_dir", "standalone_presets",
           "read_standalone", "tiles_backend"]

FORMAT_TAG = "moss_tts_lite.standalone-gptq"
Q_FILE = "quantized.safetensors"
META_FILE = "meta.json"

# "layers.<i>.<linear>.<q|qsz>"
_INT4_NAME = re.compile(r"layers\.(?P<layer>\d+)\.(?P<linear>%s)\.(?P<part>qsz|q)"
                        % "|".join(LIN_NAMES))
_PART_FIELD = {"q": "packed", "qsz": "qsz"}


def _load_meta(model_dir: str) -> dict:
    with open(os.path.join(model_dir, META_FILE), encoding="utf-8") as fh:
        return json.load(fh)


def is_standalone_dir(path: str) -> bool:
    """Whether ``path`` holds a readable ``meta.json`` carrying the standalone format tag
    (the reference's test, export.py:639-649)."""
    try:
        return _load_meta(path).get("format") == FORMAT_TAG
    except (OSError, ValueError):
        return False


def standalone_presets(path: str) -> list[str]:
    """The presets a directory offers (export.py:651-657): the keys of ``presets``, or
    the lone ``preset_name`` of a directory without that table."""
    meta = _load_meta(path)
    table = meta.get("presets") or {}
    if table:
        return list(table)
    return [meta["preset_name"]] if meta.get("preset_name") else []


def tiles_backend(meta: dict) -> str:
    """``"rocm"`` when ``meta.tool.torch`` names a ROCm build of torch, else the version
    string found (``""`` when the export does not say)."""
    version = str(((meta.get("tool") or {}).get("torch")) or "")
    return "rocm" if "+rocm" in version else version


def _pair(key: str) -> tuple[int, str]:
    layer, _, linear = key.partition(":")
    return int(layer), linear


def _preset_tables(meta: dict) -> tuple[dict, list]:
    preset = (meta.get("presets") or {}).get(meta.get("preset_name"), {})
    gmap = {_pair(k): int(g) for k, g in (preset.get("group_size_map") or {}).items()}
    keep: list = [_pair(k) for k in (preset.get("bf16_linears") or [])]
    keep.extend(int(layer) for layer in (preset.get("bf16_layers") or []))
    return gmap, keep


def _weight_path(model_dir: str, meta: dict) -> str:
    entry = meta.get("weight_file")
    name = entry.get("name", Q_FILE) if isinstance(entry, dict) else Q_FILE
    return os.path.join(model_dir, name)


def read_standalone(model_dir: str, expected_preset: str | None = None):
    """``(meta, weights, state, group_size_map, bf16_keep)`` of a standalone directory,
    with the reference reader's meaning (export.py:691-734).

    Raises:
    - ``ValueError``: the directory is of another format; an int4 record lacks its ``q``
      or ``qsz``; or its tiles were written by a torch build other than ROCm's.
    - ``SystemExit``: ``expected_preset`` is not the directory's preset (the reference
      stops there too).
    - ``FileNotFoundError``: the weight file is missing.
    """
    meta = _load_meta(model_dir)
    if meta.get("format") != FORMAT_TAG:
        raise ValueError(f"{model_dir}: meta.json has format {meta.get('format')!r}, "
                         f"expected {FORMAT_TAG!r}")
    preset = meta.get("preset_name")
    if expected_preset and expected_preset != preset:
        raise SystemExit(f"{model_dir} holds preset {preset!r}, not {expected_preset!r} "
                         f"(presets offered: {standalone_presets(model_dir)})")
    path = _weight_path(model_dir, meta)
    if not os.path.isfile(path):
        raise FileNotFoundError(f"weight file {path} is missing")
    from safetensors import safe_open

    weights: dict[str, torch.Tensor] = {}
    state: dict[int, dict[str, dict[str, torch.Tensor]]] = {}
    with safe_open(path, framework="pt", device="cpu") as fh:
        for name in fh.keys():
            hit = _INT4_NAME.fullmatch(name)
            if hit is None:
                weights[name] = fh.get_tensor(name)
                continue
            rec = state.setdefault(int(hit["layer"]), {}).setdefault(hit["linear"], {})
            rec[_PART_FIELD[hit["part"]]] = fh.get_tensor(name)
    for layer in sorted(state):
        for linear, rec in state[layer].items():
            missing = {"packed", "qsz"} - set(rec)
            if missing:
                raise ValueError(f"{model_dir}: layer {layer} {linear} has an incomplete "
                                 f"int4 record (no {', '.join(sorted(missing))})")
    if state and tiles_backend(meta) != "rocm":
        raise ValueError(f"{model_dir}: its int4 tiles were written by torch "
                         f"{tiles_backend(meta) or '(version not recorded)'}; only the "
                         "tile layout of ROCm builds is read here")
    gmap, keep = _preset_tables(meta)
    return meta, weights, state, gmap, keep
