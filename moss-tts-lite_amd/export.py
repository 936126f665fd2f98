"""Reader of the reference's standalone GPTQ export (moss_tts_lite/export.py:639-734).

A standalone directory holds ``meta.json`` (``"format": "moss_tts_lite.standalone-gptq"``)
and one safetensors file whose int4 linears are ``layers.{i}.{proj}.q`` (int32: torch's
tiled int4 tensor, ``aten._convert_weight_to_int4pack(pre, 8)``) and
``layers.{i}.{proj}.qsz`` (bf16 ``[K/g, N, 2]``); every other tensor is a bf16 weight.
:func:`read_standalone` returns what the reference's does, the ``(meta, weights, state,
group_size_map, bf16_keep)`` tuple, with ``state[li][proj] = {"packed", "qsz"}`` as read
from the file.  :class:`moss_tts_lite_amd.gptq.W4Dispatch` takes that state and converts
each ``packed`` into this build's layout on the GPU (``ops.int4pack_from_torch_tiles``).

Files are read with safetensors and json only: nothing in them is executed.
"""
from __future__ import annotations

import json
import os
import re

import torch

from .gptq import LIN_NAMES

__all__ = ["FORMAT_TAG", "META_FILE", "Q_FILE", "is_standalone_dir", "standalone_presets",
           "read_standalone"]

# names of the reference's format (export.py:29-32) and its record keys (export.py:55)
FORMAT_TAG = "moss_tts_lite.standalone-gptq"
Q_FILE = "quantized.safetensors"
META_FILE = "meta.json"
_Q_KEY = re.compile(r"^layers\.(\d+)\.(" + "|".join(LIN_NAMES) + r")\.(q|qsz)$")
_RECORD = {"q": "packed", "qsz": "qsz"}


def _meta(path: str) -> dict:
    with open(os.path.join(path, META_FILE), encoding="utf-8") as f:
        return json.load(f)


def is_standalone_dir(path: str) -> bool:
    """True if ``path`` holds a standalone export's ``meta.json`` (export.py:639-649)."""
    if not os.path.isfile(os.path.join(path, META_FILE)):
        return False
    try:
        meta = _meta(path)
    except (OSError, json.JSONDecodeError):
        return False
    return meta.get("format") == FORMAT_TAG


def standalone_presets(path: str) -> list[str]:
    """Preset names a standalone directory offers (export.py:651-657)."""
    meta = _meta(path)
    names = list(meta.get("presets") or {})
    if not names and meta.get("preset_name"):
        names = [meta["preset_name"]]
    return names


def _read_safetensors(path: str) -> dict[str, torch.Tensor]:
    from safetensors import safe_open
    out = {}
    with safe_open(path, framework="pt", device="cpu") as f:
        for key in f.keys():
            out[key] = f.get_tensor(key)
    return out


def read_standalone(model_dir: str, expected_preset: str | None = None):
    """Read a standalone directory (export.py:691-734): ``(meta, weights, state, gmap, keep)``.

    ``state[li][proj]`` is ``{"packed": int32 torch tiles, "qsz": bf16 [K/g, N, 2]}``,
    ``gmap[(li, proj)]`` the per-linear group size of the preset, ``keep`` the bf16-kept
    linears ``(li, proj)`` and layers ``li``.  Raises ``ValueError`` for a directory of
    another format or a record missing its ``q`` or ``qsz``, ``SystemExit`` when
    ``expected_preset`` is not the directory's preset, ``FileNotFoundError`` for a missing
    weight file.
    """
    meta = _meta(model_dir)
    if meta.get("format") != FORMAT_TAG:
        raise ValueError(f"{os.path.join(model_dir, META_FILE)} is not a {FORMAT_TAG} directory")
    preset = meta.get("preset_name")
    if expected_preset and expected_preset != preset:
        raise SystemExit(f"[export] {model_dir} provides preset {preset!r} only, but "
                         f"{expected_preset!r} was requested. Available: "
                         f"{standalone_presets(model_dir)}")
    wf = meta.get("weight_file")
    qfile = os.path.join(model_dir, wf["name"] if isinstance(wf, dict) else Q_FILE)
    if not os.path.isfile(qfile):
        raise FileNotFoundError(f"{qfile} not found in {model_dir}")
    weights: dict[str, torch.Tensor] = {}
    state: dict[int, dict[str, dict[str, torch.Tensor]]] = {}
    for key, t in _read_safetensors(qfile).items():
        m = _Q_KEY.match(key)
        if m:
            state.setdefault(int(m.group(1)), {}).setdefault(m.group(2), {})[_RECORD[m.group(3)]] = t
        else:
            weights[key] = t
    for li, projs in state.items():
        for proj, rec in projs.items():
            if set(rec) != {"packed", "qsz"}:
                raise ValueError(f"incomplete record for layer {li} {proj}: {sorted(rec)}")
    pmeta = (meta.get("presets") or {}).get(preset, {})
    gmap = {}
    for key, val in (pmeta.get("group_size_map") or {}).items():
        a, b = key.split(":")
        gmap[(int(a), b)] = int(val)
    keep: list = [(int(x.split(":")[0]), x.split(":")[1]) for x in (pmeta.get("bf16_linears") or [])]
    keep += [int(x) for x in (pmeta.get("bf16_layers") or [])]
    return meta, weights, state, gmap, keep
