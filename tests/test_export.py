"""Host logic of the standalone-export reader (moss_tts_lite/export.py:639-734) on CPU:
record grouping, preset metadata, bf16 keeps and the reference's error behaviour."""
import json

import pytest
import torch

from moss_tts_lite_amd import export as E


def _write_dir(path, records, meta_over=None, preset="w4-mixed"):
    from safetensors.torch import save_file
    save_file(records, str(path / E.Q_FILE), metadata={"format": E.FORMAT_TAG, "preset": preset})
    meta = {"format": E.FORMAT_TAG, "preset_name": preset,
            "weight_file": {"name": E.Q_FILE, "bytes": 0, "sha256": ""},
            "presets": {preset: {"group_size_default": 128,
                                 "group_size_map": {"0:o": 32, "1:down": 256},
                                 "bf16_linears": ["0:v"], "bf16_layers": [2]}},
            "quantization": {"method": "gptq", "inner_k_tiles": 8},
            "tool": {"name": "moss_tts_lite.export.export_standalone", "torch": "2.10.0+rocm7.0"}}
    meta.update(meta_over or {})
    (path / E.META_FILE).write_text(json.dumps(meta))


def _records():
    tiles = lambda n, k: torch.zeros(n // 8, k // 128, 32, 4, dtype=torch.int32)  # noqa: E731
    qsz = lambda n, k, g: torch.zeros(k // g, n, 2, dtype=torch.bfloat16)  # noqa: E731
    return {"layers.0.o.q": tiles(256, 512), "layers.0.o.qsz": qsz(256, 512, 32),
            "layers.1.down.q": tiles(128, 1024), "layers.1.down.qsz": qsz(128, 1024, 256),
            "layers.0.self_attn.v_proj.weight": torch.ones(64, 512, dtype=torch.bfloat16),
            "embed.weight": torch.ones(16, 512, dtype=torch.bfloat16)}


def test_read_standalone_groups_records(tmp_path):
    _write_dir(tmp_path, _records())
    assert E.is_standalone_dir(str(tmp_path))
    assert E.standalone_presets(str(tmp_path)) == ["w4-mixed"]
    meta, weights, state, gmap, keep = E.read_standalone(str(tmp_path), "w4-mixed")
    assert meta["quantization"]["inner_k_tiles"] == 8
    assert sorted(weights) == ["embed.weight", "layers.0.self_attn.v_proj.weight"]
    assert sorted(state) == [0, 1] and sorted(state[0]) == ["o"] and sorted(state[1]) == ["down"]
    assert set(state[0]["o"]) == {"packed", "qsz"}
    assert state[0]["o"]["packed"].dtype == torch.int32
    assert tuple(state[1]["down"]["packed"].shape) == (16, 8, 32, 4)
    assert state[1]["down"]["qsz"].dtype == torch.bfloat16
    assert gmap == {(0, "o"): 32, (1, "down"): 256}
    assert keep == [(0, "v"), 2]


def test_read_standalone_errors(tmp_path):
    a = tmp_path / "a"; a.mkdir()
    _write_dir(a, _records())
    with pytest.raises(SystemExit):
        E.read_standalone(str(a), "other-preset")
    b = tmp_path / "b"; b.mkdir()
    recs = _records(); recs.pop("layers.0.o.qsz")
    _write_dir(b, recs)
    with pytest.raises(ValueError, match="incomplete int4 record"):
        E.read_standalone(str(b))
    c = tmp_path / "c"; c.mkdir()
    _write_dir(c, _records(), meta_over={"format": "something-else"})
    assert not E.is_standalone_dir(str(c))
    with pytest.raises(ValueError):
        E.read_standalone(str(c))
    d = tmp_path / "d"; d.mkdir()
    _write_dir(d, _records(), meta_over={"weight_file": {"name": "missing.safetensors"}})
    with pytest.raises(FileNotFoundError):
        E.read_standalone(str(d))
    assert not E.is_standalone_dir(str(tmp_path / "nowhere"))


@pytest.mark.parametrize("torch_version", ["2.9.1+cu128", "2.9.1", None])
def test_read_standalone_refuses_tiles_of_other_torch_builds(tmp_path, torch_version):
    # a CUDA build of torch tiles the same [N/8, K/(16T), 32, T/2] shape differently: an
    # export it wrote (the reference's own, "CUDA required", export.py:438) is refused,
    # as is one that does not record its torch
    tool = {"name": "x"} if torch_version is None else {"name": "x", "torch": torch_version}
    _write_dir(tmp_path, _records(), meta_over={"tool": tool})
    assert E.tiles_backend(json.loads((tmp_path / E.META_FILE).read_text())) != "rocm"
    with pytest.raises(ValueError, match="ROCm"):
        E.read_standalone(str(tmp_path))


def test_read_standalone_without_int4_records_needs_no_backend(tmp_path):
    # a directory of plain weights only has no tiles to misread
    recs = {k: v for k, v in _records().items() if not k.endswith((".q", ".qsz"))}
    _write_dir(tmp_path, recs, meta_over={"tool": {"torch": "2.9.1+cu128"}})
    _, weights, state, _, _ = E.read_standalone(str(tmp_path))
    assert state == {} and len(weights) == 2
