"""The expert offset index and the byte-range loader (vaayu_amd/expert_offset_index.py),
on the CPU: the reference's own index tests (tests/test_expert_offset_index.py,
test_expert_offset_index_fused3d.py, test_expert_offset_index_guard.py) restated against
this implementation, plus the loader's bytes against the tensors that were written."""
import json
import struct
import time
from pathlib import Path

import pytest
import torch
from safetensors.torch import save_file

from vaayu_amd.expert_offset_index import (ExpertOffsetIndex, ExpertTensorMeta,
                                           assert_checkpoint_complete, load_expert_tensors,
                                           load_resident_experts, read_header)
from vaayu_amd.moe_patch import build_expert_blob
from vaayu_amd.synth import quantize_pack


def make_synthetic_moe_shard(tmp_path: Path, layer: str, num_experts: int = 4) -> Path:
    t = {f"{layer}.self_attn.q_proj.weight": torch.randn(8, 8),
         f"{layer}.block_sparse_moe.gate.weight": torch.randn(4, 8)}
    for e in range(num_experts):
        t[f"{layer}.block_sparse_moe.experts.{e}.w1.weight"] = torch.randn(8, 8)
        t[f"{layer}.block_sparse_moe.experts.{e}.w2.weight"] = torch.randn(8, 8)
    path = tmp_path / f"{layer}.safetensors"
    save_file(t, str(path))
    return path


def test_build_finds_expert_entries(tmp_path):
    make_synthetic_moe_shard(tmp_path, "model.layers.0")
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    assert len(idx.get_expert_offsets("model.layers.0", 0)) == 2


def test_expert_meta_fields(tmp_path):
    make_synthetic_moe_shard(tmp_path, "model.layers.0", 2)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    for meta in idx.get_expert_offsets("model.layers.0", 0).values():
        assert isinstance(meta, ExpertTensorMeta)
        assert meta.file_offset > 0 and meta.byte_length == 256
        assert meta.shape == [8, 8] and meta.dtype == "F32"


def test_non_expert_tensors_excluded_and_layer_names(tmp_path):
    make_synthetic_moe_shard(tmp_path, "model.layers.0", 2)
    make_synthetic_moe_shard(tmp_path, "model.layers.1", 2)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    for tensors in idx.index["model.layers.0"].values():
        assert all(".gate." not in k for k in tensors)
    assert sorted(idx.moe_layer_names()) == ["model.layers.0", "model.layers.1"]


def test_cache_round_trip_and_staleness(tmp_path):
    make_synthetic_moe_shard(tmp_path, "model.layers.0", 2)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    data = json.loads((tmp_path / ExpertOffsetIndex.CACHE_FILENAME).read_text())
    assert data["__vaayu_index_version__"] == 2 and "model.layers.0" in data["index"]
    idx2 = ExpertOffsetIndex(str(tmp_path))
    assert idx2.load_cached() is True
    assert idx2.index == idx.index
    time.sleep(0.05)
    (tmp_path / "model.layers.0.safetensors").touch()
    assert ExpertOffsetIndex(str(tmp_path)).load_cached() is False


def test_missing_expert_returns_none_and_build_or_load_twice(tmp_path):
    make_synthetic_moe_shard(tmp_path, "model.layers.0", 2)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build_or_load()
    assert idx.get_expert_offsets("model.layers.0", 99) is None
    assert idx.get_expert_offsets("model.layers.99", 0) is None
    idx2 = ExpertOffsetIndex(str(tmp_path))
    idx2.build_or_load()
    assert idx2.get_expert_offsets("model.layers.0", 0) is not None


# ── fused layout ────────────────────────────────────────────────────────────────────────

@pytest.mark.parametrize("key,shape,expected,want", [
    ("model.layers.0.mlp.experts.gate_up_proj_blocks", [32, 5760, 90, 16], 32, True),
    ("model.layers.0.mlp.experts.down_proj_scales", [32, 2880, 90], 32, True),
    ("model.layers.0.mlp.experts.gate_up_proj_bias", [32, 5760], 32, True),
    ("model.layers.3.block_sparse_moe.experts.w1", [8, 1024, 512], 8, True),
    ("model.layers.0.mlp.experts.0.w1.weight", [4096, 4096], 32, False),
    ("model.layers.0.mlp.experts.gate_up_proj_blocks", [16, 5760, 90], 32, False),
    ("model.layers.0.self_attn.q_proj.weight", [32, 4096], 32, False),
    ("model.layers.0.mlp.experts.gate_up_proj_blocks", [32, 5760, 90], None, False),
    ("model.layers.0.mlp.experts.gate_up_proj_bias", [32], 32, False)])
def test_fused_expert_axis_detection(key, shape, expected, want):
    assert ExpertOffsetIndex._fused_expert_axis(key, shape, expected) is want


def _write_shard(path, tensors):
    header, off = {}, 0
    for key, (dtype, shape, nbytes) in tensors.items():
        header[key] = {"dtype": dtype, "shape": shape, "data_offsets": [off, off + nbytes]}
        off += nbytes
    blob = json.dumps(header).encode()
    path.write_bytes(struct.pack("<Q", len(blob)) + blob + bytes(range(256)) * (off // 256)
                     + bytes(off % 256))
    return 8 + len(blob)


@pytest.mark.parametrize("experts,rows,cols", [(4, 8, 2), (32, 90, 16)])
def test_fused_tensor_one_contiguous_range_per_expert(tmp_path, experts, rows, cols):
    (tmp_path / "config.json").write_text(json.dumps({"num_local_experts": experts}))
    total = experts * rows * cols
    start = _write_shard(tmp_path / "model-00001-of-00001.safetensors",
                         {"model.layers.0.mlp.experts.gate_up_proj_blocks":
                          ("U8", [experts, rows, cols], total)})
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build(write_cache=False)
    shard = idx.index["model-00001-of-00001"]
    assert sorted(shard) == list(range(experts))
    per = rows * cols
    for i in range(experts):
        (meta,) = shard[i].values()
        assert meta.byte_length == per and meta.file_offset == start + i * per
        assert meta.shape == [rows, cols] and meta.dtype == "U8"
    whole = idx.fused_layer_tensors["model-00001-of-00001"][
        "model.layers.0.mlp.experts.gate_up_proj_blocks"]
    assert whole.file_offset == start and whole.byte_length == total


def test_fused_tensor_not_dividing_raises(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"num_local_experts": 3}))
    _write_shard(tmp_path / "model-00001-of-00001.safetensors",
                 {"model.layers.0.mlp.experts.gate_up_proj_blocks": ("U8", [3, 5, 1], 16)})
    with pytest.raises(RuntimeError, match="does not divide evenly"):
        ExpertOffsetIndex(str(tmp_path)).build(write_cache=False)


def test_fused_cache_round_trips_and_version1_still_loads(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"num_local_experts": 4}))
    _write_shard(tmp_path / "model-00001-of-00001.safetensors",
                 {"model.layers.0.mlp.experts.down_proj_blocks": ("U8", [4, 8, 2], 64)})
    ExpertOffsetIndex(str(tmp_path)).build()
    second = ExpertOffsetIndex(str(tmp_path))
    assert second.load_cached() is True
    assert sorted(second.index["model-00001-of-00001"]) == [0, 1, 2, 3]
    assert second.fused_layer_tensors["model-00001-of-00001"]
    v1 = {"model-00001-of-00001": {"0": {"k": {"file_offset": 8, "byte_length": 4,
                                               "shape": [1], "dtype": "U8"}}}}
    (tmp_path / ExpertOffsetIndex.CACHE_FILENAME).write_text(json.dumps(v1))
    third = ExpertOffsetIndex(str(tmp_path))
    assert third.load_cached() is True
    assert third.index["model-00001-of-00001"][0]["k"].byte_length == 4
    assert third.fused_layer_tensors == {}


def test_guard_refuses_an_empty_index_for_an_moe_config(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"num_experts": 8,
                                                      "num_experts_per_tok": 2}))
    save_file({"model.layers.0.mlp.expert_bank": torch.zeros(8, 4)},
              str(tmp_path / "model.layers.0.safetensors"))
    with pytest.raises(RuntimeError, match="found NONE"):
        ExpertOffsetIndex(str(tmp_path)).build(write_cache=False)


def test_dense_checkpoint_indexes_nothing_quietly(tmp_path):
    (tmp_path / "config.json").write_text(json.dumps({"hidden_size": 8}))
    save_file({"model.layers.0.mlp.up.weight": torch.zeros(4, 4)},
              str(tmp_path / "model.layers.0.safetensors"))
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build(write_cache=False)
    assert idx.index == {}


def test_expert_count_fields_in_order():
    assert ExpertOffsetIndex.expert_count_in({"num_experts_per_tok": 10,
                                              "num_experts": 512}) == 512
    assert ExpertOffsetIndex.expert_count_in({"n_routed_experts": 256}) == 256
    assert ExpertOffsetIndex.expert_count_in({"num_experts": True}) is None


def test_incomplete_checkpoint_raises(tmp_path):
    save_file({"a": torch.zeros(1)}, str(tmp_path / "model-00001-of-00002.safetensors"))
    with pytest.raises(RuntimeError, match="incomplete checkpoint"):
        assert_checkpoint_complete(tmp_path)
    (tmp_path / "model.safetensors.index.json").write_text(
        json.dumps({"weight_map": {"a": "model-00003.safetensors"}}))
    save_file({"a": torch.zeros(1)}, str(tmp_path / "model-00002-of-00002.safetensors"))
    with pytest.raises(RuntimeError, match="not present"):
        assert_checkpoint_complete(tmp_path)


# ── loading ─────────────────────────────────────────────────────────────────────────────

def _compressed_tensors_layer(tmp_path, layer, E, H, I, bits=4, gs=32, seed=0):
    """A compressed-tensors pack-quantized MoE layer shard; returns {expert: by_role}."""
    g = torch.Generator().manual_seed(seed)
    tensors, by_expert = {}, {}
    for e in range(E):
        by_role = {}
        for role, name, shape in (("gate", "gate_proj", (I, H)), ("down", "down_proj", (H, I)),
                                  ("up", "up_proj", (I, H))):
            w = (torch.randn(shape, generator=g) * 0.05).bfloat16()
            packed, scale = quantize_pack(w, bits, gs, torch.bfloat16)
            comps = {"weight_packed": packed, "weight_scale": scale,
                     "weight_shape": torch.tensor(list(shape))}
            by_role[role] = comps
            for c, t in comps.items():
                tensors[f"{layer}.mlp.experts.{e}.{name}.{c}"] = t
        by_expert[e] = by_role
    tensors[f"{layer}.mlp.gate.weight"] = torch.randn(E, H, generator=g).bfloat16()
    save_file(tensors, str(tmp_path / f"{layer}.safetensors"))
    return by_expert


def test_loaded_tensors_are_the_written_ones(tmp_path):
    by_expert = _compressed_tensors_layer(tmp_path, "model.layers.0", 3, 64, 32)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    for e, by_role in by_expert.items():
        got = load_expert_tensors(idx, "model.layers.0", e)
        assert len(got) == 9
        for key, t in got.items():
            role = {"gate_proj": "gate", "down_proj": "down", "up_proj": "up"}[key.split(".")[-2]]
            want = by_role[role][key.split(".")[-1]]
            assert t.dtype == want.dtype and torch.equal(t, want)


def test_resident_blobs_equal_blobs_built_in_memory(tmp_path):
    by_expert = _compressed_tensors_layer(tmp_path, "model.layers.0", 4, 64, 64, seed=3)
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build()
    blobs = load_resident_experts(idx, "model.layers.0", "cpu")
    assert sorted(blobs) == [0, 1, 2, 3]
    for e, by_role in by_expert.items():
        want = build_expert_blob(by_role)
        assert blobs[e]["geom"] == want["geom"]
        for k in ("packed", "scale"):
            assert torch.equal(blobs[e]["flat"][k], want["flat"][k])


def test_spans_merge_touching_ranges(tmp_path):
    _compressed_tensors_layer(tmp_path, "model.layers.0", 1, 64, 32)
    header, start = read_header(tmp_path / "model.layers.0.safetensors")
    idx = ExpertOffsetIndex(str(tmp_path))
    idx.build(write_cache=False)
    from vaayu_amd.expert_offset_index import _spans
    spans = _spans(idx.get_expert_offsets("model.layers.0", 0))
    assert sum(len(k) for *_ab, k in spans) == 9
    assert len(spans) < 9                  # safetensors packs one expert's tensors together
