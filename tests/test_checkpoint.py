"""Checkpoint loading on the CPU: safetensors files written by the
safetensors library itself (the published format) are read into the arena
by the store's own header parser.  Pins: every dtype path (bf16 read in
place, f16 / f32 rounded to bf16 like ``tensor.to(torch.bfloat16)``), a
sharded index, a direct file path, piecewise conversion, and the error
types the reference raises (weight_store.py:20-38, :109-171): KeyError for
missing tensors, ValueError for shapes / malformed files, FileNotFoundError
for no checkpoint.  Nothing is written to the arena when a check fails."""

import json
import struct

import pytest
import torch
from safetensors.torch import save_file

from layer_streaming import checkpoint
from layer_streaming.plan import (
    ModelPlan,
    ResidentPlacement,
    TensorSpec,
    TransferUnit,
    UnitPiece,
)
from layer_streaming.weight_store import create_weight_store


def plan_of(shapes):
    """A plan with one streamed unit per tensor, packed in order."""

    tensors, units, offset = {}, [], 0
    for key, shape in shapes.items():
        spec = TensorSpec(key, shape)
        tensors[key] = spec
        units.append(TransferUnit(unit_id=key, layer_index=0, operation="q_proj",
                                  pieces=(UnitPiece(spec, 0),), elements=spec.numel,
                                  host_offset_elements=offset))
        offset += -(-spec.numel // 128) * 128
    return ModelPlan(model_id="tiny", granularity="matrix", tensors=tensors,
                     units=tuple(units), resident=(), aliases={},
                     host_arena_elements=offset, resident_arena_elements=0,
                     slot_elements=max(u.elements for u in units))


def cpu_factory(n, **kw):
    kw.pop("pin_memory")
    return torch.zeros(n, **kw)


SHAPES = {"a.weight": (3, 5), "b.weight": (64,), "c.weight": (7, 130)}


def values(seed):
    gen = torch.Generator().manual_seed(seed)
    return {k: torch.randn(s, generator=gen) for k, s in SHAPES.items()}


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
def test_every_dtype_lands_as_bf16(tmp_path, dtype):
    src = values(1)
    save_file({k: v.to(dtype) for k, v in src.items()}, str(tmp_path / "model.safetensors"))
    store = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    store.load_checkpoint(tmp_path)
    assert store.loaded
    for key, value in src.items():
        assert torch.equal(store.tensor(key), value.to(dtype).to(torch.bfloat16)), key


def test_piecewise_conversion_matches_whole(tmp_path, monkeypatch):
    src = values(2)
    save_file(src, str(tmp_path / "model.safetensors"))
    monkeypatch.setattr(checkpoint, "_CONVERT_PIECE_BYTES", 12)  # 3 fp32 a piece
    store = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    store.load_checkpoint(tmp_path)
    for key, value in src.items():
        assert torch.equal(store.tensor(key), value.to(torch.bfloat16)), key


def test_sharded_index_and_direct_file(tmp_path):
    src = values(3)
    save_file({"a.weight": src["a.weight"].bfloat16()}, str(tmp_path / "part-1.safetensors"))
    # part 2 also holds a stale copy of a.weight that the index does not own
    save_file({"b.weight": src["b.weight"].bfloat16(),
               "c.weight": src["c.weight"].bfloat16(),
               "a.weight": torch.zeros(3, 5).bfloat16()},
              str(tmp_path / "part-2.safetensors"))
    (tmp_path / "model.safetensors.index.json").write_text(json.dumps({
        "metadata": {}, "weight_map": {"a.weight": "part-1.safetensors",
                                       "b.weight": "part-2.safetensors",
                                       "c.weight": "part-2.safetensors"}}))
    store = create_weight_store(plan_of(SHAPES), "pinned_staging", tensor_factory=cpu_factory)
    store.load_checkpoint(tmp_path)
    for key, value in src.items():
        assert torch.equal(store.tensor(key), value.bfloat16()), key
    store.close()
    single = tmp_path / "one"
    single.mkdir()
    save_file({k: v.bfloat16() for k, v in src.items()}, str(single / "w.safetensors"))
    other = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    other.load_checkpoint(single / "w.safetensors")
    assert torch.equal(other.tensor("c.weight"), src["c.weight"].bfloat16())


def test_checks_run_before_any_byte_is_written(tmp_path):
    src = values(4)
    bad = dict(src)
    bad["c.weight"] = torch.zeros(130, 7)  # transposed
    save_file(bad, str(tmp_path / "model.safetensors"))
    store = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    with pytest.raises(ValueError, match="c.weight"):
        store.load_checkpoint(tmp_path)
    assert not store.loaded
    assert int(store.arena.float().abs().sum()) == 0


def test_missing_tensors_and_bad_dtype(tmp_path):
    src = values(5)
    save_file({"a.weight": src["a.weight"]}, str(tmp_path / "model.safetensors"))
    store = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    with pytest.raises(KeyError, match="2 tensor"):
        store.load_checkpoint(tmp_path)
    ints = tmp_path / "ints"
    ints.mkdir()
    save_file({k: torch.zeros(s, dtype=torch.int32) for k, s in SHAPES.items()},
              str(ints / "model.safetensors"))
    with pytest.raises(ValueError, match="dtype"):
        store.load_checkpoint(ints)
    index_only = tmp_path / "index"
    index_only.mkdir()
    (index_only / "model.safetensors.index.json").write_text(json.dumps({"weight_map": []}))
    with pytest.raises(ValueError, match="weight_map"):
        store.load_checkpoint(index_only)
    with pytest.raises(FileNotFoundError):
        store.load_checkpoint(tmp_path / "nothing")


def test_malformed_headers_are_refused(tmp_path):
    store = create_weight_store(plan_of(SHAPES), "full_pinned", tensor_factory=cpu_factory)
    path = tmp_path / "model.safetensors"
    path.write_bytes(b"\x01\x02")
    with pytest.raises(ValueError, match="shorter"):
        store.load_checkpoint(tmp_path)
    path.write_bytes(struct.pack("<Q", 1 << 40) + b"{}")
    with pytest.raises(ValueError, match="runs past"):
        store.load_checkpoint(tmp_path)
    header = json.dumps({"a.weight": {"dtype": "BF16", "shape": [3, 5],
                                      "data_offsets": [0, 30000]}}).encode()
    path.write_bytes(struct.pack("<Q", len(header)) + header + bytes(30))
    with pytest.raises(ValueError, match="outside the file"):
        store.load_checkpoint(tmp_path)
    header = b"[1, 2]"
    path.write_bytes(struct.pack("<Q", len(header)) + header)
    with pytest.raises(ValueError, match="malformed"):
        store.load_checkpoint(tmp_path)


def test_header_parser_agrees_with_the_library(tmp_path):
    from safetensors import safe_open

    src = values(6)
    save_file(src, str(tmp_path / "x.safetensors"), metadata={"format": "pt"})
    records = checkpoint.describe_checkpoint(tmp_path / "x.safetensors")
    assert sorted(records) == sorted(src)
    with safe_open(str(tmp_path / "x.safetensors"), framework="pt") as f:
        for key in src:
            assert list(records[key].shape) == list(f.get_slice(key).get_shape())
            assert records[key].end - records[key].begin == src[key].numel() * 4
