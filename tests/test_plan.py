"""Plan byte arithmetic.

The expected numbers are the reference's own (tests/test_plan.py:11-95 of
lianghan224-cloud/Cascade-LLM) plus the per-unit byte counts of the 8B
geometry; a layout drift would break device slots and checkpoint loading.
"""

from layer_streaming.plan import (
    ALIGNMENT_BYTES,
    Granularity,
    MIB,
    build_llama31_8b_plan,
)


def test_matrix_is_default_and_uses_largest_projection():
    plan = build_llama31_8b_plan()
    assert plan.granularity == Granularity.MATRIX
    assert len(plan.units) == 32 * 7
    assert plan.slot_bytes == 112 * MIB
    assert plan.two_slot_bytes == 224 * MIB
    assert plan.stream_bytes_per_token == 32 * 416 * MIB


def test_layer_plan_allocates_two_whole_layer_slots():
    plan = build_llama31_8b_plan("layer")
    assert len(plan.units) == 32
    assert plan.slot_bytes == 416 * MIB
    assert plan.two_slot_bytes == 832 * MIB


def test_matrix_group_uses_four_whole_matrix_groups_per_layer():
    plan = build_llama31_8b_plan("matrix_group")
    assert plan.granularity == Granularity.MATRIX_GROUP
    assert len(plan.units) == 32 * 4
    assert [u.operation for u in plan.units[:4]] == [
        "qkv", "o_proj", "gate_up", "down_proj"]
    assert plan.slot_bytes == 224 * MIB
    assert plan.two_slot_bytes == 448 * MIB
    assert [u.nbytes for u in plan.units[:4]] == [
        50331648, 33554432, 234881024, 117440512]
    assert plan.stream_bytes_per_token == 13958643712


def test_separate_embedding_and_head_are_resident():
    plan = build_llama31_8b_plan("matrix")
    keys = {item.tensor.key for item in plan.resident}
    assert "model.embed_tokens.weight" in keys
    assert "lm_head.weight" in keys
    assert plan.resident_bytes == int(2004.5078125 * MIB)
    assert plan.aliases == {}


def test_tied_head_alias_does_not_duplicate_gpu_memory():
    untied = build_llama31_8b_plan("matrix", tie_word_embeddings=False)
    tied = build_llama31_8b_plan("matrix", tie_word_embeddings=True)
    assert tied.aliases["lm_head.weight"] == "model.embed_tokens.weight"
    assert untied.resident_bytes - tied.resident_bytes == 1002 * MIB


def test_matrix_plan_saves_608_mib_of_device_slots():
    layer = build_llama31_8b_plan("layer")
    matrix = build_llama31_8b_plan("matrix")
    assert layer.two_slot_bytes - matrix.two_slot_bytes == 608 * MIB
    assert abs((1.0 - matrix.two_slot_bytes / layer.two_slot_bytes)
               - 0.7307692307692308) < 1e-15


def test_streamed_vocab_is_cpu_only_and_uses_128_mib_chunks():
    plan = build_llama31_8b_plan("matrix", stream_vocab=True)
    resident = {item.tensor.key for item in plan.resident}
    host_only = {item.tensor.key for item in plan.host_only}
    assert "model.embed_tokens.weight" not in resident
    assert "lm_head.weight" not in resident
    assert host_only == {"model.embed_tokens.weight", "lm_head.weight"}
    assert plan.resident_bytes == 532480
    assert plan.vocab.chunk_bytes == 128 * MIB
    assert plan.vocab.chunk_rows == 16384
    assert plan.vocab.chunk_count == 8
    assert plan.slot_bytes == 128 * MIB
    assert plan.two_slot_bytes == 256 * MIB
    assert plan.host_arena_bytes == 16060522496
    assert plan.aliases == {}
    assert plan.vocab.chunk_bounds(7) == (7 * 16384, 128256)
    assert 128256 - 7 * 16384 == 13568


def test_matrix_group_streamed_vocab_slot_is_gate_up():
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=True)
    assert plan.slot_bytes == 224 * MIB
    assert plan.host_arena_bytes == 16060522496


def test_every_tensor_is_aligned_disjoint_and_inside_the_arena():
    for granularity in Granularity:
        for stream_vocab in (False, True):
            plan = build_llama31_8b_plan(granularity, stream_vocab=stream_vocab)
            spans = []
            for key, spec in plan.tensors.items():
                if spec.alias_of:
                    continue
                start = plan.tensor_host_offset(key)
                assert (start * 2) % ALIGNMENT_BYTES == 0
                spans.append((start, start + spec.numel))
            spans.sort()
            for (_, end), (start, _) in zip(spans, spans[1:]):
                assert end <= start
            assert spans[-1][1] <= plan.host_arena_elements
            for unit in plan.units:
                assert unit.elements * 2 <= plan.slot_bytes
                for piece in unit.pieces:
                    assert piece.unit_offset_elements + piece.tensor.numel <= unit.elements


def test_unit_pieces_are_contiguous_projection_blocks():
    # q|k|v and gate|up are back to back inside their units: the fused
    # kernels may treat them as one [6144, 4096] / [28672, 4096] matrix
    plan = build_llama31_8b_plan("matrix_group")
    qkv, _, gate_up, _ = plan.units[:4]
    assert [p.unit_offset_elements for p in qkv.pieces] == [0, 4096 * 4096, 5120 * 4096]
    assert [p.unit_offset_elements for p in gate_up.pieces] == [0, 14336 * 4096]


def test_as_dict_round_trip_fields():
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=True)
    d = plan.as_dict()
    assert d["transfer_unit_count"] == 128
    assert d["slot_bytes"] == 224 * MIB
    assert d["vocab"]["chunk_count"] == 8
    assert d["units"][0]["pieces"][1]["unit_offset_bytes"] == 4096 * 4096 * 2
    assert d["granularity"] == "matrix_group"


def test_fewer_layers_keep_the_layout_rules():
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=True, num_layers=2)
    assert len(plan.units) == 8
    assert plan.num_layers == 2
    assert plan.stream_bytes_per_token == 2 * 436207616
