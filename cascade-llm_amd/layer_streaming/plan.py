"""Static bf16 layout of a Llama-3.1-8B-shaped model and its transfer units.

The data model (TensorSpec, UnitPiece, TransferUnit, ResidentPlacement,
HostPlacement, VocabPlan, ModelPlan) and the byte layout are the reference's
(layer_streaming/plan.py:10-457): every tensor and every unit starts on a
256-byte boundary of one packed host arena, units are cut at one of three
granularities, norms are device-resident, and the vocabulary (embedding and
LM head) is either resident or host-only and streamed in row chunks.  The
layout is an interface -- device slots, arena offsets and checkpoint loading
all depend on it -- so offsets must agree with the reference byte for byte.

``build_llama31_8b_plan`` additionally accepts ``num_layers`` (default 32, the
only value the reference supports) so tests can run full-width models with
fewer decoder layers.
"""

from dataclasses import dataclass
from enum import Enum
from math import prod
from typing import Mapping, Optional, Tuple

MIB = 1024 * 1024
BF16_BYTES = 2
ALIGNMENT_BYTES = 256
_ALIGN_ELEMENTS = ALIGNMENT_BYTES // BF16_BYTES

# Llama-3.1-8B geometry (plan.py:260-264).
HIDDEN = 4096
INTERMEDIATE = 14336
KV_WIDTH = 1024
VOCAB = 128256
LAYERS = 32

# (name, shape, block) of the seven streamed projections of one layer, in
# transfer order (plan.py:265-273).
PROJECTIONS = (
    ("q_proj", (HIDDEN, HIDDEN), "self_attn"),
    ("k_proj", (KV_WIDTH, HIDDEN), "self_attn"),
    ("v_proj", (KV_WIDTH, HIDDEN), "self_attn"),
    ("o_proj", (HIDDEN, HIDDEN), "self_attn"),
    ("gate_proj", (INTERMEDIATE, HIDDEN), "mlp"),
    ("up_proj", (INTERMEDIATE, HIDDEN), "mlp"),
    ("down_proj", (HIDDEN, INTERMEDIATE), "mlp"),
)

# matrix_group units: (operation, first projection, end projection).
MATRIX_GROUPS = (
    ("qkv", 0, 3),
    ("o_proj", 3, 4),
    ("gate_up", 4, 6),
    ("down_proj", 6, 7),
)


class Granularity(str, Enum):
    """How weights are cut into transfer units: one projection, one
    projection group, or one whole decoder layer per copy."""

    MATRIX = "matrix"
    MATRIX_GROUP = "matrix_group"
    LAYER = "layer"


def align_elements(count, alignment=_ALIGN_ELEMENTS):
    """Round an element count up to the arena alignment."""

    return -(-count // alignment) * alignment


@dataclass(frozen=True)
class TensorSpec:
    key: str
    shape: Tuple[int, ...]
    resident: bool = False
    alias_of: Optional[str] = None

    @property
    def numel(self):
        return prod(self.shape)

    @property
    def nbytes(self):
        return self.numel * BF16_BYTES


@dataclass(frozen=True)
class UnitPiece:
    tensor: TensorSpec
    unit_offset_elements: int


@dataclass(frozen=True)
class TransferUnit:
    unit_id: str
    layer_index: int
    operation: str
    pieces: Tuple[UnitPiece, ...]
    elements: int
    host_offset_elements: int

    @property
    def nbytes(self):
        return self.elements * BF16_BYTES


@dataclass(frozen=True)
class ResidentPlacement:
    tensor: TensorSpec
    host_offset_elements: int
    device_offset_elements: int


@dataclass(frozen=True)
class HostPlacement:
    """A tensor that lives only in the host arena (the streamed vocabulary)."""

    tensor: TensorSpec
    host_offset_elements: int


@dataclass(frozen=True)
class VocabPlan:
    """Embedding and LM head kept on the host: the row chunks the LM head
    streams in and the keys both tables are read under."""

    embedding_key: str
    lm_head_key: str
    vocab_size: int
    hidden_size: int
    chunk_rows: int
    chunk_elements: int
    chunk_bytes: int
    chunk_count: int

    def chunk_bounds(self, chunk_index):
        """(first_row, end_row) of one vocabulary chunk."""

        first = chunk_index * self.chunk_rows
        return first, min(first + self.chunk_rows, self.vocab_size)


@dataclass(frozen=True)
class ModelPlan:
    model_id: str
    granularity: Granularity
    tensors: Mapping[str, TensorSpec]
    units: Tuple[TransferUnit, ...]
    resident: Tuple[ResidentPlacement, ...]
    aliases: Mapping[str, str]
    host_arena_elements: int
    resident_arena_elements: int
    slot_elements: int
    dtype_bytes: int = BF16_BYTES
    slot_count: int = 2
    host_only: Tuple[HostPlacement, ...] = ()
    vocab: Optional[VocabPlan] = None

    @property
    def slot_bytes(self):
        return self.slot_elements * self.dtype_bytes

    @property
    def two_slot_bytes(self):
        return self.slot_count * self.slot_bytes

    @property
    def stream_bytes_per_token(self):
        return sum(unit.nbytes for unit in self.units)

    @property
    def resident_bytes(self):
        return self.resident_arena_elements * self.dtype_bytes

    @property
    def host_arena_bytes(self):
        return self.host_arena_elements * self.dtype_bytes

    @property
    def num_layers(self):
        return 1 + max((unit.layer_index for unit in self.units), default=-1)

    def _host_offsets(self):
        cached = self.__dict__.get("_offset_cache")
        if cached is None:
            cached = {}
            for unit in self.units:
                for piece in unit.pieces:
                    cached[piece.tensor.key] = (
                        unit.host_offset_elements + piece.unit_offset_elements
                    )
            for placement in tuple(self.resident) + tuple(self.host_only):
                cached.setdefault(
                    placement.tensor.key, placement.host_offset_elements
                )
            # frozen dataclass: cache through the instance dict directly
            object.__setattr__(self, "_offset_cache", cached)
        return cached

    def tensor_host_offset(self, key):
        offsets = self._host_offsets()
        if key in offsets:
            return offsets[key]
        target = self.aliases.get(key)
        if target is not None:
            return self.tensor_host_offset(target)
        raise KeyError(key)

    def tensor_index(self, key):
        """Position of ``key`` in plan order (seeds the random-init filler)."""

        for index, name in enumerate(self.tensors):
            if name == key:
                return index
        raise KeyError(key)

    def as_dict(self):
        def shape(spec):
            return list(spec.shape)

        vocab = None
        if self.vocab is not None:
            vocab = {
                "embedding_key": self.vocab.embedding_key,
                "lm_head_key": self.vocab.lm_head_key,
                "vocab_size": self.vocab.vocab_size,
                "hidden_size": self.vocab.hidden_size,
                "chunk_rows": self.vocab.chunk_rows,
                "chunk_bytes": self.vocab.chunk_bytes,
                "chunk_count": self.vocab.chunk_count,
            }
        return {
            "model_id": self.model_id,
            "granularity": Granularity(self.granularity).value,
            "dtype": "torch.bfloat16",
            "dtype_bytes": self.dtype_bytes,
            "transfer_unit_count": len(self.units),
            "stream_bytes_per_token": self.stream_bytes_per_token,
            "slot_count": self.slot_count,
            "slot_bytes": self.slot_bytes,
            "two_slot_bytes": self.two_slot_bytes,
            "resident_bytes": self.resident_bytes,
            "host_arena_bytes": self.host_arena_bytes,
            "aliases": dict(self.aliases),
            "vocab": vocab,
            "units": [
                {
                    "unit_id": unit.unit_id,
                    "layer_index": unit.layer_index,
                    "operation": unit.operation,
                    "bytes": unit.nbytes,
                    "pieces": [
                        {
                            "key": piece.tensor.key,
                            "shape": shape(piece.tensor),
                            "unit_offset_bytes": piece.unit_offset_elements
                            * self.dtype_bytes,
                        }
                        for piece in unit.pieces
                    ],
                }
                for unit in self.units
            ],
            "resident": [
                {
                    "key": item.tensor.key,
                    "shape": shape(item.tensor),
                    "bytes": item.tensor.nbytes,
                    "device_offset_bytes": item.device_offset_elements
                    * self.dtype_bytes,
                }
                for item in self.resident
            ],
            "host_only": [
                {
                    "key": item.tensor.key,
                    "shape": shape(item.tensor),
                    "bytes": item.tensor.nbytes,
                    "host_offset_bytes": item.host_offset_elements
                    * self.dtype_bytes,
                }
                for item in self.host_only
            ],
        }


class _Arena:
    """Bump allocator over element offsets with 256-byte alignment."""

    def __init__(self):
        self.cursor = 0

    def take(self, elements):
        start = align_elements(self.cursor)
        self.cursor = start + elements
        return start


def _pack_unit(arena, unit_id, layer_index, operation, tensors):
    pieces = []
    inner = _Arena()
    for spec in tensors:
        pieces.append(UnitPiece(spec, inner.take(spec.numel)))
    elements = align_elements(inner.cursor)
    return TransferUnit(
        unit_id=unit_id,
        layer_index=layer_index,
        operation=operation,
        pieces=tuple(pieces),
        elements=elements,
        host_offset_elements=arena.take(elements),
    )


def projection_key(layer_index, operation):
    """Checkpoint key of one projection (llama31.py:156-167)."""

    for name, _, block in PROJECTIONS:
        if name == operation:
            return "model.layers.{}.{}.{}.weight".format(
                layer_index, block, name
            )
    raise ValueError("unknown projection {}".format(operation))


def build_llama31_8b_plan(
    granularity=Granularity.MATRIX,
    tie_word_embeddings=False,
    stream_vocab=False,
    vocab_chunk_bytes=128 * MIB,
    num_layers=LAYERS,
):
    """Build the packed bf16 plan for the Llama-3.1-8B geometry.

    Mirrors reference plan.py:246-457.  ``tie_word_embeddings`` aliases
    ``lm_head.weight`` to the embedding (only for checkpoints that omit the
    head); ``stream_vocab`` keeps embedding and head host-only and cuts the
    head into chunks of ``vocab_chunk_bytes`` (whole rows).
    """

    granularity = Granularity(granularity)
    num_layers = int(num_layers)
    if num_layers < 1:
        raise ValueError("num_layers must be positive")

    specs = {}

    def declare(key, shape, resident=False, alias_of=None):
        specs[key] = TensorSpec(key, tuple(shape), resident, alias_of)
        return specs[key]

    embedding = declare(
        "model.embed_tokens.weight", (VOCAB, HIDDEN), resident=not stream_vocab
    )
    head = declare(
        "lm_head.weight",
        (VOCAB, HIDDEN),
        resident=not stream_vocab,
        alias_of=embedding.key if tie_word_embeddings else None,
    )
    layer_matrices = []
    norms = []
    for layer in range(num_layers):
        layer_matrices.append(
            tuple(
                declare(projection_key(layer, name), shape)
                for name, shape, _ in PROJECTIONS
            )
        )
        for norm in ("input_layernorm", "post_attention_layernorm"):
            norms.append(
                declare(
                    "model.layers.{}.{}.weight".format(layer, norm),
                    (HIDDEN,),
                    resident=True,
                )
            )
    final_norm = declare("model.norm.weight", (HIDDEN,), resident=True)

    arena = _Arena()
    units = []
    for layer, matrices in enumerate(layer_matrices):
        if granularity == Granularity.LAYER:
            groups = (("layer", matrices),)
            names = ("layer_{:02d}".format(layer),)
        elif granularity == Granularity.MATRIX:
            groups = tuple(
                (name, (matrix,))
                for (name, _, _), matrix in zip(PROJECTIONS, matrices)
            )
            names = tuple(
                "layer_{:02d}.{}".format(layer, op) for op, _ in groups
            )
        else:
            groups = tuple(
                (op, matrices[first:end]) for op, first, end in MATRIX_GROUPS
            )
            names = tuple(
                "layer_{:02d}.{}".format(layer, op) for op, _ in groups
            )
        for unit_id, (operation, members) in zip(names, groups):
            units.append(_pack_unit(arena, unit_id, layer, operation, members))

    vocab_tensors = [embedding] + ([] if tie_word_embeddings else [head])
    host_only = []
    resident_specs = list(norms) + [final_norm]
    if stream_vocab:
        for spec in vocab_tensors:
            host_only.append(HostPlacement(spec, arena.take(spec.numel)))
    else:
        resident_specs = vocab_tensors + resident_specs
    device = _Arena()
    resident = tuple(
        ResidentPlacement(spec, arena.take(spec.numel), device.take(spec.numel))
        for spec in resident_specs
    )

    vocab_plan = None
    if stream_vocab:
        row_bytes = HIDDEN * BF16_BYTES
        if int(vocab_chunk_bytes) < row_bytes:
            raise ValueError("vocab chunk must hold at least one row")
        rows = int(vocab_chunk_bytes) // row_bytes
        vocab_plan = VocabPlan(
            embedding_key=embedding.key,
            lm_head_key=head.key,
            vocab_size=VOCAB,
            hidden_size=HIDDEN,
            chunk_rows=rows,
            chunk_elements=rows * HIDDEN,
            chunk_bytes=rows * HIDDEN * BF16_BYTES,
            chunk_count=-(-VOCAB // rows),
        )

    slot_elements = max(unit.elements for unit in units)
    if vocab_plan is not None:
        slot_elements = max(slot_elements, vocab_plan.chunk_elements)
    return ModelPlan(
        model_id="meta-llama/Llama-3.1-8B",
        granularity=granularity,
        tensors=specs,
        units=tuple(units),
        resident=resident,
        aliases={head.key: embedding.key} if tie_word_embeddings else {},
        host_arena_elements=align_elements(arena.cursor),
        resident_arena_elements=align_elements(device.cursor),
        slot_elements=slot_elements,
        host_only=tuple(host_only),
        vocab=vocab_plan,
    )
