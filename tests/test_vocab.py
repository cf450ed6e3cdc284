"""merge_topk and the streamed top-k contract (CPU).

The known answer is the reference's (tests/test_vocab.py:8-34): logits
[-2, 7, 1, 3, 9, -1, 8, 4] streamed in chunks of 3 with k = 3 give values
[9, 8, 7] at indices [4, 6, 1].  Beyond it, brute force: the online merge
equals a stable descending sort of the whole vector, including ties.
"""

import random

import pytest
import torch

from layer_streaming.vocab import merge_topk
from oracle import llama_oracle as ref


@pytest.mark.parametrize("merge", [merge_topk, ref.merge_topk])
def test_online_merge_matches_full_topk(merge):
    logits = torch.tensor([[[-2.0, 7.0, 1.0, 3.0, 9.0, -1.0, 8.0, 4.0]]])
    values = indices = None
    for start in (0, 3, 6):
        part = logits[..., start : start + 3]
        lv, li = torch.topk(part, k=min(3, part.shape[-1]), dim=-1)
        if merge is ref.merge_topk:
            lv, li = lv.reshape(-1), li.reshape(-1)
        values, indices = merge(values, indices, lv, li + start, top_k=3)
    assert values.reshape(-1).tolist() == [9.0, 8.0, 7.0]
    assert indices.reshape(-1).tolist() == [4, 6, 1]


def brute_topk(values, k):
    order = sorted(range(len(values)), key=lambda i: (-values[i], i))[:k]
    return [values[i] for i in order], order


@pytest.mark.parametrize("seed", range(6))
def test_streamed_merge_equals_brute_force_with_ties(seed):
    rng = random.Random(seed)
    n = rng.randint(1, 300)
    # few distinct values -> many ties
    vals = [float(rng.randint(-5, 5)) for _ in range(n)]
    logits = torch.tensor(vals)
    k = rng.randint(1, 12)
    chunk = rng.randint(1, 50)
    values = indices = None
    for start in range(0, n, chunk):
        part = logits[start : start + chunk]
        lv, li = ref.topk(part, min(k, part.numel()))
        values, indices = merge_topk(values, indices, lv, li + start, k)
    bv, bi = brute_topk(vals, k)
    assert values.tolist() == bv
    assert indices.tolist() == bi
    ov, oi = brute_topk(vals, k)
    rv, ri = ref.topk(logits, k)
    assert rv.tolist() == ov and ri.tolist() == oi


def test_oracle_topk_is_stable_sort():
    logits = torch.tensor([1.0, 3.0, 3.0, 2.0, 3.0, -1.0])
    v, i = ref.topk(logits, 4)
    assert i.tolist() == [1, 2, 4, 3]
    assert v.tolist() == [3.0, 3.0, 3.0, 2.0]


def test_oracle_streamed_lm_head_equals_full_topk():
    gen = torch.Generator().manual_seed(3)
    w = (torch.randn(1000, 64, generator=gen) * 0.1).to(torch.bfloat16)
    h = torch.randn(64, generator=gen).to(torch.bfloat16)
    v, i, logits = ref.streamed_lm_head(h, w, 128, 10)
    fv, fi = ref.topk(ref.lm_head_logits(h, w), 10)
    assert torch.equal(i, fi) and torch.equal(v, fv)
    assert logits.shape == (1000,)


def test_streamed_vocabulary_needs_two_device_slots():
    # reference vocab.py:63-64: the LM-head chunks alternate over two slots,
    # so a single-slot transformer runtime is refused before any allocation
    from types import SimpleNamespace

    from layer_streaming.plan import build_llama31_8b_plan
    from layer_streaming.vocab import VocabStreamingRuntime

    plan = build_llama31_8b_plan("matrix_group", num_layers=1, stream_vocab=True)
    one_slot = SimpleNamespace(device_slots=[torch.empty(plan.slot_elements,
                                                         dtype=torch.bfloat16,
                                                         device="meta")])
    with pytest.raises(ValueError, match="two device slots"):
        VocabStreamingRuntime(plan, store=None, transformer_runtime=one_slot)


@pytest.mark.parametrize("row_buffer", [1, 3, 256])
@pytest.mark.parametrize("count", [1, 5, 300])
def test_embedding_rows_through_alternating_buffer_halves(monkeypatch, row_buffer,
                                                          count):
    # the gathered rows equal the table's; group g reuses a half only after
    # waiting for the copy of group g - 2 (the last one that read it)
    from types import SimpleNamespace

    from layer_streaming import _hip
    from layer_streaming import vocab as vocab_mod
    from layer_streaming.plan import build_llama31_8b_plan
    from layer_streaming.weight_store import WeightStoreMode

    log = []

    class Event:
        def __init__(self, enable_timing=False):
            self.id = len([e for e in log if e[0] == "new"])
            log.append(("new", self.id))

        def record(self, stream=None):
            log.append(("record", self.id))

        def synchronize(self):
            log.append(("sync", self.id))

    def copy(dst, src, nbytes, stream):
        dst.view(-1)[: nbytes // 2].copy_(src.reshape(-1)[: nbytes // 2])
        log.append(("copy", src.data_ptr()))

    monkeypatch.setattr(_hip, "load", lambda: None)
    monkeypatch.setattr(_hip, "HipEvent", Event)
    monkeypatch.setattr(_hip, "memcpy_h2d_async", copy)
    monkeypatch.setattr(vocab_mod, "_pinned_rows",
                        lambda n, w: torch.empty((n, w), dtype=torch.bfloat16))
    monkeypatch.setattr(vocab_mod.torch.cuda, "current_stream", lambda device=None: None)
    plan = build_llama31_8b_plan("matrix_group", num_layers=1, stream_vocab=True)
    gen = torch.Generator().manual_seed(count)
    table = torch.randn(400, 4096, generator=gen).to(torch.bfloat16)
    store = SimpleNamespace(mode=WeightStoreMode.FULL_PINNED,
                            tensor=lambda key: table)
    slots = [torch.empty(plan.slot_elements, dtype=torch.bfloat16, device="meta")
             for _ in range(2)]
    runtime = SimpleNamespace(device_slots=slots, device=torch.device("cpu"),
                              copy_stream=None, compute_stream=None,
                              coordinator=None, stage_call_ahead=lambda: None)
    vocab = vocab_mod.VocabStreamingRuntime(plan, store, runtime,
                                            embedding_staging_rows=row_buffer)
    ids = torch.randint(0, 400, (1, count), generator=gen)
    del log[:]
    out = vocab.embedding(ids)
    assert out.shape == (1, count, 4096)
    assert torch.equal(out[0], table[ids[0]])
    halves = len(vocab._rows_free)
    assert halves == min(2, row_buffer)
    group = max(1, row_buffer // 2)
    groups = -(-count // group)
    sources = [e[1] for e in log if e[0] == "copy"]
    assert len(sources) == groups
    assert len(set(sources)) == min(groups, halves)
    waits = [e for e in log if e[0] in ("sync", "record")]
    for n in range(groups):
        half = vocab._rows_free[n % halves].id
        assert waits[2 * n] == ("sync", half) and waits[2 * n + 1] == ("record", half)


def test_release_hook_holds_the_vocabulary_runtime_weakly(monkeypatch):
    # The transformer runtime's release hook forwards to the vocabulary
    # runtime while it lives; dropping the vocabulary runtime frees it by
    # reference counting alone (no cycle through the hook), after which the
    # hook returns False and the transformer runtime prefetches its next
    # call into the slot instead.
    import gc
    import weakref
    from types import SimpleNamespace

    from layer_streaming import _hip
    from layer_streaming import vocab as vocab_mod
    from layer_streaming.plan import build_llama31_8b_plan
    from layer_streaming.weight_store import WeightStoreMode

    class Event:
        def __init__(self, enable_timing=False):
            pass

    released = []
    monkeypatch.setattr(_hip, "load", lambda: None)
    monkeypatch.setattr(_hip, "HipEvent", Event)
    monkeypatch.setattr(vocab_mod, "_pinned_rows",
                        lambda n, w: torch.empty((n, w), dtype=torch.bfloat16))
    monkeypatch.setattr(vocab_mod.VocabStreamingRuntime, "_copy_first_chunk",
                        lambda self, slot: released.append(slot))
    plan = build_llama31_8b_plan("matrix_group", num_layers=1, stream_vocab=True)
    table = torch.zeros(8, 4096, dtype=torch.bfloat16)
    store = SimpleNamespace(mode=WeightStoreMode.FULL_PINNED, tensor=lambda key: table)
    slots = [torch.empty(plan.slot_elements, dtype=torch.bfloat16, device="meta")
             for _ in range(2)]
    runtime = SimpleNamespace(device_slots=slots, device=torch.device("cpu"),
                              copy_stream=None, compute_stream=None,
                              coordinator=None, stage_call_ahead=lambda: None)
    vocab = vocab_mod.VocabStreamingRuntime(plan, store, runtime)
    assert runtime.release_hook(1) is None
    assert released == [1]
    alive = weakref.ref(vocab)
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        del vocab
        assert alive() is None
    finally:
        if was_enabled:
            gc.enable()
    assert runtime.release_hook(0) is False
    assert released == [1]
