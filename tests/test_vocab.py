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
