"""Flags of tools/run_llama31.py on the CPU: the reference CLI's flags and
defaults (tools/run_llama31.py:27-60 in the reference), plus --decode-graph,
which needs the resident LM head."""

import pytest


def parse(*argv):
    from tools import run_llama31

    return run_llama31.parse_args(list(argv))


def test_reference_flags_and_defaults():
    a = parse("--random-init")
    assert (a.weight_store, a.granularity, a.vocab_mode) == (
        "full_pinned", "matrix_group", "streamed")
    assert a.max_new_tokens == 8 and a.top_k == 10 and a.device == "cuda:0"
    assert a.prompt == "The meaning of life is" and not a.decode_graph
    b = parse("--random-init", "--weight-store", "pinned_staging", "--granularity",
              "matrix", "--vocab-mode", "resident", "--top-k", "5",
              "--max-new-tokens", "3")
    assert (b.weight_store, b.granularity, b.vocab_mode, b.top_k,
            b.max_new_tokens) == ("pinned_staging", "matrix", "resident", 5, 3)


def test_bad_combinations_are_refused():
    with pytest.raises(SystemExit):
        parse()  # neither --checkpoint nor --random-init
    with pytest.raises(SystemExit):
        parse("--random-init", "--decode-graph")  # streamed vocabulary
    with pytest.raises(SystemExit):
        parse("--random-init", "--granularity", "tensor")
    assert parse("--random-init", "--decode-graph", "--vocab-mode",
                 "resident").decode_graph
