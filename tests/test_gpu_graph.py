"""Decode steps with a device-held position, and their HIP-graph replay.

Kernel level: cascade_qkv_rope_at_bf16 and cascade_decode_attention_at_bf16
must give, bit for bit, what the host-position entry points give at the same
position / length (the attention's grid follows the capacity and its splits
the length word, so cases whose capacity has more splits than the length
check that the splits past the length's plan contribute exactly nothing);
cascade_decode_step_begin_bf16
must gather, record and advance as declared, and refuse a full history.

Model level: a 2-layer, full-width Llama-3.1-8B-shaped resident model decodes
greedily, first eagerly through the host-position kernels, then from the same
cache state through DecodeGraph.  Every replay's logits and top-k must equal
the eager step's bit for bit; replays are interleaved with eager work and
synchronisations.  The eager path itself is held to the CPU oracle by
test_gpu_model.py, so bit equality carries that parity over.
"""

import pytest
import torch

from layer_streaming import (
    DecodeGraph,
    Llama31Config,
    Llama31DecodeExecutor,
    ResidentDeviceArena,
    ResidentTransformerRuntime,
    build_llama31_8b_plan,
)
from layer_streaming import _hip
from layer_streaming.rope import RopeTable, rope_parameters

pytestmark = pytest.mark.gpu

LAYERS = 2
TOP_K = 10


def _say(*parts):
    print(*parts, flush=True)


# ----------------------------------------------------------------- kernels


@pytest.mark.parametrize("pos,capacity", [(0, 40), (17, 40), (39, 40),
                                          (2100, 2200)])
def test_qkv_at_equals_host_position(gpu_device, pos, capacity):
    dev = torch.device(gpu_device)
    gen = torch.Generator(device=dev).manual_seed(pos)

    def rnd(*shape, std=1.0):
        return (torch.randn(*shape, generator=gen, device=dev) * std).to(torch.bfloat16)

    wq, wk, wv = rnd(4096, 4096, std=0.02), rnd(1024, 4096, std=0.02), rnd(1024, 4096, std=0.02)
    x, norm = rnd(4096), rnd(4096)
    rope = RopeTable(128, rope_parameters(Llama31Config()), dev, capacity)
    stride = capacity * 128
    out = {}
    for mode in ("host", "at"):
        q = torch.zeros(4096, dtype=torch.bfloat16, device=dev)
        kc = torch.zeros(8 * stride, dtype=torch.bfloat16, device=dev)
        vc = torch.zeros_like(kc)
        _say("qkv", mode, "pos", pos, "capacity", capacity)
        if mode == "host":
            cos, sin = rope.row(pos)
            _hip.qkv_rope(wq, wk, wv, x, norm, 1e-5, cos, sin, q,
                          kc[pos * 128:], vc[pos * 128:], stride)
        else:
            length = torch.tensor([pos + 1], dtype=torch.int64, device=dev)
            _hip.qkv_rope_at(wq, wk, wv, x, norm, 1e-5, rope.cos, rope.sin, q,
                             kc, vc, stride, length, capacity)
        torch.cuda.synchronize(dev)
        out[mode] = (q.cpu(), kc.cpu(), vc.cpu())
    for a, b in zip(out["host"], out["at"]):
        assert torch.equal(a, b)
    # only position pos was written
    kc = out["at"][1].view(8, capacity, 128)
    assert kc[:, pos].abs().sum() > 0
    assert kc.abs().sum(-1).count_nonzero() == 8


def test_qkv_at_clamps_a_length_past_capacity(gpu_device):
    dev = torch.device(gpu_device)
    capacity = 40
    wk = (torch.randn(1024, 4096, device=dev) * 0.02).to(torch.bfloat16)
    x = torch.randn(4096, device=dev).to(torch.bfloat16)
    rope = RopeTable(128, rope_parameters(Llama31Config()), dev, capacity)
    stride = capacity * 128
    caches = []
    for word in (capacity, capacity + 9):
        kc = torch.zeros(8 * stride, dtype=torch.bfloat16, device=dev)
        length = torch.tensor([word], dtype=torch.int64, device=dev)
        _say("qkv_at clamp, length word", word)
        _hip.qkv_rope_at(None, wk, None, x, None, 1e-5, rope.cos, rope.sin, None,
                         kc, None, stride, length, capacity)
        caches.append(kc)
    torch.cuda.synchronize(dev)
    assert torch.equal(caches[0].cpu(), caches[1].cpu())


# (splits of the length's plan, of the capacity's): (1, 1), (1, 1), (2, 2),
# (2, 64), then 64 and 64, with rows past the length NaN in the last block
# ((33, 40), (2049, 2080)) and the longer splits of the two plans starting
# at different rows ((2101, 2200), (32769, 34800))
@pytest.mark.parametrize("length,capacity", [(1, 1), (7, 12), (33, 40),
                                             (40, 2200), (2049, 2080),
                                             (2101, 2200), (4100, 4100),
                                             (32769, 34800)])
def test_attention_at_equals_attention(gpu_device, length, capacity):
    dev = torch.device(gpu_device)
    gen = torch.Generator(device=dev).manual_seed(length)
    stride = capacity * 128
    q = torch.randn(4096, generator=gen, device=dev).to(torch.bfloat16)
    kc = torch.randn(8 * stride, generator=gen, device=dev).to(torch.bfloat16)
    vc = torch.randn(8 * stride, generator=gen, device=dev).to(torch.bfloat16)
    if capacity > length:
        # rows past the length must never be read: make them poison
        kc.view(8, capacity, 128)[:, length:] = float("nan")
        vc.view(8, capacity, 128)[:, length:] = float("nan")
    ws = torch.zeros(_hip.attention_workspace_bytes(capacity), dtype=torch.uint8,
                     device=dev)
    host = torch.empty(4096, dtype=torch.bfloat16, device=dev)
    dev_out = torch.empty_like(host)
    _say("attention host length", length)
    _hip.decode_attention(q, kc, vc, stride, length, host, ws, 128 ** -0.5)
    word = torch.tensor([length], dtype=torch.int64, device=dev)
    _say("attention_at length", length, "capacity", capacity)
    _hip.decode_attention_at(q, kc, vc, stride, word, capacity, dev_out, ws,
                             128 ** -0.5)
    torch.cuda.synchronize(dev)
    assert torch.isfinite(dev_out.float()).all()
    assert torch.equal(host.cpu(), dev_out.cpu())


def test_step_begin_gathers_records_and_advances(gpu_device):
    dev = torch.device(gpu_device)
    table = torch.randn(100, 64, device=dev).to(torch.bfloat16)
    history = torch.full((8,), -1, dtype=torch.int64, device=dev)
    length = torch.tensor([3], dtype=torch.int64, device=dev)
    err = torch.zeros(1, dtype=torch.int32, device=dev)
    out = torch.empty(64, dtype=torch.bfloat16, device=dev)
    ids = torch.tensor([[42, 7]], dtype=torch.int64, device=dev)
    _say("step_begin id 42 at length 3")
    _hip.decode_step_begin(table, ids[:, :1], out, length, history, err)
    torch.cuda.synchronize(dev)
    assert torch.equal(out.cpu(), table[42].cpu())
    assert int(length.item()) == 4 and int(err.item()) == 0
    assert history.cpu().tolist() == [-1, -1, -1, 42, -1, -1, -1, -1]
    # a full history: gathered, not recorded, length kept, error raised
    length.fill_(8)
    _say("step_begin at a full history")
    _hip.decode_step_begin(table, ids[:, 1:], out, length, history, err)
    torch.cuda.synchronize(dev)
    assert torch.equal(out.cpu(), table[7].cpu())
    assert int(length.item()) == 8 and int(err.item()) == 1
    assert history.cpu().tolist() == [-1, -1, -1, 42, -1, -1, -1, -1]
    # an id outside the vocabulary: zero row, recorded, error raised
    err.zero_()
    length.fill_(4)
    bad = torch.tensor([100], dtype=torch.int64, device=dev)
    _say("step_begin with id 100 of 100")
    _hip.decode_step_begin(table, bad, out, length, history, err)
    torch.cuda.synchronize(dev)
    assert out.abs().sum().item() == 0
    assert int(length.item()) == 5 and int(err.item()) == 1


# ------------------------------------------------------------------- model


@pytest.fixture(scope="module")
def model(gpu_device):
    dev = torch.device(gpu_device)
    plan = build_llama31_8b_plan("matrix_group", stream_vocab=False,
                                 num_layers=LAYERS)
    _say("drawing a {}-layer 8B-shaped resident model".format(LAYERS))
    resident = ResidentDeviceArena(plan, None, dev, fill=False).fill_random(5)
    runtime = ResidentTransformerRuntime(plan, None, resident, dev,
                                         synchronize=False).fill_random(5)
    return resident, runtime


@pytest.mark.parametrize("past,max_new", [(6, 6), (40, 2000), (2100, 100)])
def test_decode_graph_replays_equal_eager_steps(gpu_device, model, past, max_new):
    # (40, 2000): the capacity's grid has 64 splits, the lengths' plans 2;
    # (2100, 100): 64 splits in both, rows moving between them as the
    # length grows
    dev = torch.device(gpu_device)
    resident, runtime = model
    steps = 6
    ex = Llama31DecodeExecutor(Llama31Config(num_hidden_layers=LAYERS), resident,
                               top_k=TOP_K)
    ex.reserve(past + max_new)
    gen = torch.Generator(device=dev).manual_seed(past)
    for layer in range(LAYERS):
        ex.kv_cache.buffer[layer, :, :, :past].normal_(generator=gen)
        ex.kv_cache.set_length(layer, past)
    first = torch.tensor([[4242]], dtype=torch.int64, device=dev)
    eager = []
    token = first
    with torch.inference_mode():
        for i in range(steps):
            state = ex.finish(runtime.run(ex, ex.begin(token)))
            eager.append((state.logits.reshape(-1).cpu(),
                          state.topk_values.reshape(-1).cpu(),
                          state.topk_indices.reshape(-1).cpu()))
            token = state.topk_indices.reshape(1, -1)[:, :1]
        torch.cuda.synchronize(dev)
        _say("eager tokens", [int(e[2][0]) for e in eager])
        for layer in range(LAYERS):
            ex.kv_cache.set_length(layer, past)
        _say("capturing the decode step, past", past, "capacity", past + max_new)
        graph = DecodeGraph(ex, runtime, first, max_new)
        buffers = graph.step_buffers
        for i in range(steps):
            if i:
                graph.step()
            torch.cuda.synchronize(dev)
            # eager work between replays
            scratch = torch.randn(1 << 20, device=dev).sum()
            torch.cuda.synchronize(dev)
            del scratch
            _say("replay", i, "top-1", int(buffers.indices.view(-1)[0]))
            logits, values, indices = eager[i]
            assert torch.equal(buffers.logits.reshape(-1).cpu(), logits), i
            assert torch.equal(buffers.values.reshape(-1).cpu(), values), i
            assert torch.equal(buffers.indices.reshape(-1).cpu(), indices), i
        graph.check()
        tokens = graph.tokens().cpu().reshape(-1).tolist()
        assert tokens == [int(e[2][0]) for e in eager]
        assert int(buffers.length.item()) == past + steps
        hist = buffers.history.cpu()
        assert hist[past] == 4242
        assert hist[past + 1:past + steps].tolist() == tokens[:-1]
        assert ex.kv_cache.sequence_length() == past + steps
        with pytest.raises(RuntimeError):  # the executor belongs to the graph
            ex.begin(first)
        if max_new == steps:
            with pytest.raises(RuntimeError):
                graph.step()
        graph.close()
        assert ex._device_step is None and runtime.synchronize is False
