"""Host logic of the decode executor, on the CPU.

The executor launches kernels with raw pointers and byte offsets (hidden
rows, q / attention / intermediate scratch rows, KV-cache slots per layer
and head, RoPE rows).  Here every buffer lives in host memory and the
kernel entry points are replaced by test doubles that read and write
through exactly those pointers with the oracle's math.  Both the doubles
and the oracle model use float64-exact products (rounded to bf16) and a
float64 softmax, so executor-with-doubles and OracleLlama must agree bit
for bit: any addressing or orchestration slip (wrong slot, position,
layer, norm or buffer row; wrong unit dispatch for a granularity) shows up
as a mismatch.  The GPU kernels themselves are covered by the gpu tests.
"""

import ctypes
import math

import pytest
import torch
import torch.nn.functional as F

from layer_streaming import _hip, build_llama31_8b_plan, create_weight_store
from layer_streaming.llama31 import Llama31Config, Llama31DecodeExecutor, SimpleKVCache
from layer_streaming.rope import inverse_frequencies, rope_parameters
from layer_streaming.runtime import _unit_views
from oracle import llama_oracle as ref

BF16 = torch.bfloat16
LAYERS = 2


def at(ptr, n, dtype=BF16):
    size = torch.empty((), dtype=dtype).element_size()
    return torch.frombuffer((ctypes.c_char * (n * size)).from_address(ptr),
                            dtype=dtype, count=n)


_DOUBLE_WEIGHTS = {}


def exact_linear(x, w):
    key = (w.data_ptr(), tuple(w.shape))
    wd = _DOUBLE_WEIGHTS.get(key)
    if wd is None:
        wd = _DOUBLE_WEIGHTS[key] = w.double().t().contiguous()
    y = x.double().reshape(-1, x.shape[-1]) @ wd
    return y.reshape(*x.shape[:-1], w.shape[0]).to(BF16)


def exact_attention(q, k, v, past):
    heads, seq, dim = q.shape
    groups = heads // k.shape[0]
    kf = k.double().repeat_interleave(groups, 0)
    vf = v.double().repeat_interleave(groups, 0)
    scores = (q.double() @ kf.transpose(1, 2)) / math.sqrt(dim)
    allowed = torch.arange(k.shape[1])[None, :] <= (past + torch.arange(seq))[:, None]
    scores = scores.masked_fill(~allowed[None], float("-inf"))
    out = torch.softmax(scores, -1) @ vf
    return out.transpose(0, 1).reshape(seq, heads * dim).to(q.dtype)


class FakeKernels:
    """Pointer-level doubles of the libcascade_hip entry points."""

    def __init__(self):
        self.calls = []

    def qkv(self, wq, wk, wv, nq, nk, nv, k, x, norm, eps, cos, sin, q_out,
            k_out, v_out, stride, stream):
        self.calls.append("qkv")
        n = ref.rms_norm(at(x, k).reshape(1, k), at(norm, k), eps)
        c, s = at(cos, 64), at(sin, 64)
        c, s = torch.cat((c, c))[None], torch.cat((s, s))[None]
        for w, rows, rope, write in ((wq, nq, True, "q"), (wk, nk, True, "k"),
                                     (wv, nv, False, "v")):
            if not rows:
                continue
            y = ref.linear(n, at(w, rows * k).view(rows, k)).view(rows // 128, 1, 128)
            if rope:
                y = ref.apply_rope(y, c, s)
            if write == "q":
                at(q_out, rows).copy_(y.reshape(-1))
            else:
                base = k_out if write == "k" else v_out
                for h in range(rows // 128):
                    at(base + 2 * h * stride, 128).copy_(y[h, 0])
        return 0

    def attention(self, q, k0, v0, stride, length, hq, hkv, dim, scale, out,
                  ws, ws_bytes, stream):
        self.calls.append("attention")
        keys = torch.stack([at(k0 + 2 * h * stride, length * dim).view(length, dim)
                            for h in range(hkv)])
        vals = torch.stack([at(v0 + 2 * h * stride, length * dim).view(length, dim)
                            for h in range(hkv)])
        qq = at(q, hq * dim).view(hq, 1, dim)
        at(out, hq * dim).copy_(ref.attention(qq, keys, vals, length - 1).reshape(-1))
        return 0

    # device-position forms: the C ABI's position / length rules, then the
    # host-position doubles at those pointers
    def qkv_at(self, wq, wk, wv, nq, nk, nv, k, x, norm, eps, cos_t, sin_t,
               q_out, k_cache, v_cache, stride, length, capacity, stream):
        p = min(max(int(at(length, 1, torch.int64)[0]) - 1, 0), capacity - 1)
        self.qkv(wq, wk, wv, nq, nk, nv, k, x, norm, eps, cos_t + 128 * p,
                 sin_t + 128 * p, q_out, k_cache + 256 * p if k_cache else 0,
                 v_cache + 256 * p if v_cache else 0, stride, stream)
        self.calls[-1] = "qkv_at"
        return 0

    def attention_at(self, q, k0, v0, stride, length, capacity, hq, hkv, dim,
                     scale, out, ws, ws_bytes, stream):
        n = min(max(int(at(length, 1, torch.int64)[0]), 1), capacity)
        self.attention(q, k0, v0, stride, n, hq, hkv, dim, scale, out, ws,
                       ws_bytes, stream)
        self.calls[-1] = "attention_at"
        return 0

    def step_begin(self, table, vocab, hidden, ids, out, length, history,
                   capacity, error, stream):
        self.calls.append("step_begin")
        token = int(at(ids, 1, torch.int64)[0])
        word = at(length, 1, torch.int64)
        n = int(word[0])
        at(out, hidden).copy_(at(table + 2 * token * hidden, hidden))
        if 0 <= n < capacity:
            at(history, capacity, torch.int64)[n] = token
            word[0] = n + 1
        else:
            at(error, 1, torch.int32)[0] = 1
        return 0

    def residual(self, w, x, res, y, n, k, stream):
        self.calls.append("residual")
        out = at(res, n).reshape(1, n) + ref.linear(at(x, k).reshape(1, k),
                                                    at(w, n * k).view(n, k))
        at(y, n).copy_(out.reshape(-1))
        return 0

    def _normed(self, x, norm, k, eps):
        xx = at(x, k).reshape(1, k)
        return ref.rms_norm(xx, at(norm, k), eps) if norm else xx

    def swiglu(self, wg, wu, n, k, x, norm, eps, y, stream):
        self.calls.append("swiglu")
        nn = self._normed(x, norm, k, eps)
        out = F.silu(ref.linear(nn, at(wg, n * k).view(n, k))) * ref.linear(
            nn, at(wu, n * k).view(n, k))
        at(y, n).copy_(out.reshape(-1))
        return 0

    def silu(self, wg, n, k, x, norm, eps, y, stream):
        self.calls.append("silu")
        out = F.silu(ref.linear(self._normed(x, norm, k, eps), at(wg, n * k).view(n, k)))
        at(y, n).copy_(out.reshape(-1))
        return 0

    def mul(self, wu, n, k, x, norm, eps, gate, y, stream):
        self.calls.append("mul")
        out = at(gate, n).reshape(1, n) * ref.linear(self._normed(x, norm, k, eps),
                                                     at(wu, n * k).view(n, k))
        at(y, n).copy_(out.reshape(-1))
        return 0

    def rmsnorm(self, x, w, y, rows, n, eps, stream):
        self.calls.append("rmsnorm")
        at(y, rows * n).copy_(ref.rms_norm(at(x, rows * n).view(rows, n),
                                           at(w, n), eps).reshape(-1))
        return 0

    def head(self, w, rows, k, offset, h, top_k, first, logits, ws, ws_bytes,
             values, indices, stream):
        self.calls.append("lm_head")
        lg = ref.lm_head_logits(at(h, k), at(w, rows * k).view(rows, k))
        at(logits, rows, torch.float32).copy_(lg)
        v, i = ref.topk(lg, top_k)
        at(values, top_k, torch.float32).copy_(v)
        at(indices, top_k, torch.int64).copy_(i + offset)
        return 0

    # -------------------------------------- batched (S > 1) entry points

    def qkv_gemm(self, x, m, wq, wk, wv, nq, nk, nv, k, cos, sin, positions,
                 pos0, q_out, k_out, v_out, stride, slot0, stream):
        self.calls.append("qkv_gemm")
        n = at(x, m * k).view(m, k)  # rows are already normalised
        if nq or nk:
            c = at(cos, positions * 64).view(positions, 64)[pos0:pos0 + m]
            s = at(sin, positions * 64).view(positions, 64)[pos0:pos0 + m]
            c, s = torch.cat((c, c), -1), torch.cat((s, s), -1)
        for w, rows, rope, write in ((wq, nq, True, "q"), (wk, nk, True, "k"),
                                     (wv, nv, False, "v")):
            if not rows:
                continue
            y = ref.linear(n, at(w, rows * k).view(rows, k))
            y = y.view(m, rows // 128, 128).transpose(0, 1)
            if rope:
                y = ref.apply_rope(y, c, s)
            if write == "q":
                at(q_out, m * rows).copy_(y.transpose(0, 1).reshape(-1))
            else:
                base = k_out if write == "k" else v_out
                for h in range(rows // 128):
                    at(base + 2 * (h * stride + slot0 * 128), m * 128).copy_(
                        y[h].reshape(-1))
        return 0

    def prefill_attention(self, q, k0, v0, stride, past, tokens, hq, hkv, dim,
                          scale, out, stream):
        self.calls.append("prefill_attention")
        length = past + tokens
        keys = torch.stack([at(k0 + 2 * h * stride, length * dim).view(length, dim)
                            for h in range(hkv)])
        vals = torch.stack([at(v0 + 2 * h * stride, length * dim).view(length, dim)
                            for h in range(hkv)])
        qq = at(q, tokens * hq * dim).view(tokens, hq, dim).transpose(0, 1)
        at(out, tokens * hq * dim).copy_(
            ref.attention(qq, keys, vals, past).reshape(-1))
        return 0

    def gemm_residual(self, x, w, res, y, m, n, k, stream):
        self.calls.append("gemm_residual")
        out = at(res, m * n).view(m, n) + ref.linear(at(x, m * k).view(m, k),
                                                     at(w, n * k).view(n, k))
        at(y, m * n).copy_(out.reshape(-1))
        return 0

    def gemm_residual_ws(self, x, w, res, y, m, n, k, ws, ws_bytes, stream):
        return self.gemm_residual(x, w, res, y, m, n, k, stream)

    def swiglu_gemm(self, x, wg, wu, y, m, n, k, stream):
        self.calls.append("swiglu_gemm")
        xx = at(x, m * k).view(m, k)
        out = F.silu(ref.linear(xx, at(wg, n * k).view(n, k))) * ref.linear(
            xx, at(wu, n * k).view(n, k))
        at(y, m * n).copy_(out.reshape(-1))
        return 0

    def silu_gemm(self, x, wg, y, m, n, k, stream):
        self.calls.append("silu_gemm")
        out = F.silu(ref.linear(at(x, m * k).view(m, k), at(wg, n * k).view(n, k)))
        at(y, m * n).copy_(out.reshape(-1))
        return 0

    def mul_gemm(self, x, wu, gate, y, m, n, k, stream):
        self.calls.append("mul_gemm")
        out = at(gate, m * n).view(m, n) * ref.linear(at(x, m * k).view(m, k),
                                                      at(wu, n * k).view(n, k))
        at(y, m * n).copy_(out.reshape(-1))
        return 0

    def f32_gemm(self, x, w, y, m, n, k, stream):
        # each row as the oracle's LM head computes it, so the last row's
        # logits (and their top-k) match the oracle bit for bit
        self.calls.append("f32_gemm")
        xs, ws = at(x, m * k).view(m, k), at(w, n * k).view(n, k)
        out = torch.stack([ref.lm_head_logits(xs[r], ws) for r in range(m)])
        at(y, m * n, torch.float32).copy_(out.reshape(-1))
        return 0

    def topk(self, logits, rows, top_k, ws, ws_bytes, values, indices, stream):
        self.calls.append("topk")
        v, i = ref.topk(at(logits, rows, torch.float32), top_k)
        at(values, top_k, torch.float32).copy_(v)
        at(indices, top_k, torch.int64).copy_(i)
        return 0


class HostResident:
    """CPU stand-in for ResidentDeviceArena (views into the host store)."""

    def __init__(self, plan, store):
        self.plan = plan
        self.store = store
        self.device = torch.device("cpu")

    def __getitem__(self, key):
        return self.store.tensor(key)


def lenient_require(tensor, name, dtype=None, min_numel=None, contiguous=True):
    assert isinstance(tensor, torch.Tensor), name
    if dtype is not None:
        assert tensor.dtype == dtype, name
    if contiguous:
        assert tensor.is_contiguous(), name
    if min_numel is not None:
        assert tensor.numel() >= min_numel, name
    return tensor


@pytest.fixture(scope="module")
def weights():
    plan = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    store = create_weight_store(plan, "pinned_staging",
                                tensor_factory=lambda n, **kw: torch.empty(
                                    n, dtype=kw["dtype"]))
    store.fill_random(seed=11, norm="random")
    yield store
    _DOUBLE_WEIGHTS.clear()


@pytest.fixture
def exact_oracle(monkeypatch):
    monkeypatch.setattr(ref, "linear", exact_linear)
    monkeypatch.setattr(ref, "attention", exact_attention)
    monkeypatch.setattr(_hip, "require_device", lenient_require)


def make_executor(monkeypatch, plan, store):
    fakes = FakeKernels()

    def gather(table, ids, out, error_flag=None, stream=None):
        out.view(-1, table.shape[1]).copy_(table[ids.cpu()])
        return out

    monkeypatch.setattr(_hip, "embedding_gather", gather)
    cache = SimpleKVCache(LAYERS, device="cpu")
    ex = Llama31DecodeExecutor(Llama31Config(num_hidden_layers=LAYERS),
                               HostResident(plan, store), kv_cache=cache, top_k=5)
    ex._stream = lambda: 0
    ex._k_qkv, ex._k_attn, ex._k_residual = fakes.qkv, fakes.attention, fakes.residual
    ex._k_swiglu, ex._k_silu, ex._k_mul = fakes.swiglu, fakes.silu, fakes.mul
    ex._k_rmsnorm, ex._k_head = fakes.rmsnorm, fakes.head
    ex._k_qkv_gemm, ex._k_prefill_attn = fakes.qkv_gemm, fakes.prefill_attention
    ex._k_gemm_residual, ex._k_swiglu_gemm = fakes.gemm_residual, fakes.swiglu_gemm
    ex._k_gemm_residual_ws = fakes.gemm_residual_ws
    ex._k_silu_gemm, ex._k_mul_gemm = fakes.silu_gemm, fakes.mul_gemm
    ex._k_f32_gemm, ex._k_topk = fakes.f32_gemm, fakes.topk
    ex._k_qkv_at, ex._k_attn_at = fakes.qkv_at, fakes.attention_at
    ex._k_step_begin = fakes.step_begin
    return ex, fakes


def run_units(plan, store, executor, state):
    for unit in plan.units:
        views = _unit_views(unit, store.unit_source(unit))
        state = executor(unit, views, state)
    return state


@pytest.mark.parametrize("granularity", ["matrix_group", "matrix", "layer"])
def test_executor_addressing_matches_oracle_bit_for_bit(monkeypatch, weights,
                                                        exact_oracle, granularity):
    plan = build_llama31_8b_plan(granularity, num_layers=LAYERS)
    # every granularity packs the arena identically, so one store serves all
    for key in plan.tensors:
        assert plan.tensor_host_offset(key) == weights.plan.tensor_host_offset(key)
    store = weights
    executor, fakes = make_executor(monkeypatch, plan, store)
    oracle = ref.OracleLlama(store.tensor, LAYERS)
    prompt = [7, 99, 1234, 5, 128255, 0]
    expected_logits, ev, ei = oracle.step(prompt, 5)
    state = run_units(plan, store, executor,
                      executor.begin(torch.tensor([prompt])))
    state = executor.finish(state)
    assert torch.equal(state.logits[0, -1], expected_logits)
    assert state.topk_indices.reshape(-1).tolist() == ei.tolist()
    token = int(ei[0])
    for _ in range(3):
        expected_logits, ev, ei = oracle.step([token], 5)
        state = run_units(plan, store, executor,
                          executor.begin(torch.tensor([[token]])))
        state = executor.finish(state)
        assert torch.equal(state.logits[0, -1], expected_logits)
        assert state.topk_indices.reshape(-1).tolist() == ei.tolist()
        token = int(ei[0])
    assert executor.kv_cache.sequence_length() == len(prompt) + 3
    # the oracle's cache and the executor's cache hold the same K / V
    for layer in range(LAYERS):
        k, v = executor.kv_cache.entries[layer]
        assert torch.equal(k[0], oracle.caches[layer]["k"])
        assert torch.equal(v[0], oracle.caches[layer]["v"])
    per_token = {"matrix_group": 5, "matrix": 8, "layer": 5}[granularity]
    # prefill, per layer: input norm, q/k/v GEMM(s), causal attention,
    # o GEMM, post-attention norm, MLP GEMM(s), down GEMM
    per_prefill = {"matrix_group": 7, "matrix": 10, "layer": 7}[granularity]
    # decode, per layer and token: qkv launch(es), attention, o residual,
    # MLP, down; finish: one rmsnorm, then (prefill) one logits GEMM over
    # every position and the top-k of the last row's logits, (decode) one
    # LM-head launch
    assert fakes.calls.count("prefill_attention") == LAYERS
    assert fakes.calls.count("f32_gemm") == 1
    assert fakes.calls.count("topk") == 1
    expected = (LAYERS * per_prefill + 3) + 3 * (LAYERS * per_token + 2)
    assert len(fakes.calls) == expected


def test_device_step_decode_matches_oracle(monkeypatch, weights, exact_oracle):
    # The executor in DecodeGraph's mode (position and length read from a
    # device word, top-k into fixed buffers whose first id feeds the next
    # step): same logits, top-k and cache as the oracle, and the length word
    # and token history advance by one per step.
    from layer_streaming.graph import DeviceStep

    plan = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    executor, fakes = make_executor(monkeypatch, plan, weights)
    oracle = ref.OracleLlama(weights.tensor, LAYERS)
    prompt = [7, 99, 1234, 5, 128255, 0]
    _, _, ei = oracle.step(prompt, 5)
    executor.finish(run_units(plan, weights, executor,
                              executor.begin(torch.tensor([prompt]))))
    past = len(prompt)
    step = DeviceStep("cpu", past + 4, 128256, 5)
    executor.reserve(past + 4)
    step.length.fill_(past)
    token = int(ei[0])
    step.indices.view(-1)[0] = token
    executor._device_step = step
    with pytest.raises(RuntimeError):  # only the owning DecodeGraph may step
        executor.begin(step.ids)
    step.active = True
    fakes.calls.clear()
    for i in range(3):
        expected_logits, _, ei = oracle.step([token], 5)
        state = run_units(plan, weights, executor, executor.begin(step.ids))
        state = executor.finish(state)
        assert state.logits is step.logits
        assert torch.equal(step.logits[0, -1], expected_logits)
        assert step.indices.reshape(-1).tolist() == ei.tolist()
        assert int(step.length[0]) == past + i + 1
        assert int(step.history[past + i]) == token
        token = int(ei[0])
    assert int(step.error[0]) == 0
    # every position-dependent launch took the device-word form
    assert fakes.calls.count("step_begin") == 3
    assert fakes.calls.count("qkv_at") == 3 * LAYERS
    assert fakes.calls.count("attention_at") == 3 * LAYERS
    assert "qkv" not in fakes.calls and "attention" not in fakes.calls
    for layer in range(LAYERS):
        k, v = executor.kv_cache.entries[layer]
        assert torch.equal(k[0], oracle.caches[layer]["k"])
        assert torch.equal(v[0], oracle.caches[layer]["v"])
    # a step past the capacity is refused by the first launch
    step.length.fill_(past + 4)
    run_units(plan, weights, executor, executor.begin(step.ids))
    assert int(step.error[0]) == 1 and int(step.length[0]) == past + 4


def test_rope_table_equals_oracle_cos_sin():
    params = rope_parameters(Llama31Config())
    assert torch.equal(inverse_frequencies(128, params), ref.llama3_inv_freq(128))
    from layer_streaming.rope import cos_sin_rows

    cos, sin = cos_sin_rows(inverse_frequencies(128, params), 0, 40000)
    positions = [0, 1, 2047, 8192, 32768, 39999]
    oc, os_ = ref.rope_cos_sin(ref.llama3_inv_freq(128), positions)
    assert torch.equal(cos[positions], oc[:, :64])
    assert torch.equal(sin[positions], os_[:, :64])
    assert torch.equal(oc[:, :64], oc[:, 64:])


def test_kv_cache_growth_keeps_entries():
    cache = SimpleKVCache(2, num_kv_heads=2, head_dim=4, device="cpu")
    k = torch.randn(1, 2, 300, 4).to(BF16)
    v = torch.randn(1, 2, 300, 4).to(BF16)
    cache.append(0, k, v)
    cache.append(1, k, v)
    assert cache.capacity == 512 and cache.sequence_length() == 300
    cache.append(0, k, v)  # grows to 768 slots, copying the first 300
    assert cache.capacity >= 600
    assert torch.equal(cache.entries[0][0][0, :, :300], k[0])
    assert torch.equal(cache.entries[0][0][0, :, 300:], k[0])
    cache.clear()
    assert cache.sequence_length() == 0 and cache.entries[0] is None


def test_begin_rejects_multi_token_after_prefill(monkeypatch, weights, exact_oracle):
    plan = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    executor, _ = make_executor(monkeypatch, plan, weights)
    with pytest.raises(ValueError):
        executor.begin(torch.tensor([1, 2]))
    executor.kv_cache.reserve(8)
    executor.kv_cache.set_length(0, 3)
    with pytest.raises(ValueError):
        executor.begin(torch.tensor([[1, 2]]))
    with pytest.raises(ValueError):
        Llama31DecodeExecutor(Llama31Config(num_hidden_layers=LAYERS, hidden_size=8),
                              HostResident(plan, weights))


def test_layer_count_must_match_the_plan(monkeypatch, weights, exact_oracle):
    # The reference accepts only the 32-layer config (llama31.py:93-109).
    # Here the config must match the plan the resident arena was built from:
    # a full 32-layer plan takes only the 32-layer config, as in the
    # reference; a truncated plan (the tests' full-width 2-layer models, the
    # CLI's --layers) takes only its own layer count.
    full = build_llama31_8b_plan("matrix_group")
    monkeypatch.setattr(_hip, "load", lambda: None)
    for layers in (31, 33, 2):
        with pytest.raises(ValueError, match="num_hidden_layers"):
            Llama31DecodeExecutor(Llama31Config(num_hidden_layers=layers),
                                  HostResident(full, weights))
    small = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    with pytest.raises(ValueError, match="num_hidden_layers"):
        Llama31DecodeExecutor(Llama31Config(), HostResident(small, weights))


def test_begin_rejects_token_ids_outside_the_vocabulary(monkeypatch, weights,
                                                        exact_oracle):
    # F.embedding raises on such an id (the reference's resident table,
    # llama31.py:144-148); host-held ids are checked before any launch
    plan = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    executor, fakes = make_executor(monkeypatch, plan, weights)
    for bad in ([[128256]], [[-1]], [[5, 128256, 7]]):
        with pytest.raises(IndexError):
            executor.begin(torch.tensor(bad))
    assert fakes.calls == []
    executor.begin(torch.tensor([[128255]]))  # the last valid id


def test_error_word_bits_name_their_cause():
    # 1 (the embedding gather's id check) raises IndexError; the fused
    # attention's bits raise RuntimeError after the reset hook has run
    from layer_streaming.llama31 import _ErrorWord

    resets = []
    word = _ErrorWord(torch.device("cpu"), "token id outside [0, 10)",
                      on_attention_error=resets.append)
    word.raise_if_set()  # nothing published yet
    word.publish()
    word.raise_if_set()  # published zero
    word.flag.fill_(1)
    word.publish()
    with pytest.raises(IndexError):
        word.raise_if_set()
    assert resets == [] and int(word.flag[0]) == 0
    for bit in (_hip.ATTN_EPLACEMENT, _hip.ATTN_ETIMEOUT,
                _hip.ATTN_EPLACEMENT | 1):
        word.flag.fill_(bit)
        word.publish()
        with pytest.raises(RuntimeError, match="fused decode attention"):
            word.raise_if_set()
        assert int(word.flag[0]) == 0
    assert resets == [_hip.ATTN_EPLACEMENT, _hip.ATTN_ETIMEOUT,
                      _hip.ATTN_EPLACEMENT | 1]


def test_executor_is_freed_without_a_cycle_collection(monkeypatch, weights, exact_oracle):
    # The error word keeps the executor's attention-failure method weakly:
    # once the caller drops the executor (after a prefill and a decode step),
    # reference counting alone frees it and its buffers, with the cyclic
    # collector switched off.
    import gc
    import weakref

    plan = build_llama31_8b_plan("matrix_group", num_layers=LAYERS)
    executor, _ = make_executor(monkeypatch, plan, weights)
    state = executor.finish(run_units(plan, weights, executor,
                                      executor.begin(torch.tensor([list(range(3, 23))]))))
    token = state.topk_indices.reshape(1, -1)[:, :1].clone()
    executor.finish(run_units(plan, weights, executor, executor.begin(token)))
    alive = weakref.ref(executor)
    was_enabled = gc.isenabled()
    gc.disable()
    try:
        del executor, state
        assert alive() is None
    finally:
        if was_enabled:
            gc.enable()
