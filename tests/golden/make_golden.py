"""Write the golden fixtures that pin the CPU oracle.

Run from the repository root:  python tests/golden/make_golden.py

Source of truth: the installed transformers library (the third-party
dependency the reference calls for RoPE, layer_streaming/llama31.py:84-87,
pinned there at transformers==4.45.2; installed here: see the fixture's
"transformers_version").  The reference's own code is not imported.  The
fixtures hold inputs and outputs only:

  rope_llama3.json   inverse frequencies of the Llama-3.1 "llama3" RoPE
                     (head_dim 128, theta 500000, factor 8, low 1, high 4,
                     original context 8192), cos / sin rows as bf16 bits at
                     selected positions, and apply_rotary_pos_emb on seeded
                     bf16 q / k.
  tiny_llama.npz     a 2-layer LlamaForCausalLM (hidden 64, 4 heads, 2 KV
                     heads, SwiGLU 128, vocab 97, llama3 RoPE) with seeded
                     fp32 weights; its fp32 logits for a 6-token prompt and
                     a 4-token greedy continuation.
  tiny_llama_bf16.json
                     the reference's CPU path itself
                     (benchmarks/real_llama31_correctness.py:87-129:
                     AutoModelForCausalLM in bf16, default sdpa attention,
                     greedy argmax) on a 2-layer model of the 8B's head
                     geometry (hidden 512, 4 query heads of 128 sharing one
                     KV head, SwiGLU 1024, vocab 97, llama3 RoPE): every
                     decoder layer's output, the final norm and the bf16
                     logits (as bf16 bits) for a 6-token prompt and 3
                     greedy tokens.  The weights are not stored: the recipe
                     below regenerates them (checksums included), and the
                     parameters are cast to bf16 after construction with
                     the RoPE inverse frequencies left in fp32, as
                     from_pretrained(torch_dtype=torch.bfloat16) leaves
                     them.
"""

import json
from pathlib import Path

import numpy as np
import torch

import transformers
from transformers import LlamaConfig, LlamaForCausalLM
from transformers.models.llama.modeling_llama import (
    LlamaRotaryEmbedding,
    apply_rotary_pos_emb,
)

OUT = Path(__file__).resolve().parent
ROPE = {
    "rope_type": "llama3",
    "rope_theta": 500000.0,
    "factor": 8.0,
    "low_freq_factor": 1.0,
    "high_freq_factor": 4.0,
    "original_max_position_embeddings": 8192,
}
POSITIONS = [0, 1, 2, 7, 100, 2047, 2048, 8191, 8192, 32767, 32768, 131071]


def bits(t):
    return t.contiguous().view(torch.int16).to(torch.int32).bitwise_and(0xFFFF).reshape(-1).tolist()


def rope_fixture():
    cfg = LlamaConfig(hidden_size=4096, num_attention_heads=32,
                      num_key_value_heads=8, rope_parameters=dict(ROPE),
                      max_position_embeddings=131072)
    rotary = LlamaRotaryEmbedding(config=cfg)
    pos = torch.tensor([POSITIONS])
    x = torch.zeros(1, 1, 1, 128, dtype=torch.bfloat16)
    cos, sin = rotary(x, pos)
    gen = torch.Generator().manual_seed(1234)
    q = torch.randn(1, 4, 1, 128, generator=gen).to(torch.bfloat16)
    k = torch.randn(1, 2, 1, 128, generator=gen).to(torch.bfloat16)
    p = torch.tensor([[2048]])
    c1, s1 = rotary(q, p)
    q_out, k_out = apply_rotary_pos_emb(q, k, c1, s1)
    return {
        "transformers_version": transformers.__version__,
        "rope": ROPE,
        "head_dim": 128,
        "inv_freq": rotary.inv_freq.tolist(),
        "positions": POSITIONS,
        "cos_bf16_bits": bits(cos[0]),
        "sin_bf16_bits": bits(sin[0]),
        "apply_position": 2048,
        "q_bf16_bits": bits(q),
        "k_bf16_bits": bits(k),
        "q_out_bf16_bits": bits(q_out),
        "k_out_bf16_bits": bits(k_out),
    }


def tiny_model_fixture():
    cfg = LlamaConfig(
        hidden_size=64, intermediate_size=128, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, vocab_size=97,
        rms_norm_eps=1e-5, rope_parameters=dict(ROPE),
        max_position_embeddings=131072, tie_word_embeddings=False,
    )
    torch.manual_seed(99)
    model = LlamaForCausalLM(cfg).eval()
    gen = torch.Generator().manual_seed(4321)
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 1:
                p.copy_(1.0 + 0.1 * torch.randn(p.shape, generator=gen))
            else:
                p.copy_(0.2 * torch.randn(p.shape, generator=gen))
    prompt = [5, 17, 42, 3, 88, 61]
    ids = torch.tensor([prompt])
    steps = []
    tokens = []
    with torch.no_grad():
        out = model(ids, use_cache=True)
        past = out.past_key_values
        logits = out.logits[0, -1].float()
        steps.append(logits.numpy())
        tokens.append(int(torch.argmax(logits)))
        for _ in range(3):
            out = model(torch.tensor([[tokens[-1]]]), past_key_values=past,
                        use_cache=True)
            past = out.past_key_values
            logits = out.logits[0, -1].float()
            steps.append(logits.numpy())
            tokens.append(int(torch.argmax(logits)))
    arrays = {name: p.detach().numpy().astype(np.float32)
              for name, p in model.named_parameters()}
    arrays["__prompt"] = np.array(prompt, dtype=np.int64)
    arrays["__tokens"] = np.array(tokens, dtype=np.int64)
    arrays["__logits"] = np.stack(steps).astype(np.float32)
    return arrays


BF16_CONFIG = {"hidden_size": 512, "intermediate_size": 1024,
               "num_hidden_layers": 2, "num_attention_heads": 4,
               "num_key_value_heads": 1, "head_dim": 128, "vocab_size": 97,
               "rms_norm_eps": 1e-5}
BF16_PROMPT = [5, 17, 42, 3, 88, 61]


def bf16_weight(index, shape):
    """Weight recipe of the bf16 fixture: parameter ``index`` (in
    named_parameters order) drawn in fp32 from its own generator, norm
    vectors 1 + 0.1 N(0, 1), matrices 0.04 N(0, 1), rounded to bf16."""

    gen = torch.Generator().manual_seed(1000 + index)
    values = torch.randn(tuple(shape), generator=gen)
    values = 1.0 + 0.1 * values if len(shape) == 1 else 0.04 * values
    return values.to(torch.bfloat16)


def tiny_bf16_fixture():
    cfg = LlamaConfig(**BF16_CONFIG, rope_parameters=dict(ROPE),
                      max_position_embeddings=131072, tie_word_embeddings=False,
                      attn_implementation="sdpa")
    model = LlamaForCausalLM(cfg).eval()
    names, shapes, checksums = [], [], []
    with torch.no_grad():
        for index, (name, p) in enumerate(model.named_parameters()):
            # parameters only: the rotary inverse frequencies stay fp32
            p.data = bf16_weight(index, p.shape)
            names.append(name)
            shapes.append(list(p.shape))
            checksums.append(float(p.data.double().sum()))
    assert model.model.rotary_emb.inv_freq.dtype == torch.float32
    layer_out = {}
    hooks = [layer.register_forward_hook(
        lambda mod, args, out, i=i: layer_out.__setitem__(i, out[0] if isinstance(out, tuple) else out))
        for i, layer in enumerate(model.model.layers)]
    hooks.append(model.model.norm.register_forward_hook(
        lambda mod, args, out: layer_out.__setitem__("norm", out)))
    steps, tokens = [], []
    past = None
    ids = list(BF16_PROMPT)
    with torch.inference_mode():
        for _ in range(4):
            out = model(input_ids=torch.tensor([ids]), past_key_values=past,
                        use_cache=True)
            past = out.past_key_values
            logits = out.logits[0, -1]
            assert logits.dtype == torch.bfloat16
            steps.append({
                "ids": ids,
                "layer_out_bf16_bits": [bits(layer_out[i][0])
                                        for i in range(len(model.model.layers))],
                "final_norm_bf16_bits": bits(layer_out["norm"][0]),
                "logits_bf16_bits": bits(logits),
            })
            token = int(logits.float().argmax())  # the reference's greedy step
            tokens.append(token)
            ids = [token]
    for hook in hooks:
        hook.remove()
    return {
        "transformers_version": transformers.__version__,
        "torch_version": torch.__version__,
        "config": BF16_CONFIG,
        "rope": ROPE,
        "attn_implementation": "sdpa",
        "weight_recipe": "bf16_weight(index, shape) in tests/golden/make_golden.py",
        "weight_names": names,
        "weight_shapes": shapes,
        "weight_checksums": checksums,
        "prompt": BF16_PROMPT,
        "tokens": tokens,
        "steps": steps,
    }


def main():
    (OUT / "rope_llama3.json").write_text(
        json.dumps(rope_fixture(), indent=1) + "\n", encoding="utf-8")
    np.savez_compressed(OUT / "tiny_llama.npz", **tiny_model_fixture())
    (OUT / "tiny_llama_bf16.json").write_text(
        json.dumps(tiny_bf16_fixture()) + "\n", encoding="utf-8")
    print("wrote", OUT / "rope_llama3.json", OUT / "tiny_llama.npz",
          OUT / "tiny_llama_bf16.json")


if __name__ == "__main__":
    main()
