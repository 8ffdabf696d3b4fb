"""Writes tests/golden/tiny_qwen3_transformers.npz: an independent Qwen3 implementation's output on
the tiny seeded checkpoint, used to pin the oracle.

transformers' Qwen3ForCausalLM is built from a local Qwen3Config (no download), loaded with the
seeded bf16 weights widened to f32, and run in f32 on a 24-token prompt: the fixture holds its
logits at every position and its 16-token greedy continuation. The architecture features this
pins are those the reference's forward has (cpu_inference.rs:100-179): q/k RMSNorm before
rotate-half RoPE, GQA head mapping, SwiGLU, tied lm_head.

The same run is repeated with a KV cache that rounds every key and value it stores to bf16
(torch's float32 -> bfloat16 conversion, round to nearest even) and attends with the rounded
values: the semantics of a bf16 KV cache, which pins the oracle's bf16-cache mode
(`*_bf16kv` arrays).

Run from the repo root: python tests/golden/make_tiny_fixture.py
"""
import os
import sys
import tempfile

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "mac-gpu-compiler_amd")]

import qe  # noqa: E402

TINY = qe.Config(256, 512, 2, 4, 2, 128, 1000, 1e-6, 1e6, 999)
SEED = 1234
PROMPT_SEED = 21
PROMPT_LEN = 24
GEN = 16


def transformers_model(ckpt_path):
    import torch
    from safetensors.torch import load_file
    from transformers import Qwen3Config, Qwen3ForCausalLM

    cfg = Qwen3Config(vocab_size=TINY.vocab_size, hidden_size=TINY.hidden_size,
                      intermediate_size=TINY.intermediate_size, num_hidden_layers=TINY.num_hidden_layers,
                      num_attention_heads=TINY.num_attention_heads, num_key_value_heads=TINY.num_key_value_heads,
                      head_dim=TINY.head_dim, rms_norm_eps=TINY.rms_norm_eps, rope_theta=TINY.rope_theta,
                      tie_word_embeddings=True, max_position_embeddings=4096, attention_bias=False,
                      hidden_act="silu")
    cfg._attn_implementation = "eager"
    model = Qwen3ForCausalLM(cfg).float().eval()
    sd = {k: v.float() for k, v in load_file(ckpt_path).items()}
    missing, unexpected = model.load_state_dict(sd, strict=False)
    assert not missing and not unexpected, (missing, unexpected)
    return model, torch


def rounding_cache():
    """A DynamicCache that stores keys and values rounded to bf16 (the rounded values are also
    what the current step attends with)."""
    import torch
    from transformers import DynamicCache

    class Bf16Cache(DynamicCache):
        def update(self, key_states, value_states, layer_idx, *args, **kwargs):
            key_states = key_states.to(torch.bfloat16).to(torch.float32)
            value_states = value_states.to(torch.bfloat16).to(torch.float32)
            return super().update(key_states, value_states, layer_idx, *args, **kwargs)

    return Bf16Cache()


def run(ckpt_path, kv_bf16=False):
    model, torch = transformers_model(ckpt_path)
    prompt = qe.random_prompt(PROMPT_SEED, PROMPT_LEN, TINY.vocab_size)
    with torch.no_grad():
        if not kv_bf16:
            logits = model(torch.tensor(prompt[None].astype(np.int64))).logits[0].numpy().astype(np.float32)
            ids = torch.tensor(prompt[None].astype(np.int64))
            gen = []
            for _ in range(GEN):
                nxt = int(model(ids).logits[0, -1].argmax())
                gen.append(nxt)
                ids = torch.cat([ids, torch.tensor([[nxt]])], dim=1)
            return prompt, logits, np.array(gen, np.int64)
        # one pass over the prompt with the rounding cache, then one token per step
        cache = rounding_cache()
        out = model(torch.tensor(prompt[None].astype(np.int64)), past_key_values=cache, use_cache=True)
        logits = out.logits[0].numpy().astype(np.float32)
        gen = []
        nxt = int(out.logits[0, -1].argmax())
        for _ in range(GEN):
            gen.append(nxt)
            out = model(torch.tensor([[nxt]]), past_key_values=out.past_key_values, use_cache=True)
            nxt = int(out.logits[0, -1].argmax())
    return prompt, logits, np.array(gen, np.int64)


def main():
    with tempfile.TemporaryDirectory() as d:
        ckpt = qe.write_random_checkpoint(d, SEED, TINY)
        prompt, logits, gen = run(ckpt)
        _, logits16, gen16 = run(ckpt, kv_bf16=True)
    out = os.path.join(os.path.dirname(os.path.abspath(__file__)), "tiny_qwen3_transformers.npz")
    np.savez_compressed(out, seed=SEED, prompt_seed=PROMPT_SEED, prompt=prompt.astype(np.int64), logits=logits,
                        greedy=gen, logits_bf16kv=logits16, greedy_bf16kv=gen16)
    print(f"wrote {out}: greedy {gen.tolist()}")


if __name__ == "__main__":
    main()
