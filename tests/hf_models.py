"""Tiny random-init HuggingFace models for the patch_hf tests (no downloads)."""
from __future__ import annotations

import torch


def tiny_llama(gqa: bool = True, layers: int = 2, hidden: int = 128, heads: int = 4, seed: int = 0):
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(seed)
    cfg = LlamaConfig(vocab_size=512, hidden_size=hidden, intermediate_size=2 * hidden,
                      num_hidden_layers=layers, num_attention_heads=heads,
                      num_key_value_heads=heads // 2 if gqa else heads,
                      max_position_embeddings=2048, rope_theta=10000.0)
    return LlamaForCausalLM(cfg).eval()


def tiny_qwen2(seed: int = 0):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    torch.manual_seed(seed)
    cfg = Qwen2Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=2048)
    return Qwen2ForCausalLM(cfg).eval()


def tiny_qwen3(seed: int = 0):
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(seed)
    cfg = Qwen3Config(vocab_size=512, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=32,
                      max_position_embeddings=2048)
    return Qwen3ForCausalLM(cfg).eval()


def tiny_gpt2(seed: int = 0):
    from transformers import GPT2Config, GPT2LMHeadModel
    torch.manual_seed(seed)
    cfg = GPT2Config(vocab_size=512, n_embd=128, n_layer=2, n_head=4, n_positions=2048,
                     attn_pdrop=0.0, resid_pdrop=0.0, embd_pdrop=0.0)
    return GPT2LMHeadModel(cfg).eval()


def tiny_mamba(seed: int = 0):
    from transformers import MambaConfig, MambaForCausalLM
    torch.manual_seed(seed)
    cfg = MambaConfig(vocab_size=512, hidden_size=64, num_hidden_layers=2, state_size=8)
    return MambaForCausalLM(cfg).eval()


def token_ids(n: int, vocab: int = 512, batch: int = 1, seed: int = 0, device="cpu"):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randint(0, vocab, (batch, n), generator=g).to(device)
