"""A tiny seeded Qwen2 with head_dim 128 (the reference's model tests use a tiny seeded
Qwen2 too, test_packed_model.py:27-35; head_dim 128 here so that the HIP kernels apply)."""
from __future__ import annotations

import torch


def tiny_qwen(device="cuda", layers: int = 2):
    from transformers import Qwen2Config, Qwen2ForCausalLM
    from winnow_amd import packed_backend as pb
    torch.manual_seed(0)
    cfg = Qwen2Config(vocab_size=128, hidden_size=512, intermediate_size=512, num_hidden_layers=layers,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512,
                      initializer_range=0.25, architectures=["Qwen2ForCausalLM"])
    m = Qwen2ForCausalLM(cfg).eval().to(device)
    pb.register()
    return m


def prompts(n, seed=1, lo=5, hi=70):
    g = torch.Generator().manual_seed(seed)
    return [torch.randint(0, 128, (int(torch.randint(lo, hi, (1,), generator=g)),), generator=g).tolist()
            for _ in range(n)]
