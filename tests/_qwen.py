"""Random-init Qwen2 models for the bridge tests (no checkpoint is available
offline): the Qwen2.5-1.5B attention shape (12 q / 2 kv heads, head_dim 128),
weights drawn with std 0.05 so that attention dominates the residual stream
and the logits are peaked."""

import torch

# bound on |log p(bridge) - log p(dense fp32 reference)| per token
LOGP_MAX = 0.05


def tiny_qwen(layers=2, vocab=512, seed=0, dtype=torch.float32, device="cpu"):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    cfg = Qwen2Config(vocab_size=vocab, hidden_size=1536, intermediate_size=512,
                      num_hidden_layers=layers, num_attention_heads=12, num_key_value_heads=2,
                      max_position_embeddings=4096, initializer_range=0.05,
                      tie_word_embeddings=False)
    torch.manual_seed(seed)
    with torch.device(device):
        model = Qwen2ForCausalLM(cfg)
    return model.to(dtype).eval()
