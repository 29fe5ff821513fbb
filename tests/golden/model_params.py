"""Deterministic parameters and inputs for the NSAAttention golden vectors.

Shared by the fixture generator (make_nsa_model_golden.py) and the tests, so
both sides build bit-identical layers without storing the weights.
"""

import torch

# (name, NSAAttention kwargs, B, T): small layers covering G=4 with D=16 and
# G=2 with D=32, T with and without a trailing partial block, and rows with
# fewer complete blocks than n_selected_blocks (the tied fillers).
CONFIGS = [
    ("g4_d16", dict(d_model=64, n_q_heads=4, n_kv_heads=1, block_size=16, n_selected_blocks=3, window=24), 1, 88),
    ("g2_d32", dict(d_model=64, n_q_heads=2, n_kv_heads=1, block_size=16, n_selected_blocks=4, window=40), 1, 72),
]


def init_params(module, seed):
    """Overwrite every parameter, in name order, from one seeded generator."""
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(module.named_parameters()):
            x = torch.randn(p.shape, generator=g, dtype=torch.float64)
            if p.dim() == 2 and "intra_pos" not in name:
                x = x / p.shape[1] ** 0.5          # Linear weight: unit-variance outputs
            else:
                x = x * 0.5                        # biases, pool logits, intra-block positions
            p.copy_(x.to(p.dtype))


def inputs(cfg, B, T, seed, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, T, cfg["d_model"], generator=g, dtype=torch.float64)
    dy = torch.randn(B, T, cfg["d_model"], generator=g, dtype=torch.float64)
    return x.to(dtype), dy.to(dtype)


# (name, NSATransformer kwargs, B, T): a two-layer model with NSA attention
# (a trailing partial block, rows with tied fillers) and the same model with
# the dense control arm.
MODEL_CONFIGS = [
    ("tf_nsa", dict(vocab_size=96, d_model=64, n_layers=2, n_q_heads=4, n_kv_heads=2, max_seq_len=80, ffn_mult=2,
                    block_size=16, n_selected_blocks=3, window=24, attn_type="nsa"), 2, 72),
    ("tf_full", dict(vocab_size=96, d_model=64, n_layers=2, n_q_heads=4, n_kv_heads=2, max_seq_len=80, ffn_mult=2,
                     block_size=16, n_selected_blocks=3, window=24, attn_type="full"), 2, 72),
]


def tokens(cfg, B, T, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randint(0, cfg["vocab_size"], (B, T), generator=g)
    y = torch.randint(0, cfg["vocab_size"], (B, T), generator=g)
    return x, y
