"""Named model configurations. ``dev`` is the 12-layer, 59,079,408-parameter benchmark model
(reference chroma/models/variants.py:3-20)."""

from chroma_amd.models.gpt_oss import ModelConfig

dev = ModelConfig(
    num_hidden_layers=12,
    num_experts=12,
    experts_per_token=4,
    vocab_size=201088,
    hidden_size=128,
    intermediate_size=128,
    swiglu_limit=7.0,
    head_dim=16,
    num_attention_heads=8,
    num_key_value_heads=1,
    sliding_window=0,
    initial_context_length=128,
    rope_theta=150000.0,
    rope_scaling_factor=1.0,
    rope_ntk_alpha=1.0,
    rope_ntk_beta=32.0,
)

# GPT-OSS-20B's shape (24 layers, hidden 2880, 64/8 heads of 64, 32 experts top-4, 128-token windows on
# even layers, YaRN factor 32 from a 4096 context, rope theta 150000).
gpt_oss_20b = ModelConfig(
    num_hidden_layers=24,
    num_experts=32,
    experts_per_token=4,
    vocab_size=201088,
    hidden_size=2880,
    intermediate_size=2880,
    swiglu_limit=7.0,
    head_dim=64,
    num_attention_heads=64,
    num_key_value_heads=8,
    sliding_window=128,
    initial_context_length=4096,
    rope_theta=150000.0,
    rope_scaling_factor=32.0,
    rope_ntk_alpha=1.0,
    rope_ntk_beta=32.0,
)
