"""Shape and routing constants of DeepSeek-V4-Flash used by the MoE path
(reference src/home_seek/model_config.py:9-53)."""
from dataclasses import dataclass


@dataclass
class MoEConfig:
    num_hidden_layers: int = 43          # model_config.py:9
    hidden_size: int = 4096              # :10
    moe_intermediate_size: int = 2048    # :11
    vocab_size: int = 129280             # :21
    rms_norm_eps: float = 1e-6           # :23
    swiglu_limit: float = 10.0           # :25
    n_routed_experts: int = 256          # :26
    n_shared_experts: int = 1            # :27
    num_experts_per_tok: int = 6         # :28
    routed_scaling_factor: float = 1.5   # :29
    num_hash_layers: int = 3             # :33
    tie_word_embeddings: bool = False    # :40
    mtp_num_draft: int = 2               # hardware_config.py:64
    cublas_max_tokens: int = 8           # hardware_config.py:43
