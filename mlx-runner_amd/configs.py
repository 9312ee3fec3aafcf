"""Model configurations of the workloads (Hugging Face config.json fields plus MLX quantization).

The five configs of the benchmark plan, plus small shapes for tests. Synthetic weights are drawn
by mlxr.synth_write from a seed.
"""
import copy


def _q(bits=4, gs=64):
    return {"bits": bits, "group_size": gs}


QWEN3_0_6B = {  # config 1
    "model_type": "qwen3", "hidden_size": 1024, "num_hidden_layers": 28, "num_attention_heads": 16,
    "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 3072, "vocab_size": 151936,
    "tie_word_embeddings": True, "rope_theta": 1000000.0, "rms_norm_eps": 1e-6, "max_position_embeddings": 40960,
    "quantization": _q(),
}
QWEN3_8B = {  # config 2 (untied lm_head, as Qwen3-8B)
    "model_type": "qwen3", "hidden_size": 4096, "num_hidden_layers": 36, "num_attention_heads": 32,
    "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 12288, "vocab_size": 151936,
    "tie_word_embeddings": False, "rope_theta": 1000000.0, "rms_norm_eps": 1e-6, "max_position_embeddings": 40960,
    "quantization": _q(),
}
LLAMA3_8B = {  # config 3 (no llama3 rope_scaling)
    "model_type": "llama", "hidden_size": 4096, "num_hidden_layers": 32, "num_attention_heads": 32,
    "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 14336, "vocab_size": 128256,
    "tie_word_embeddings": False, "rope_theta": 500000.0, "rms_norm_eps": 1e-5, "max_position_embeddings": 8192,
    "quantization": _q(),
}
QWEN2_5_32B = {  # config 5 (qwen2: q/k/v biases)
    "model_type": "qwen2", "hidden_size": 5120, "num_hidden_layers": 64, "num_attention_heads": 40,
    "num_key_value_heads": 8, "head_dim": 128, "intermediate_size": 27648, "vocab_size": 152064,
    "tie_word_embeddings": False, "rope_theta": 1000000.0, "rms_norm_eps": 1e-6, "max_position_embeddings": 32768,
    "quantization": _q(),
}

CONFIGS = {"qwen3-0.6b": QWEN3_0_6B, "qwen3-8b": QWEN3_8B, "llama3-8b": LLAMA3_8B, "qwen2.5-32b": QWEN2_5_32B}


def tiny(model_type="qwen3", layers=2, hidden=256, heads=4, kv_heads=2, inter=512, vocab=1000, bits=4, gs=64,
         tie=True, theta=1000000.0):
    """A small model of the same family (head_dim 128) for parity tests."""
    return {
        "model_type": model_type, "hidden_size": hidden, "num_hidden_layers": layers, "num_attention_heads": heads,
        "num_key_value_heads": kv_heads, "head_dim": 128, "intermediate_size": inter, "vocab_size": vocab,
        "tie_word_embeddings": tie, "rope_theta": theta, "rms_norm_eps": 1e-6, "max_position_embeddings": 40960,
        "quantization": _q(bits, gs),
    }


def with_layers(cfg, n):
    c = copy.deepcopy(cfg)
    c["num_hidden_layers"] = n
    return c
