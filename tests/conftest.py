"""Shared fixtures. Tiny random transformers checkpoints (fp32, CPU) are the model-math oracle the
reference's own tests use (code/tests/conftest.py:16-94); the same shapes are built here offline."""
import os
import sys
from pathlib import Path

import pytest
import torch

ROOT = Path(__file__).resolve().parents[1]
for p in (ROOT, ROOT / "ridgefill-data_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

os.environ.setdefault("HF_HUB_OFFLINE", "1")
os.environ.setdefault("HF_HUB_DISABLE_IMPLICIT_TOKEN", "1")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) and the built HIP library")


def _perturb_vectors(model, skip=()):
    """Non-trivial 1-D weights (norm gains): + 0.1 N(0, 1), as the reference fixtures do."""
    with torch.no_grad():
        for name, p in model.named_parameters():
            if p.dim() == 1 and not any(s in name for s in skip):
                p.add_(0.1 * torch.randn_like(p))


@pytest.fixture(scope="session")
def hf_llama():
    """Llama with llama3 RoPE scaling, GQA 4/2, d 16, 6 layers."""
    from transformers import LlamaConfig, LlamaForCausalLM
    torch.manual_seed(0)
    cfg = LlamaConfig(vocab_size=300, hidden_size=64, intermediate_size=160, num_hidden_layers=6,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-5,
                      rope_theta=500000.0, max_position_embeddings=4096, tie_word_embeddings=False,
                      rope_scaling=dict(rope_type="llama3", factor=8.0, low_freq_factor=1.0, high_freq_factor=4.0,
                                        original_max_position_embeddings=64))
    m = LlamaForCausalLM(cfg).float().eval()
    _perturb_vectors(m)
    return m


@pytest.fixture(scope="session")
def hf_qwen3():
    """Dense Qwen3 (per-head q/k RMSNorm), 4 layers."""
    from transformers import Qwen3Config, Qwen3ForCausalLM
    torch.manual_seed(0)
    cfg = Qwen3Config(vocab_size=300, hidden_size=64, intermediate_size=160, num_hidden_layers=4,
                      num_attention_heads=4, num_key_value_heads=2, head_dim=16, rms_norm_eps=1e-6,
                      max_position_embeddings=4096, tie_word_embeddings=False,
                      rope_parameters=dict(rope_type="default", rope_theta=1000000.0))
    m = Qwen3ForCausalLM(cfg).float().eval()
    _perturb_vectors(m)
    return m


@pytest.fixture(scope="session")
def hf_qwen35():
    """Qwen3.5 hybrid: 3 GDN : 1 attention, nk 2 / nv 4, dk = dv = 16, partial RoPE 0.25."""
    from transformers import Qwen3_5ForCausalLM, Qwen3_5TextConfig
    torch.manual_seed(0)
    types = (["linear_attention"] * 3 + ["full_attention"]) * 2
    cfg = Qwen3_5TextConfig(vocab_size=300, hidden_size=64, intermediate_size=160, num_hidden_layers=8,
                            num_attention_heads=4, num_key_value_heads=2, head_dim=32, layer_types=types,
                            linear_num_key_heads=2, linear_num_value_heads=4, linear_key_head_dim=16,
                            linear_value_head_dim=16, linear_conv_kernel_dim=4, rms_norm_eps=1e-6,
                            max_position_embeddings=4096, tie_word_embeddings=False,
                            rope_parameters=dict(rope_type="default", rope_theta=10000000, partial_rotary_factor=0.25,
                                                 mrope_interleaved=True, mrope_section=[2, 1, 1]))
    m = Qwen3_5ForCausalLM(cfg).float().eval()
    _perturb_vectors(m, skip=("A_log", "dt_bias"))
    return m


def ids_of(n, seed=0, vocab=300):
    return torch.randint(0, vocab, (n,), generator=torch.Generator().manual_seed(seed))
