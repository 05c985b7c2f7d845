"""Seeded synthetic weights for the benchmark and parity configurations.

The reference initialises ``Linear`` with a truncated normal of std
``sqrt(2/(in+out))`` (``src/llmlab/model/layers.py:18-31``), ``Embedding`` with a
truncated unit normal (``layers.py:59-65``) and RMSNorm gains with ones
(``layers.py:129-131``). The parity configurations instead specify weights drawn
from N(0, 0.02) from a seed, so this module defines that generator:

* ``g = torch.Generator().manual_seed(seed)`` on the CPU;
* every non-norm tensor, in the reference's ``state_dict`` order, is
  ``torch.randn(shape, generator=g, dtype=float32) * 0.02``;
* every RMSNorm gain is 1.0.

The result is a plain fp32 ``state_dict`` with the reference's keys
(``tests/test_model.py:185-199`` in the reference), so it loads into either model.
"""

from __future__ import annotations

import hashlib

import torch

from .config import ModelConfig

BLOCK_KEYS = (
    "attn_norm.weight",
    "attn.q_proj.weight",
    "attn.k_proj.weight",
    "attn.v_proj.weight",
    "attn.output_proj.weight",
    "ffn_norm.weight",
    "ffn.w1.weight",
    "ffn.w2.weight",
    "ffn.w3.weight",
)


def state_dict_shapes(config: ModelConfig) -> list[tuple[str, tuple[int, ...]]]:
    """Keys and shapes in the order ``TransformerLM.state_dict()`` lists them."""
    d, f, v = config.d_model, config.d_ff, config.vocab_size
    shapes = {
        "attn_norm.weight": (d,),
        "attn.q_proj.weight": (d, d),
        "attn.k_proj.weight": (d, d),
        "attn.v_proj.weight": (d, d),
        "attn.output_proj.weight": (d, d),
        "ffn_norm.weight": (d,),
        "ffn.w1.weight": (f, d),
        "ffn.w2.weight": (d, f),
        "ffn.w3.weight": (f, d),
    }
    out = [("token_embeddings.weight", (v, d))]
    for layer in range(config.num_layers):
        out.extend((f"layers.{layer}.{key}", shapes[key]) for key in BLOCK_KEYS)
    out.append(("ln_final.weight", (d,)))
    out.append(("lm_head.weight", (v, d)))
    return out


def seeded_state_dict(config: ModelConfig, seed: int, std: float = 0.02) -> dict[str, torch.Tensor]:
    """Return the fp32 N(0, std) state_dict described in the module docstring."""
    generator = torch.Generator().manual_seed(seed)
    state = {}
    for name, shape in state_dict_shapes(config):
        if name.endswith("norm.weight") or name == "ln_final.weight":
            state[name] = torch.ones(shape, dtype=torch.float32)
        else:
            state[name] = torch.randn(shape, generator=generator, dtype=torch.float32) * std
    return state


def state_dict_sha256(state: dict[str, torch.Tensor]) -> str:
    """SHA-256 over keys and raw little-endian fp32 bytes, in dict order."""
    digest = hashlib.sha256()
    for name, tensor in state.items():
        digest.update(name.encode())
        digest.update(tensor.detach().to(torch.float32).contiguous().numpy().tobytes())
    return digest.hexdigest()


def seeded_prompt(vocab_size: int, batch: int, length: int, seed: int) -> torch.Tensor:
    """Uniform token ids in ``[0, vocab_size)`` from a CPU generator, int64 ``[batch, length]``."""
    generator = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab_size, (batch, length), generator=generator, dtype=torch.int64)
