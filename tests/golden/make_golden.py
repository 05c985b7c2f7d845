"""Write golden vectors from the reference ``TransformerLM`` (run in the build container only).

The reference model (``src/llmlab/model/*.py``, pure torch + einops) is imported
from ``/root/reference/src`` to pin what no closed form fixes: its exact fp32
logits on seeded weights (einsum order, RoPE rounding, SDPA math path) and the
greedy token sequence of the 22.7M configuration. Only the numbers are
committed (``*.npz`` + ``golden.json``); the reference never travels.

    python tests/golden/make_golden.py            # rewrites the fixtures here
"""

from __future__ import annotations

import hashlib
import json
import sys
import time
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO))
sys.path.insert(0, "/root/reference/src")

from llmlab.model.attention import RotaryPositionalEmbedding  # noqa: E402
from llmlab.model.transformer import TransformerLM  # noqa: E402

from systems_for_llms_amd.config import ModelConfig, load_model_config  # noqa: E402
from systems_for_llms_amd.weights import seeded_prompt, seeded_state_dict, state_dict_sha256  # noqa: E402

TINY = ModelConfig(vocab_size=97, context_length=32, d_model=64, num_layers=2, num_heads=4,
                   d_ff=160, rope_theta=10000.0, attention_backend="sdpa")
TINY_SEED, TINY_PROMPT_SEED = 1234, 4321
C1_SEED, C1_PROMPT_SEED, C1_PROMPT, C1_STEPS = 1337, 2027, 64, 192
ROPE_CASES = ((10000.0, 16, 32), (10000.0, 32, 256), (10000.0, 64, 1024), (10000.0, 64, 4096), (500.0, 128, 64))


def sha(t: torch.Tensor) -> str:
    return hashlib.sha256(t.contiguous().numpy().tobytes()).hexdigest()


def reference_model(config: ModelConfig, state, dtype=torch.float32, backend=None):
    model = TransformerLM(vocab_size=config.vocab_size, context_length=config.context_length,
                          d_model=config.d_model, num_layers=config.num_layers,
                          num_heads=config.num_heads, d_ff=config.d_ff, rope_theta=config.rope_theta,
                          attention_backend=backend or config.attention_backend)
    model.load_state_dict(state, strict=True)
    return model.to(dtype).eval()


def main() -> None:
    torch.set_num_threads(8)
    meta: dict = {"generator": "tests/golden/make_golden.py", "torch": torch.__version__,
                  "weights": "seeded_state_dict: randn*0.02 in state_dict order, norms 1.0"}
    arrays: dict[str, np.ndarray] = {}

    rope = []
    for theta, dk, n in ROPE_CASES:
        module = RotaryPositionalEmbedding(theta, dk, n)
        rope.append({"theta": theta, "d_k": dk, "max_seq_len": n,
                     "cos_sha256": sha(module.cos), "sin_sha256": sha(module.sin),
                     "dtype": str(module.cos.dtype)})
    meta["rope"] = rope

    state = seeded_state_dict(TINY, TINY_SEED)
    ids = seeded_prompt(TINY.vocab_size, 3, 24, TINY_PROMPT_SEED)
    meta["tiny"] = {"config": TINY.to_dict(), "seed": TINY_SEED, "prompt_seed": TINY_PROMPT_SEED,
                    "batch": 3, "length": 24, "weights_sha256": state_dict_sha256(state)}
    with torch.no_grad():
        for backend in ("sdpa", "eager"):
            arrays[f"tiny_logits_fp32_{backend}"] = reference_model(TINY, state, backend=backend)(ids).numpy()
        arrays["tiny_logits_bf16_eager"] = (
            reference_model(TINY, state, torch.bfloat16, "eager")(ids).float().numpy())
    arrays["tiny_ids"] = ids.numpy()

    c1 = load_model_config("pilot-22m-s256")
    state = seeded_state_dict(c1, C1_SEED)
    prompt = seeded_prompt(c1.vocab_size, 1, C1_PROMPT, C1_PROMPT_SEED)
    model = reference_model(c1, state)
    started = time.time()
    ids = prompt.clone()
    margins, snapshots = [], {}
    with torch.no_grad():
        for step in range(C1_STEPS):
            last = model(ids)[:, -1, :]
            top = torch.topk(last, 2, dim=-1).values
            margins.append(float(top[0, 0] - top[0, 1]))
            if step in (0, 95, C1_STEPS - 1):
                snapshots[step] = last[0].clone()
            ids = torch.cat([ids, torch.argmax(last, dim=-1, keepdim=True)], dim=1)
    meta["c1"] = {"config": c1.to_dict(), "seed": C1_SEED, "prompt_seed": C1_PROMPT_SEED,
                  "prompt_length": C1_PROMPT, "steps": C1_STEPS,
                  "weights_sha256": state_dict_sha256(state),
                  "min_top2_margin": min(margins), "seconds": round(time.time() - started, 1),
                  "snapshot_steps": sorted(snapshots)}
    arrays["c1_ids"] = ids.numpy()
    arrays["c1_margins"] = np.asarray(margins, dtype=np.float32)
    for step, logits in snapshots.items():
        arrays[f"c1_logits_step{step}"] = logits.numpy()

    np.savez_compressed(HERE / "golden.npz", **arrays)
    (HERE / "golden.json").write_text(json.dumps(meta, indent=2) + "\n")
    print(json.dumps(meta, indent=2))


if __name__ == "__main__":
    main()
