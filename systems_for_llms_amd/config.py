"""Model configuration, mirroring the reference's ``ModelConfig``.

Follows ``src/llmlab/config.py:7-17`` (field names, order and defaults) and the
``"model"`` section of the reference's JSON configs (``configs/*.json``), which
``load_config`` (``src/llmlab/config.py:93-106``) turns into a ``ModelConfig``.
Only the model section is read here: the training, data and optimizer sections
of those files configure a training loop that this package does not provide.
"""

from __future__ import annotations

import json
import math
from dataclasses import asdict, dataclass
from pathlib import Path

CONFIG_DIR = Path(__file__).resolve().parent / "configs"

# Named model shapes used by the benchmarks and parity tests.
#   pilot-22m-s256   : 22.7M parameters, d=512, 4 layers, 16 heads of 32, ctx 256
#   scale-100m-s1024 : 100.3M parameters, d=768, 12 layers, 12 heads of 64, ctx 1024
#   scale-324m-s4096 : 324.1M parameters, d=1024, 24 layers, 16 heads of 64, ctx 4096
NAMED_CONFIGS = ("pilot-22m-s256", "scale-100m-s1024", "scale-324m-s4096")


@dataclass(frozen=True)
class ModelConfig:
    vocab_size: int = 32
    context_length: int = 8
    d_model: int = 16
    num_layers: int = 1
    num_heads: int = 2
    d_ff: int = 32
    rope_theta: float = 10000.0
    attention_backend: str = "eager"
    activation_checkpointing: str = "none"

    def validate(self) -> None:
        """Raise ValueError with the reference's wording (``config.py:54-56,70-75``)."""
        for name in ("vocab_size", "context_length", "d_model", "num_layers", "num_heads", "d_ff"):
            if type(getattr(self, name)) is not int or getattr(self, name) <= 0:
                raise ValueError(f"model.{name} must be a positive integer")
        if not math.isfinite(self.rope_theta) or self.rope_theta <= 0:
            raise ValueError("model.rope_theta must be finite and positive")
        if self.attention_backend not in {"eager", "sdpa"}:
            raise ValueError("model.attention_backend must be eager or sdpa")
        if self.activation_checkpointing not in {"none", "block"}:
            raise ValueError("model.activation_checkpointing must be none or block")

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    def parameter_count(self) -> int:
        d, f, v, n = self.d_model, self.d_ff, self.vocab_size, self.num_layers
        per_layer = 4 * d * d + 3 * d * f + 2 * d
        return 2 * v * d + n * per_layer + d

    def to_dict(self) -> dict:
        return asdict(self)


def load_model_config(path: str | Path) -> ModelConfig:
    """Read the ``"model"`` section of a reference-style JSON config file.

    A bare name from ``NAMED_CONFIGS`` resolves to the copy shipped with this
    package. Unknown model keys raise TypeError, as ``ModelConfig(**raw)`` does
    in the reference (``config.py:96``).
    """
    path = Path(path)
    if not path.suffix and str(path) in NAMED_CONFIGS:
        path = CONFIG_DIR / f"{path}.json"
    raw = json.loads(Path(path).read_text())
    config = ModelConfig(**raw["model"])
    config.validate()
    return config
