"""``TransformerLM``: the reference model API, run by the gfx950 kernels.

Keeps the constructor, validation messages, module tree and ``state_dict``
keys of ``src/llmlab/model/transformer.py:51-139`` (and of the layers in
``layers.py`` / ``attention.py``), so a reference checkpoint's ``model`` dict
loads unchanged. Parameters are initialised as the reference does
(``layers.py:18-31,59-65,129-131``).

Execution is inference-only and on the GPU: ``forward(input_ids)`` returns the
logits of every position from one prefill pass of MFMA GEMMs and causal
attention (in the model dtype: bf16, fp16 or fp32; equal to the reference's
forward up to float reassociation and, for 16-bit models, the rounding of
what the pass stores), and ``generate`` runs the greedy token loop the
reference lacks: the prefill, then KV-cached decode steps. There is no CPU
path: calling the model on CPU tensors raises.
"""

from __future__ import annotations

import math

import torch
from torch import nn

from . import engine as _engine


def _trunc_normal(shape, std, bound, device, dtype):
    weight = torch.empty(shape, device=device, dtype=dtype)
    nn.init.trunc_normal_(weight, mean=0.0, std=std, a=-bound, b=bound)
    return nn.Parameter(weight)


class Linear(nn.Module):
    """``layers.py:6-35``: weight ``[out, in]``, no bias."""

    def __init__(self, in_features, out_features, device=None, dtype=None):
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        std = math.sqrt(2 / (in_features + out_features))
        self.weight = _trunc_normal((out_features, in_features), std, 3 * std, device, dtype)


class Embedding(nn.Module):
    """``layers.py:39-70``."""

    def __init__(self, num_embeddings, embedding_dim, device=None, dtype=None):
        super().__init__()
        self.num_embeddings, self.embedding_dim = num_embeddings, embedding_dim
        self.weight = _trunc_normal((num_embeddings, embedding_dim), 1.0, 3.0, device, dtype)


class RMSNorm(nn.Module):
    """``layers.py:118-141``: gain initialised to ones, eps 1e-5."""

    def __init__(self, d_model, eps=1e-5, device=None, dtype=None):
        super().__init__()
        self.d_model, self.eps = d_model, eps
        self.weight = nn.Parameter(torch.ones(d_model, device=device, dtype=dtype))


class SwiGLU(nn.Module):
    """``layers.py:77-115``: ``w2(silu(w1 x) * w3 x)``; default d_ff rounds 8d/3 up to 64."""

    def __init__(self, d_model, d_ff=None, device=None, dtype=None):
        super().__init__()
        if d_ff is None:
            d_ff = 64 * math.ceil(int(8 * d_model / 3) / 64)
        self.d_model, self.d_ff = d_model, d_ff
        self.w1 = Linear(d_model, d_ff, device, dtype)
        self.w2 = Linear(d_ff, d_model, device, dtype)
        self.w3 = Linear(d_model, d_ff, device, dtype)


class MultiHeadSelfAttention(nn.Module):
    """Parameters and validation of ``attention.py:101-142`` (+ RoPE checks ``:20-26``)."""

    def __init__(self, d_model, num_heads, theta=None, max_seq_len=None, device=None, dtype=None,
                 attention_backend="eager"):
        super().__init__()
        if d_model <= 0 or num_heads <= 0:
            raise ValueError("d_model and num_heads must be positive")
        if d_model % num_heads != 0:
            raise ValueError("d_model must be divisible by num_heads")
        if attention_backend not in {"eager", "sdpa"}:
            raise ValueError("attention_backend must be 'eager' or 'sdpa'")
        if (theta is None) != (max_seq_len is None):
            raise ValueError("theta and max_seq_len must be provided together")
        self.d_model, self.num_heads = d_model, num_heads
        self.d_k = d_model // num_heads
        self.attention_backend = attention_backend
        self.max_seq_len = max_seq_len
        self.theta = theta
        if theta is not None:
            if self.d_k <= 0 or self.d_k % 2 != 0:
                raise ValueError("d_k must be positive and even because RoPE rotates dimension pairs")
            if not math.isfinite(theta) or theta <= 0:
                raise ValueError("theta must be finite and positive")
            if max_seq_len <= 0:
                raise ValueError("max_seq_len must be positive")
        self.q_proj = Linear(d_model, d_model, device, dtype)
        self.k_proj = Linear(d_model, d_model, device, dtype)
        self.v_proj = Linear(d_model, d_model, device, dtype)
        self.output_proj = Linear(d_model, d_model, device, dtype)


class TransformerBlock(nn.Module):
    """``transformer.py:8-48``: pre-norm attention and SwiGLU with residuals."""

    def __init__(self, d_model, num_heads, d_ff, theta, max_seq_len, device=None, dtype=None,
                 attention_backend="eager"):
        super().__init__()
        self.attn_norm = RMSNorm(d_model, device=device, dtype=dtype)
        self.attn = MultiHeadSelfAttention(d_model, num_heads, theta, max_seq_len, device, dtype,
                                           attention_backend)
        self.ffn_norm = RMSNorm(d_model, device=device, dtype=dtype)
        self.ffn = SwiGLU(d_model, d_ff, device, dtype)


def rope_tables(theta: float, d_k: int, max_seq_len: int) -> tuple[torch.Tensor, torch.Tensor]:
    """fp32 cos/sin ``[max_seq_len, d_k/2]`` built as ``attention.py:31-42`` builds them.

    The kernels read this host-built table instead of evaluating sin/cos on the
    device, so the rotation angles match the reference bit for bit.
    """
    positions = torch.arange(max_seq_len)
    pairs = torch.arange(0, d_k, 2)
    inverse = 1.0 / (theta ** (pairs / d_k))
    angles = positions.to(torch.float32)[:, None] * inverse[None, :]
    return torch.cos(angles), torch.sin(angles)


class TransformerLM(nn.Module):
    """Drop-in for ``llmlab.model.transformer.TransformerLM`` (inference on gfx950)."""

    def __init__(self, vocab_size, context_length, d_model, num_layers, num_heads, d_ff, rope_theta,
                 device=None, dtype=None, attention_backend="eager", activation_checkpointing="none"):
        super().__init__()
        dimensions = {"vocab_size": vocab_size, "context_length": context_length, "d_model": d_model,
                      "num_layers": num_layers, "num_heads": num_heads, "d_ff": d_ff}
        for name, value in dimensions.items():
            if not isinstance(value, int) or value <= 0:
                raise ValueError(f"{name} must be a positive integer")
        if activation_checkpointing not in {"none", "block"}:
            raise ValueError("activation_checkpointing must be 'none' or 'block'")
        self.vocab_size, self.context_length, self.d_model = vocab_size, context_length, d_model
        self.num_layers, self.num_heads, self.d_ff = num_layers, num_heads, d_ff
        self.theta = rope_theta
        self.attention_backend = attention_backend
        self.activation_checkpointing = activation_checkpointing
        # Not in the reference: True keeps every decode output at one writer (no fp32
        # atomics), so repeated forward/generate calls give bit-identical results;
        # None (the default) chooses it for float32 models, whose greedy ids must not
        # depend on the order of fp32 additions, and the faster fused path otherwise.
        self.deterministic = None
        self.token_embeddings = Embedding(vocab_size, d_model, device, dtype)
        self.layers = nn.ModuleList([
            TransformerBlock(d_model, num_heads, d_ff, rope_theta, context_length, device, dtype,
                             attention_backend)
            for _ in range(num_layers)
        ])
        self.ln_final = RMSNorm(d_model, device=device, dtype=dtype)
        self.lm_head = Linear(d_model, vocab_size, device, dtype)

    @classmethod
    def from_config(cls, config, device=None, dtype=None) -> "TransformerLM":
        return cls(config.vocab_size, config.context_length, config.d_model, config.num_layers,
                   config.num_heads, config.d_ff, config.rope_theta, device=device, dtype=dtype,
                   attention_backend=config.attention_backend,
                   activation_checkpointing=config.activation_checkpointing)

    @classmethod
    def from_checkpoint(cls, path, device=None, dtype=None) -> "TransformerLM":
        """The model a reference training checkpoint describes, with its weights.

        Reads the ``checkpoint.pt`` written by ``src/llmlab/train.py:265-275``
        (``format_version`` 1): the training configuration as a dict under
        ``"config"``, whose ``"model"`` section gives the shape (``config.py:7-17``),
        and the module ``state_dict`` under ``"model"``. The file is read with
        ``torch.load(weights_only=True)``, which executes nothing from it; the
        optimizer and RNG states it also holds are ignored. Weights are cast to
        ``dtype`` (default: as stored) and moved to ``device``.
        """
        from .config import ModelConfig

        checkpoint = torch.load(path, map_location="cpu", weights_only=True)
        if not isinstance(checkpoint, dict) or "model" not in checkpoint or "config" not in checkpoint:
            raise ValueError("checkpoint must hold 'config' and 'model' entries")
        if checkpoint.get("format_version", 1) != 1:
            raise ValueError(f"unsupported checkpoint format_version {checkpoint['format_version']}")
        config = ModelConfig(**checkpoint["config"]["model"])
        config.validate()
        state = checkpoint["model"]
        if dtype is None:
            dtype = state["lm_head.weight"].dtype
        model = cls.from_config(config, device="meta", dtype=dtype)
        model = model.to_empty(device=device or "cpu")
        model.load_state_dict({k: v.to(dtype) for k, v in state.items()}, strict=True)
        return model

    @property
    def head_dim(self) -> int:
        return self.d_model // self.num_heads

    def _gemm_prefill(self) -> bool:
        """Models whose head dim the prefill attention supports prefill in one pass (16-bit: the
        masked MFMA kernel, head dims 32/64/128; float32: the fp32 kernel, 16/32/64/128)."""
        if self.lm_head.weight.dtype == torch.float32:
            return self.head_dim in (16, 32, 64, 128)
        return self.head_dim in (32, 64, 128)

    def _check_ids(self, input_ids: torch.Tensor) -> None:
        if input_ids.ndim < 1:
            raise ValueError("input_ids must have a sequence dimension")
        if not 0 < input_ids.shape[-1] <= self.context_length:
            raise ValueError("sequence length must be between 1 and context_length")

    def decode_session(self, batch: int, capacity: int, *, record_logits: bool = False,
                       deterministic: bool | None = None) -> "_engine.DecodeSession":
        """A ``DecodeSession`` of at least ``capacity`` positions for ``batch`` sequences.

        The last session is kept and reused by later calls with the same batch,
        logits recording and determinism and no larger capacity, while the
        parameters are unchanged; its packed weights are shared through
        ``engine.decode_weights`` (remade only after a parameter changes), so
        repeated ``forward``/``generate`` calls neither repack weights nor
        reallocate the KV cache.
        """
        if deterministic is None:
            deterministic = _engine.default_deterministic(self.lm_head.weight.dtype)
        session = getattr(self, "_sfl_session", None)
        reuse = (session is not None and session.batch == batch and capacity <= session.cap
                 and (session.logits is not None) == record_logits and session.deterministic == deterministic
                 and session.weights is _engine.decode_weights(self))
        if not reuse:
            self._sfl_session = None  # free the previous KV cache first
            session = self._sfl_session = _engine.DecodeSession(
                self, batch=batch, capacity=capacity, record_logits=record_logits, deterministic=deterministic)
        return session

    def release_sessions(self) -> None:
        """Free the device memory ``forward``/``generate`` keep between calls.

        The last ``DecodeSession`` (its KV cache ``[L, B, H, cap, dk]``, and on
        the step path a ``[B, cap, vocab]`` fp32 logits buffer) and the packed
        decode weights (about one more copy of the projection weights) stay
        allocated so that repeated calls reuse them; this drops both. The next
        call makes them again.
        """
        self._sfl_session = None
        self._sfl_decode_weights = None

    @torch.no_grad()
    def forward(self, input_ids: torch.Tensor) -> torch.Tensor:
        """Logits ``[..., T, vocab]`` for every position (``transformer.py:121-139``)."""
        self._check_ids(input_ids)
        lead = input_ids.shape[:-1]
        ids = input_ids.reshape(-1, input_ids.shape[-1])
        t = ids.shape[-1]
        if self._gemm_prefill():
            # One pass of MFMA GEMMs and masked attention over the whole prompt.
            session = self.decode_session(ids.shape[0], t, deterministic=self.deterministic)
            logits = session.prefill(ids, all_logits=True, logits_dtype=self.lm_head.weight.dtype)
            return logits.reshape(*lead, t, self.vocab_size)
        session = self.decode_session(ids.shape[0], t, record_logits=True, deterministic=self.deterministic)
        session.start(ids)
        session.run(t)
        # The reference returns logits in the parameter dtype (transformer.py:138), a new
        # tensor every call: copy out of the session's buffer, which the next call reuses.
        logits = session.logits[:, :t].to(self.lm_head.weight.dtype, copy=True)
        return logits.reshape(*lead, t, self.vocab_size)

    @torch.no_grad()
    def generate(self, input_ids: torch.Tensor, max_new_tokens: int, *, use_graph: bool = True,
                 capacity: int | None = None) -> torch.Tensor:
        """Greedy continuation: ids ``[B, T + max_new_tokens]`` (argmax, first index on ties).

        NaN logits are never chosen (``torch.argmax`` would return a NaN's
        index); a row whose logits are all NaN continues with token 0.
        ``capacity`` (default T + max_new_tokens) sizes the KV cache and must
        hold the whole result.
        """
        self._check_ids(input_ids)
        if input_ids.ndim != 2:
            raise ValueError("generate expects input_ids of shape [batch, sequence]")
        total = input_ids.shape[1] + max_new_tokens
        if max_new_tokens < 0 or total > self.context_length:
            raise ValueError("sequence length must be between 1 and context_length")
        if capacity is not None and not total <= capacity <= self.context_length:
            raise ValueError("capacity must be in [prompt length + max_new_tokens, context_length]")
        session = self.decode_session(input_ids.shape[0], capacity or total, deterministic=self.deterministic)
        if self._gemm_prefill() and max_new_tokens > 0:
            session.prefill(input_ids)  # positions 0..T-1 at once; token T chosen
            session.run(max_new_tokens - 1, use_graph=use_graph)
        else:
            session.start(input_ids)
            session.run(total - 1, use_graph=use_graph)
        return session.tokens[:, :total].clone()
