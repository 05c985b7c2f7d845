"""Device-resident greedy token loop for ``TransformerLM`` on gfx950.

A ``DecodeSession`` owns everything one decode step touches -- packed weights,
the KV cache ``[L, B, H, cap, dk]`` in the model dtype, the fp32 residual
stream, scratch, and the token/position/length state -- and issues one step as
a fixed sequence of C-ABI launches on the current stream:

    per layer:  rmsnorm_qkv_rope_append -> decode_attention_out_proj
                -> rmsnorm_swiglu -> linear_residual (w2)
    then:       rmsnorm_lm_head (+ tile argmax) -> next_token

With more than one KV split the attention and output_proj run as
decode_attention (split-KV + merge) and linear_residual instead.

RMSNorm is folded into its consumer: x stays a plain fp32 tensor, and the
q/k/v, w1/w3 and lm_head GEMVs read it with their norm's gain, forming x * g
and the sum of x^2 as they go. The producers of x only add to it, so the
output projection is accumulated by the attention workgroups and w2 is split
along K over several workgroups, both with fp32 atomics.

All step state lives in device memory and is advanced by ``next_token``, so a
step has no host inputs: it is captured once into a HIP graph and replayed.
While a sequence is inside its prompt, ``next_token`` keeps the prompt token
(teacher forcing) and still records the model's argmax in ``predicted``.

The reference has no KV cache or token loop (``transformer.py:121-139``
recomputes from position 0); this loop reproduces
``argmax(forward(ids)[:, -1])`` one position at a time.
"""

from __future__ import annotations

import torch

from . import _lib
from .decode import auto_splits

ROW_BLOCK = 16  # batch rows per GEMV workgroup (the activation layout's block)


def residual_ksplit(n: int, target_groups: int = 256) -> int:
    """Workgroups per 16-row tile along K for a residual GEMV with ``n`` outputs.

    ``n / 16`` tiles cover few of the 256 CUs at these model widths (64 at
    d_model 1024); the K parts add their partial sums into x with atomics.
    """
    return max(1, min(16, target_groups // max(1, n // 16)))


def default_deterministic(dtype) -> bool:
    """Whether a session runs the one-writer decode path when the caller does not say.

    float32 models do: their greedy ids are checked for identity with the
    reference, so they must not depend on the order in which the fused path's
    fp32 atomics add the heads' output projections (or w2's K parts) into x.
    16-bit models take the faster fused path; its run-to-run differences are
    fp32 reassociation, far below their storage rounding.
    """
    return dtype == torch.float32


def parameter_version(model) -> tuple:
    """Changes whenever a parameter is replaced or modified in place (``Tensor._version``)."""
    return tuple((p.data_ptr(), p._version, p.dtype, p.device) for p in model.parameters())


class DecodeWeights:
    """Device copies of a model's weights in the layouts the kernels read, made once.

    ``wqkv``: ``[q; k; v]`` stacked, ``[3d, d]`` (prefill GEMM); ``p_*``: every
    projection in the decode GEMVs' packed tile layout (one contiguous 1 KB
    block per 16 rows x K chunk); ``w13``: W1/W3 interleaved in blocks of 8
    rows, the layout the prefill SwiGLU GEMM pairs in-lane (made on first use).
    ``version`` is the model's ``parameter_version`` when they were made.
    """

    def __init__(self, model):
        self.version = parameter_version(model)
        self.model = model
        self.wqkv = [torch.cat([blk.attn.q_proj.weight, blk.attn.k_proj.weight, blk.attn.v_proj.weight])
                     .contiguous() for blk in model.layers]
        pk = _lib.pack_gemv
        self.p_qkv = [pk(w) for w in self.wqkv]
        self.p_out = [pk(blk.attn.output_proj.weight) for blk in model.layers]
        self.p_w1 = [pk(blk.ffn.w1.weight) for blk in model.layers]
        self.p_w3 = [pk(blk.ffn.w3.weight) for blk in model.layers]
        self.p_w2 = [pk(blk.ffn.w2.weight) for blk in model.layers]
        self.p_head = pk(model.lm_head.weight)
        self._w13 = None

    def w13(self):
        if self._w13 is None:
            f, d = self.model.d_ff, self.model.d_model
            self._w13 = [torch.stack([blk.ffn.w1.weight.view(f // 8, 8, d), blk.ffn.w3.weight.view(f // 8, 8, d)],
                                     dim=1).reshape(2 * f, d).contiguous() for blk in self.model.layers]
        return self._w13


def decode_weights(model) -> DecodeWeights:
    """The model's ``DecodeWeights``, remade only after a parameter changed."""
    cached = getattr(model, "_sfl_decode_weights", None)
    if cached is None or cached.version != parameter_version(model):
        model._sfl_decode_weights = None  # drop the stale copies before packing anew
        cached = model._sfl_decode_weights = DecodeWeights(model)
    return cached


class DecodeSession:
    def __init__(self, model, batch: int, capacity: int | None = None, *, splits: int | None = None,
                 record_logits: bool = False, deterministic: bool | None = None):
        param = model.lm_head.weight
        if param.device.type != "cuda":
            raise RuntimeError("systems_for_llms_amd runs on the GPU: move the model to a HIP device first")
        if param.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            raise TypeError("model dtype must be float32, bfloat16 or float16")
        _lib.lib()
        cap = capacity or model.context_length
        if not 0 < cap <= model.context_length:
            raise ValueError("capacity must be in [1, context_length]")
        if model.d_model % 32 or model.d_ff % 32:
            raise ValueError("the decode step needs d_model and d_ff to be multiples of 32")
        self.model = model
        self.device = param.device
        self.dtype = param.dtype
        self.code = _lib.dtype_code(self.dtype)
        self.batch, self.cap = batch, cap
        d, h, f, v, n = model.d_model, model.num_heads, model.d_ff, model.vocab_size, model.num_layers
        self.d, self.heads, self.dk, self.d_ff, self.vocab, self.layers = d, h, d // h, f, v, n
        dev, dt = self.device, self.dtype

        from .model import rope_tables
        cos, sin = rope_tables(model.theta, self.dk, cap)
        self.cos, self.sin = cos.to(dev), sin.to(dev)
        # The prefill GEMMs take the tables feature-major ([dk/2, cap]).
        self.cos_fm, self.sin_fm = self.cos.t().contiguous(), self.sin.t().contiguous()
        # Packed copies shared by every session of this model while its parameters are
        # unchanged; the session keeps a reference, so its captured launches stay valid.
        self.weights = w = decode_weights(model)
        self.wqkv, self.p_qkv, self.p_out = w.wqkv, w.p_qkv, w.p_out
        self.p_w1, self.p_w3, self.p_w2, self.p_head = w.p_w1, w.p_w3, w.p_w2, w.p_head
        self.k_cache = torch.zeros((n, batch, h, cap, self.dk), device=dev, dtype=dt)
        self.v_cache = torch.zeros_like(self.k_cache)
        self.x = torch.zeros((batch, d), device=dev, dtype=torch.float32)
        # Only weights and the KV cache use the model dtype. x and q are fp32; the
        # GEMV inputs (attention output, SwiGLU hidden) are 4 bytes per value:
        # fp32 for fp32 models, the split-bf16 (hi, lo) format for bf16 models.
        self.q = torch.zeros((batch, h, self.dk), device=dev, dtype=torch.float32)
        # GEMV inputs in the activation layout: whole blocks of 16 rows, 4 bytes per
        # value (viewed here as fp32 words): the attention output (only when the
        # attention is not fused with output_proj) and the SwiGLU hidden state.
        # The normalized consumers read x itself with their RMSNorm gain.
        blocks = -(-batch // ROW_BLOCK)
        self.attn = torch.zeros((blocks, ROW_BLOCK * d), device=dev, dtype=torch.float32)
        self.hidden = torch.zeros((blocks, ROW_BLOCK * f), device=dev, dtype=torch.float32)
        self.act_code = {torch.bfloat16: _lib.DTYPE_BF16X2, torch.float16: _lib.DTYPE_F16X2}.get(dt, _lib.DTYPE_F32X)
        if deterministic is None:
            deterministic = default_deterministic(dt)
        self.deterministic = deterministic
        # GEMM prefill with each layer's RMSNorm folded into the GEMMs beside it
        # (where the 32x32 MFMA kernels take every shape); see ``prefill``.
        self.fold_prefill_norm = True
        self.prefill_norm_folded = False  # whether the last prefill did
        self.splits = splits or auto_splits(batch, h, cap)
        self.pmax = torch.empty((batch, h, self.splits), device=dev, dtype=torch.float32)
        self.psum = torch.empty_like(self.pmax)
        self.pout = torch.empty((batch, h, self.splits, self.dk), device=dev, dtype=torch.float32)
        self.tiles = _lib.lib().sfl_lm_head_tiles(v)
        self.best_val = torch.empty((self.tiles, batch), device=dev, dtype=torch.float32)
        self.best_idx = torch.empty((self.tiles, batch), device=dev, dtype=torch.int32)
        self.tokens = torch.zeros((batch, cap), device=dev, dtype=torch.int64)
        self.predicted = torch.full((batch, cap), -1, device=dev, dtype=torch.int64)
        self.pos = torch.zeros(batch, device=dev, dtype=torch.int32)
        self.lengths = torch.ones(batch, device=dev, dtype=torch.int32)
        self.prompt_len = torch.ones(batch, device=dev, dtype=torch.int32)
        self.logits = (torch.zeros((batch, cap, v), device=dev, dtype=torch.float32)
                       if record_logits else None)
        # One split: the attention kernel also applies output_proj and adds it to x
        # (fp32 atomics from the 16 heads: the summation order varies from run to run).
        # deterministic=True keeps output_proj and w2 as plain GEMVs whose every output
        # has one writer, so repeated runs give bit-identical logits.
        self.fused_out_proj = not deterministic and self.splits == 1 \
            and self.dk % (16 if dt == torch.float32 else 32) == 0 and self.dk <= 128 and self.dk & (self.dk - 1) == 0
        self.ksplit = 1 if deterministic else residual_ksplit(d)
        self.position = 0  # host mirror of every row's position (all rows move together)
        self.graph = None
        self._calls = self._plan()

    # -- launch plan --------------------------------------------------------
    def _plan(self):
        """The ctypes calls of one step over every row, in launch order."""
        bufs = {"attn": self.attn, "hidden": self.hidden, "pmax": self.pmax, "psum": self.psum,
                "pout": self.pout, "best_val": self.best_val, "best_idx": self.best_idx}
        layers, tail = self._plan_rows(0, self.batch, bufs, self.splits, self.fused_out_proj)
        return [call for layer in layers for call in layer] + tail

    def _plan_rows(self, r0, nb, bufs, splits, fused):
        """One step's ctypes calls (every argument but the stream bound) for rows
        r0 .. r0 + nb - 1: ``(layers, tail)``, where ``layers[i]`` lists layer i's
        launches, and ``tail`` is the lm_head and
        the token step."""
        lib = _lib.lib()
        d, h, dk, f, v, cap, code = self.d, self.heads, self.dk, self.d_ff, self.vocab, self.cap, self.code
        m = self.model
        scale = float(dk) ** -0.5
        x, q = self.x[r0:].data_ptr(), self.q[r0:].data_ptr()
        pos, lengths = self.pos[r0:].data_ptr(), self.lengths[r0:].data_ptr()
        attn, hidden = bufs["attn"].data_ptr(), bufs["hidden"].data_ptr()
        layers = []
        for layer, blk in enumerate(m.layers):
            kc, vc = self.k_cache[layer, r0:].data_ptr(), self.v_cache[layer, r0:].data_ptr()
            calls = [(lib.sfl_rmsnorm_qkv_rope_append, (
                x, blk.attn_norm.weight.data_ptr(), self.p_qkv[layer].data_ptr(), self.cos.data_ptr(),
                self.sin.data_ptr(), pos, q, kc, vc, nb, d, h, cap, code))]
            if fused:
                calls.append((lib.sfl_decode_attention_out_proj, (
                    q, kc, vc, lengths, self.p_out[layer].data_ptr(), x, nb, h, cap, dk, scale, code)))
            else:
                calls.append((lib.sfl_decode_attention, (
                    q, kc, vc, lengths, bufs["pmax"].data_ptr(), bufs["psum"].data_ptr(), bufs["pout"].data_ptr(),
                    attn, nb, h, h, cap, dk, splits, scale, code, _lib.DTYPE_CODES[torch.float32],
                    self.act_code)))
                calls.append((lib.sfl_linear_residual, (
                    attn, self.p_out[layer].data_ptr(), x, nb, d, d, self.ksplit, code)))
            calls.append((lib.sfl_rmsnorm_swiglu, (
                x, blk.ffn_norm.weight.data_ptr(), self.p_w1[layer].data_ptr(), self.p_w3[layer].data_ptr(),
                hidden, nb, d, f, code)))
            calls.append((lib.sfl_linear_residual, (hidden, self.p_w2[layer].data_ptr(), x, nb, d, f,
                                                    self.ksplit, code)))
            layers.append(calls)
        logits = self.logits[r0:].data_ptr() if self.logits is not None else None
        tail = [(lib.sfl_rmsnorm_lm_head, (
                    x, m.ln_final.weight.data_ptr(), self.p_head.data_ptr(), logits, cap * v, pos, v,
                    bufs["best_val"].data_ptr(), bufs["best_idx"].data_ptr(), nb, nb, d, v, code)),
                (lib.sfl_next_token, (
                    bufs["best_val"].data_ptr(), bufs["best_idx"].data_ptr(), self.tiles, nb,
                    self.tokens[r0:].data_ptr(), self.predicted[r0:].data_ptr(), cap,
                    self.prompt_len[r0:].data_ptr(), pos, lengths, m.token_embeddings.weight.data_ptr(), x,
                    nb, d, cap, code))]
        return layers, tail

    # -- state --------------------------------------------------------------
    @torch.no_grad()
    def start(self, prompt: torch.Tensor, forced_length: int | None = None) -> None:
        """Load ``prompt [B, T]`` and set every row to position 0.

        Positions below ``forced_length`` (default T) keep the given token; the
        step at position p writes the next token at p + 1.
        """
        if prompt.shape[0] != self.batch or not 0 < prompt.shape[1] <= self.cap:
            raise ValueError("prompt must be [batch, T] with 0 < T <= capacity")
        low, high = torch.aminmax(prompt)
        if low.item() < 0 or high.item() >= self.vocab:
            raise ValueError("token ids must be in [0, vocab_size)")
        self.tokens.zero_()
        self.tokens[:, :prompt.shape[1]] = prompt.to(self.device)
        self.predicted.fill_(-1)
        self.pos.zero_()
        self.lengths.fill_(1)
        self.prompt_len.fill_(forced_length or prompt.shape[1])
        self.position = 0
        self._embed_current()

    def _embed_current(self) -> None:
        """x = embedding of each row's token at pos."""
        stream = _lib.stream_handle(self.device)
        _lib.call("sfl_embedding_gather", self.tokens.data_ptr(), self.cap, self.pos.data_ptr(),
                  self.model.token_embeddings.weight.data_ptr(), self.x.data_ptr(), self.batch,
                  self.d, self.code, stream)

    # -- prefill ------------------------------------------------------------
    @torch.no_grad()
    def prefill(self, prompt: torch.Tensor, all_logits: bool = False,
                forced: torch.Tensor | None = None, logits_dtype=torch.float32) -> torch.Tensor | None:
        """Process ``prompt [B, T]`` with MFMA GEMMs and masked attention, then pick token T.

        Fills the KV cache at positions 0..T-1, computes the logits of position
        T-1 with the decode head, and leaves every row at position T (the next
        token written, embedded and ready for ``step``). With ``all_logits`` it
        also returns logits ``[B, T, V]`` for every position (the reference's
        ``forward``). 16-bit models store their GEMM inputs in the model dtype;
        float32 models run the same pass in fp32 (fp32 MFMA GEMMs, fp32
        attention, separate norm passes). ``forced [B, L]`` (L > T, starting
        with the prompt) makes the following positions up to L teacher-forced.
        ``logits_dtype`` (float32 or the model dtype) is the type the
        all-positions lm_head GEMM stores: a 16-bit model dtype rounds its fp32
        sums once, as a cast of the fp32 logits would, with half the stores and
        no cast pass.
        """
        b, t = prompt.shape
        if b != self.batch or not 0 < t <= self.cap:
            raise ValueError("prompt must be [batch, T] with 0 < T <= capacity")
        if logits_dtype not in (torch.float32, self.dtype):
            raise TypeError("logits_dtype must be torch.float32 or the model dtype")
        low, high = torch.aminmax(prompt)
        if low.item() < 0 or high.item() >= self.vocab:
            raise ValueError("token ids must be in [0, vocab_size)")
        from .attention import causal_prefill

        d, h, dk, f, v = self.d, self.heads, self.dk, self.d_ff, self.vocab
        m_rows = b * t
        F32 = _lib.DTYPE_CODES[torch.float32]
        dev, code = self.device, self.code
        w13 = self.weights.w13()
        self.tokens.zero_()
        self.tokens[:, :t] = prompt.to(dev)
        self.predicted.fill_(-1)
        self.prompt_len.fill_(t)
        if forced is not None:
            if forced.shape[0] != b or not t <= forced.shape[1] <= self.cap:
                raise ValueError("forced must be [batch, L] with T <= L <= capacity")
            self.tokens[:, :forced.shape[1]] = forced.to(dev)
            self.prompt_len.fill_(forced.shape[1])
        ids = self.tokens[:, :t].contiguous().view(-1)
        if self.dtype == torch.float32:
            return self._prefill_f32(ids, b, t, all_logits)
        x = torch.empty((m_rows, d), device=dev, dtype=torch.float32)
        act = torch.empty((m_rows, d), device=dev, dtype=self.dtype)
        q = torch.empty((b, h, t, dk), device=dev, dtype=self.dtype)
        attn = torch.empty((b, t, h, dk), device=dev, dtype=self.dtype)
        hid = torch.empty((m_rows, f), device=dev, dtype=self.dtype)
        st = _lib.stream_handle(dev)
        call = _lib.call
        call("sfl_embed_rows", ids.data_ptr(), self.model.token_embeddings.weight.data_ptr(), x.data_ptr(),
             m_rows, d, code, st)
        # Folded norms: a layer's GEMM input is T(x * g) and the GEMM scales its
        # products by 1 / rms(x); the residual GEMM that updates x also writes the
        # next norm's input and per-128-feature sums of x^2 (one more small kernel
        # turns them into the scales), so no pass of its own re-reads x.
        self.prefill_norm_folded = fold = self._fold_norm(m_rows)
        layers = self.model.layers
        if fold:
            parts = -(-d // 128)
            ss = torch.empty((parts, m_rows), device=dev, dtype=torch.float32)
            rsc = torch.empty((m_rows,), device=dev, dtype=torch.float32)
            call("sfl_rmsnorm_rows_scaled", x.data_ptr(), layers[0].attn_norm.weight.data_ptr(), act.data_ptr(),
                 rsc.data_ptr(), m_rows, d, code, st)
        for layer, blk in enumerate(layers):
            kc, vc = self.k_cache[layer], self.v_cache[layer]
            if fold:
                call("sfl_gemm_qkv_rope_scaled", act.data_ptr(), self.wqkv[layer].data_ptr(), rsc.data_ptr(), m_rows,
                     t, d, h, self.cos_fm.data_ptr(), self.sin_fm.data_ptr(), q.data_ptr(), kc.data_ptr(),
                     vc.data_ptr(), self.cap, code, st)
            else:
                call("sfl_rmsnorm_rows", x.data_ptr(), blk.attn_norm.weight.data_ptr(), act.data_ptr(), m_rows, d,
                     code, code, st)
                call("sfl_gemm_qkv_rope", act.data_ptr(), self.wqkv[layer].data_ptr(), m_rows, t, d, h,
                     self.cos_fm.data_ptr(), self.sin_fm.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                     self.cap, code, st)
            causal_prefill(q, kc[:, :, :t], vc[:, :, :t], attn.transpose(1, 2))
            if fold:
                call("sfl_gemm_residual_norm", attn.data_ptr(), blk.attn.output_proj.weight.data_ptr(), x.data_ptr(),
                     m_rows, d, d, blk.ffn_norm.weight.data_ptr(), act.data_ptr(), ss.data_ptr(), code, st)
                call("sfl_norm_scale", ss.data_ptr(), parts, m_rows, d, rsc.data_ptr(), st)
                call("sfl_gemm_swiglu_scaled", act.data_ptr(), w13[layer].data_ptr(), rsc.data_ptr(), hid.data_ptr(),
                     m_rows, f, d, code, st)
            else:
                call("sfl_gemm", attn.data_ptr(), blk.attn.output_proj.weight.data_ptr(), x.data_ptr(),
                     m_rows, d, d, code, F32, 1, st)
                call("sfl_rmsnorm_rows", x.data_ptr(), blk.ffn_norm.weight.data_ptr(), act.data_ptr(), m_rows, d,
                     code, code, st)
                call("sfl_gemm_swiglu", act.data_ptr(), w13[layer].data_ptr(), hid.data_ptr(), m_rows, f, d, code, st)
            if fold and layer + 1 < len(layers):
                call("sfl_gemm_residual_norm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m_rows,
                     d, f, layers[layer + 1].attn_norm.weight.data_ptr(), act.data_ptr(), ss.data_ptr(), code, st)
                call("sfl_norm_scale", ss.data_ptr(), parts, m_rows, d, rsc.data_ptr(), st)
            else:
                call("sfl_gemm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m_rows, d, f, code, F32,
                     1, st)
        logits = None
        if all_logits:
            call("sfl_rmsnorm_rows", x.data_ptr(), self.model.ln_final.weight.data_ptr(), act.data_ptr(),
                 m_rows, d, code, code, st)
            logits = torch.empty((m_rows, v), device=dev, dtype=logits_dtype)
            call("sfl_gemm", act.data_ptr(), self.model.lm_head.weight.data_ptr(), logits.data_ptr(),
                 m_rows, v, d, code, _lib.dtype_code(logits_dtype), 0, st)
            logits = logits.view(b, t, v)
        self._hand_over(x, b, t, st)
        return logits

    def _hand_over(self, x, b, t, st) -> None:
        """Hand the prompt's last position to the decode head: pick token T and advance."""
        self.x.copy_(x.view(b, t, self.d)[:, t - 1])
        self.pos.fill_(t - 1)
        self.lengths.fill_(t)
        self.position = t
        for fn, args in self._calls[-2:]:  # the lm_head and the token step
            status = fn(*args, st)
            if status != 0:
                raise RuntimeError(f"{fn.__name__} failed ({status}): "
                                   f"{_lib.lib().sfl_last_error().decode(errors='replace')}")

    def _prefill_f32(self, ids, b, t, all_logits):
        """``prefill`` of a float32 model: the reference's fp32 forward (transformer.py:121-139)
        as one pass of fp32 MFMA GEMMs (q/k/v + RoPE + cache, output_proj + residual, SwiGLU,
        w2 + residual) and fp32 causal attention, the norms as separate fp32 passes."""
        from .attention import causal_prefill

        d, h, dk, f, v = self.d, self.heads, self.dk, self.d_ff, self.vocab
        m_rows, dev, F32 = b * t, self.device, _lib.DTYPE_CODES[torch.float32]
        w13 = self.weights.w13()
        x = torch.empty((m_rows, d), device=dev, dtype=torch.float32)
        act = torch.empty((m_rows, d), device=dev, dtype=torch.float32)
        q = torch.empty((b, h, t, dk), device=dev, dtype=torch.float32)
        attn = torch.empty((b, t, h, dk), device=dev, dtype=torch.float32)
        hid = torch.empty((m_rows, f), device=dev, dtype=torch.float32)
        st = _lib.stream_handle(dev)
        call = _lib.call
        call("sfl_embed_rows", ids.data_ptr(), self.model.token_embeddings.weight.data_ptr(), x.data_ptr(), m_rows, d,
             F32, st)
        for layer, blk in enumerate(self.model.layers):
            kc, vc = self.k_cache[layer], self.v_cache[layer]
            call("sfl_rmsnorm_rows", x.data_ptr(), blk.attn_norm.weight.data_ptr(), act.data_ptr(), m_rows, d, F32,
                 F32, st)
            call("sfl_gemm_qkv_rope", act.data_ptr(), self.wqkv[layer].data_ptr(), m_rows, t, d, h,
                 self.cos_fm.data_ptr(), self.sin_fm.data_ptr(), q.data_ptr(), kc.data_ptr(), vc.data_ptr(),
                 self.cap, F32, st)
            causal_prefill(q, kc[:, :, :t], vc[:, :, :t], attn.transpose(1, 2))
            call("sfl_gemm", attn.data_ptr(), blk.attn.output_proj.weight.data_ptr(), x.data_ptr(), m_rows, d, d,
                 F32, F32, 1, st)
            call("sfl_rmsnorm_rows", x.data_ptr(), blk.ffn_norm.weight.data_ptr(), act.data_ptr(), m_rows, d, F32,
                 F32, st)
            call("sfl_gemm_swiglu", act.data_ptr(), w13[layer].data_ptr(), hid.data_ptr(), m_rows, f, d, F32, st)
            call("sfl_gemm", hid.data_ptr(), blk.ffn.w2.weight.data_ptr(), x.data_ptr(), m_rows, d, f, F32, F32, 1,
                 st)
        logits = None
        if all_logits:
            call("sfl_rmsnorm_rows", x.data_ptr(), self.model.ln_final.weight.data_ptr(), act.data_ptr(), m_rows, d,
                 F32, F32, st)
            logits = torch.empty((m_rows, v), device=dev, dtype=torch.float32)
            call("sfl_gemm", act.data_ptr(), self.model.lm_head.weight.data_ptr(), logits.data_ptr(), m_rows, v, d,
                 F32, F32, 0, st)
            logits = logits.view(b, t, v)
        self.prefill_norm_folded = False
        self._hand_over(x, b, t, st)
        return logits

    def _fold_norm(self, m_rows: int) -> bool:
        """Whether ``prefill`` folds the norms: the 32x32 MFMA GEMMs take every shape
        (K multiples of 64, operands under 2^30 elements) and the norm kernel d_model."""
        d, f, lim = self.d, self.d_ff, 1 << 30
        return (self.fold_prefill_norm and d % 64 == 0 and f % 64 == 0 and d <= 2048
                and m_rows * max(d, f) < lim and 3 * d * d < lim and 2 * f * d < lim)

    def set_position(self, position: int) -> None:
        """Rewind/advance every row to ``position`` (the cache below it is kept) and re-embed."""
        if not 0 <= position < self.cap:
            raise ValueError(f"position must be in [0, capacity={self.cap})")
        self.pos.fill_(position)
        self.lengths.fill_(position + 1)
        self.position = position
        self._embed_current()

    def _advance(self, steps: int) -> None:
        """Account for ``steps`` steps; the last may run at position capacity - 1.

        A step at position p appends K/V at p and picks token p + 1; at
        p = capacity - 1 it still produces the logits of p but records no token
        and leaves the device position where it is, so no further step may run
        until the session is restarted or rewound.
        """
        if self.position + steps > self.cap:
            raise ValueError(f"{steps} steps from position {self.position} run past capacity {self.cap}")
        self.position += steps

    # -- execution ----------------------------------------------------------
    def step(self) -> None:
        """Launch one decode step on the current stream (no host synchronisation)."""
        self._advance(1)
        self._launch()

    def _launch(self) -> None:
        self._launch_calls(self._calls)

    def _launch_calls(self, calls) -> None:
        stream = _lib.stream_handle(self.device)
        for fn, args in calls:
            status = fn(*args, stream)
            if status != 0:
                raise RuntimeError(f"{fn.__name__} failed ({status}): "
                                   f"{_lib.lib().sfl_last_error().decode(errors='replace')}")

    def capture(self, steps_per_graph: int = 1) -> torch.cuda.CUDAGraph:
        """Capture ``steps_per_graph`` steps into one HIP graph (replayable, state on device).

        Capturing records the launches without executing them; ``replay`` runs
        ``steps_per_graph`` steps from wherever the device state stands.
        """
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(steps_per_graph):
                self._launch()
        self.graph, self.graph_steps = graph, steps_per_graph
        return graph

    def replay(self) -> None:
        """Replay the captured graph (``graph_steps`` steps)."""
        self._advance(self.graph_steps)
        self.graph.replay()

    def run(self, steps: int, use_graph: bool = False) -> None:
        """Advance every row by ``steps`` positions (graph replays when ``use_graph``)."""
        if steps <= 0:
            return
        self._advance(steps)  # checked up front: nothing launches if it would overrun
        self.position -= steps
        if not use_graph:
            for _ in range(steps):
                self.step()
            return
        # Warm up eagerly once (first-call kernel attributes), then capture.
        self.step()
        steps -= 1
        if steps == 0:
            return
        if self.graph is None or self.graph_steps != 1:
            self.capture(1)
        for _ in range(steps):
            self.replay()
