"""Decode throughput of the 324.1M llmlab decoder on one MI355X.

Workload: d_model 1024, 24 layers, 16 heads of 64, SwiGLU d_ff 2752, vocab
10000, bf16 weights N(0, 0.02) from seed 1337; batch 16; 3072 uniform random
prompt tokens (seed 2027) are prefilled, then greedy decode runs to context
4096. The prompt is prefilled in one pass (MFMA GEMMs + masked attention),
which also picks token 3072. One step = one decode position for all 16
sequences (16 tokens), replayed from a captured HIP graph. The K timed steps
are centred on the decode's mean attention length (3584: lengths run 3073 ..
4095 over the 1023 steps from position 3072 to context 4096), so a short run
measures the same per-step cost as the whole range: they start at position
3584 - (K+1)//2 (3072 for the default K = 1023, the full range). Untimed
decode steps first fill the cache and tokens up to that position (at least W
of them; the state is rewound when W runs past it).

Printed JSON (one line): decode tok/s; ``roofline`` for the dominant kernel,
decode attention fused with the output projection (the model path's kernel),
timed with HIP events on its launch stream at the decode's mean attention
length 3584, rotating over the 24 layers' caches so that every call streams
from HBM as it does inside the decode loop; ``decode_attention_operator``: the
same measurement for the standalone split-KV attention operator; ``prefill``
(the prompt pass, MFMA TFLOP/s against the bf16 dense peak);
``decode_attention_config4`` and ``masked_attention_config5`` (BASELINE
configs 4 and 5 as operator microbenchmarks); ``cpu_baseline``: the CPU
oracle's KV-cached decode step on this host's cores on a bounded sample, and
``cpu_reference_semantics``: one full-recompute forward over the prompt, as the
reference produces a token.

    python bench.py [--steps K] [--warmup W] [--gpus 1] [--no-cpu-baseline] [--no-reference-shapes]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
MFMA_BF16_PEAK_TFLOPS = 2500.0
PROMPT = 3072
CONTEXT = 4096
MEAN_LEN = (PROMPT + 1 + CONTEXT - 1) // 2  # mean attention length of the decode, 3584
BATCH = 16
WEIGHT_SEED, PROMPT_SEED = 1337, 2027


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def attention_bytes(lengths, heads, dim, elem=2, q_elem=4):
    """Algorithmic decode-attention bytes: K+V rows up to each length, plus q read and out write."""
    return sum(int(n) for n in lengths) * heads * dim * 2 * elem + len(lengths) * heads * dim * 2 * q_elem


def fused_attention_bytes(lengths, heads, dim, d_model, w_elem=2):
    """Algorithmic bytes of attention + output projection: K+V rows, q (fp32), W_o, x read and write."""
    kv = sum(int(n) for n in lengths) * heads * dim * 2 * w_elem
    return kv + len(lengths) * heads * dim * 4 + d_model * d_model * w_elem + 2 * len(lengths) * d_model * 4


def step_bytes(cfg, batch, length):
    """Algorithmic HBM bytes of one decode step at attention length ``length`` (bf16)."""
    weights = 2 * (cfg.parameter_count() - cfg.vocab_size * cfg.d_model)
    kv_read = cfg.num_layers * batch * length * 2 * cfg.d_model * 2
    kv_append = cfg.num_layers * batch * 2 * cfg.d_model * 2
    return weights + kv_read + kv_append


def prefill_flops(cfg, batch, length):
    """MFMA work of the prefill: the per-layer GEMMs over B*T rows, the mask-exact
    causal attention (QK^T and PV, 4*dk flops per admissible pair), and the head
    for the last row of each sequence (the only row the decode loop needs)."""
    rows = batch * length
    d, f = cfg.d_model, cfg.d_ff
    gemm = 2 * rows * cfg.num_layers * (4 * d * d + 3 * d * f) + 2 * batch * d * cfg.vocab_size
    attention = 4 * cfg.head_dim * (length * (length + 1) // 2) * batch * cfg.num_heads * cfg.num_layers
    return gemm, attention


def time_events(fn, reps):
    import torch

    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / reps


def time_graph(fn, inner=10, reps=12):
    """Median per-call time of ``inner`` calls captured in one HIP graph.

    The protocol of ``attention_lab/benchmark.py:42-84``: warm up eagerly,
    capture a batch of calls, replay it ``reps`` times with events around each
    replay and take the median, so host-side argument handling is not timed.
    """
    import torch

    fn()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(inner):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(reps):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        end.synchronize()
        times.append(start.elapsed_time(end) / inner)
    return sorted(times)[len(times) // 2]


# The reference's published attention timings (H100 80GB HBM3):
# cuda_decode rows as (B, Hq, Hkv, N, D, custom us, Flash SDPA us) from
# attention_lab/results/h100-extensions-20261105/decode/study/benchmark.json, and
# interval-schedule masked attention (B=1, H=8, N=4096) as (D, mask, us) from the
# h100-20261104 ablation cases.
H100_DECODE = ((1, 32, 4, 1024, 128, 11.0, 10.1), (1, 32, 4, 4096, 128, 28.7, 15.8),
               (1, 32, 4, 16384, 128, 141.4, 27.6), (1, 32, 4, 65536, 128, 653.8, 63.8),
               (8, 32, 4, 4096, 128, 108.8, 33.2), (8, 32, 4, 16384, 128, 410.2, 99.9),
               (32, 32, 4, 4096, 128, 360.0, 96.7), (1, 16, 16, 16384, 64, 174.0, 33.6),
               (1, 32, 8, 4096, 64, 30.6, 13.6), (8, 32, 8, 4096, 64, 77.8, 31.5))
H100_MASKED = ((64, "causal", 100.0), (128, "causal", 139.2), (64, "causal, window_left 127", 10.6),
               (128, "causal, window_left 127", 18.5))


def published_shapes():
    """This build's latency on the shapes the reference publishes H100 numbers for.

    Full-capacity caches (the reference's benchmark uses lengths = N), bf16,
    N(0, 1) inputs; graph-replayed medians as the reference times them
    (benchmark.py:42-84). Informational: the headline metric is decode tok/s.
    """
    import torch

    from systems_for_llms_amd.attention import attention
    from systems_for_llms_amd.decode import prepare
    from systems_for_llms_amd.masks import MaskSpec, compile_mask

    g = torch.Generator(device="cuda").manual_seed(11)
    decode_rows = []
    for b, hq, hkv, n, d, custom, flash in H100_DECODE:
        q = torch.randn((b, hq, d), device="cuda", generator=g, dtype=torch.bfloat16)
        k = torch.randn((b, hkv, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
        v = torch.randn_like(k)
        op = prepare(q, k, v, splits=None)  # the split count chosen from the shape
        us = time_graph(op) * 1000
        kv_bytes = 2 * b * hkv * n * d * 2
        decode_rows.append({"shape": f"B={b} Hq={hq} Hkv={hkv} N={n} D={d}", "us": round(us, 1),
                            "kv_gbs": round(kv_bytes / us / 1e3, 1), "splits": op.splits,
                            "h100_custom_us": custom, "h100_flash_us": flash})
        del q, k, v, op
    masked_rows = []
    for d, mask, ref_us in H100_MASKED:
        spec = MaskSpec(causal=True, window_left=127 if "window" in mask else None)
        q, k, v = (torch.randn((1, 8, 4096, d), device="cuda", generator=g, dtype=torch.bfloat16)
                   for _ in range(3))
        sched = compile_mask(4096, spec, 64, 64)
        out = torch.empty_like(q)
        us = time_graph(lambda: attention(q, k, v, sched, spec, implementation="interval", out=out)) * 1000
        masked_rows.append({"shape": f"B=1 H=8 N=4096 D={d} {mask}, interval schedule", "us": round(us, 1),
                            "h100_interval_us": ref_us})
        del q, k, v, out
    log("published shapes: " + "; ".join(f"{r['shape']}: {r['us']} us" for r in decode_rows + masked_rows))
    return {"note": "this build on MI355X vs the reference's published H100 numbers (same shapes, bf16); "
                    "informational, not the metric",
            "decode_attention": decode_rows, "masked_attention": masked_rows}


def cpu_baseline(cfg, seconds=12.0, max_steps=32):
    """KV-cached fp32 decode step of the CPU oracle at this workload's shape and context."""
    import torch

    from oracle.model import KVCacheOracle
    from systems_for_llms_amd.weights import seeded_state_dict

    threads = os.cpu_count() or 1
    torch.set_num_threads(threads)
    sd = seeded_state_dict(cfg, WEIGHT_SEED)
    cache = KVCacheOracle(sd, cfg, BATCH, MEAN_LEN + max_steps + 1)
    cache.k.fill_(0.01)  # touch every page: the step streams the whole cache
    cache.v.fill_(0.01)
    cache.length = MEAN_LEN - 1  # the decode's mean attention length, as the GPU figures
    tokens = torch.randint(0, cfg.vocab_size, (BATCH, 1), generator=torch.Generator().manual_seed(5))
    cache.step(tokens)  # first call pays one-time allocations
    started = time.perf_counter()
    steps = 0
    while steps < max_steps and time.perf_counter() - started < seconds:
        cache.step(tokens)
        steps += 1
    elapsed = time.perf_counter() - started
    return {"value": round(BATCH * steps / elapsed, 2), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"{steps} KV-cached fp32 decode steps of the CPU oracle (oracle/model.py KVCacheOracle), "
                      f"324M, batch {BATCH}, attention length {MEAN_LEN}..{MEAN_LEN + steps}; os.cpu_count()={threads}"}


def cpu_reference_semantics(cfg, length=PROMPT):
    """One step as the reference must run it: a full forward over the whole prefix (no KV cache),
    fp32 on the host cores, for one sequence of ``length`` tokens; its cost per generated token."""
    import torch

    from oracle.model import forward
    from systems_for_llms_amd.weights import seeded_prompt, seeded_state_dict

    torch.set_num_threads(os.cpu_count() or 1)
    sd = seeded_state_dict(cfg, WEIGHT_SEED)
    ids = seeded_prompt(cfg.vocab_size, 1, length, PROMPT_SEED)
    started = time.perf_counter()
    with torch.no_grad():
        forward(sd, cfg, ids, torch.float32)
    elapsed = time.perf_counter() - started
    return {"value": round(1.0 / elapsed, 4), "unit": "tok/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"one full-recompute fp32 forward of the CPU oracle (oracle/model.py forward) over a "
                      f"{length}-token prefix, batch 1 = one generated token: {elapsed:.2f} s"}


def profile_target_attention(reps: int = 24) -> int:
    """Counter-collection target: the roofline's fused attention launches plus a calibration copy.

    Same shapes as the ``roofline`` measurement (324M cache layout, B=16, H=16,
    D=64, d_model 1024, length 3584, one call per layer cache so nothing is
    re-read from the last-level cache), with random cache contents and weights,
    followed by one device copy of 256 MiB whose HBM traffic is known (256 MiB
    read + 256 MiB written). Run it under ``rocprofv3 --pmc FETCH_SIZE`` and
    ``--pmc WRITE_SIZE``.
    """
    import torch

    from systems_for_llms_amd import _lib

    layers, heads, dim, length = 24, 16, 64, PROMPT + 512  # the timed region's mean length, 3584
    d_model = heads * dim
    k = torch.randn((layers, BATCH, heads, CONTEXT, dim), device="cuda", dtype=torch.bfloat16)
    v = torch.randn_like(k)
    w_out = [_lib.pack_gemv(torch.randn((d_model, d_model), device="cuda", dtype=torch.bfloat16) * 0.02)
             for _ in range(layers)]
    q = torch.randn((BATCH, heads, dim), device="cuda", dtype=torch.float32)
    x = torch.zeros((BATCH, d_model), device="cuda", dtype=torch.float32)
    lengths = torch.full((BATCH,), length, device="cuda", dtype=torch.int32)
    for i in range(reps):
        _lib.call("sfl_decode_attention_out_proj", q.data_ptr(), k[i % layers].data_ptr(), v[i % layers].data_ptr(),
                  lengths.data_ptr(), w_out[i % layers].data_ptr(), x.data_ptr(), BATCH, heads, CONTEXT, dim,
                  dim ** -0.5, 1, _lib.stream_handle())
    src = torch.ones(256 << 20, device="cuda", dtype=torch.uint8)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile target: {reps} fused attention + output_proj launches (length {length}, "
        f"{fused_attention_bytes([length] * BATCH, heads, dim, d_model)} algorithmic bytes each) "
        f"+ one 256 MiB copy")
    return 0



def profile_target_decode(steps: int = 4) -> int:
    """Counter-collection target: ``steps`` eager decode steps of the 324M model at B=16
    and attention length 3584 (every launch of the step: the q/k/v, SwiGLU, w2 and
    lm_head GEMVs, the fused attention, the token step), then one device copy of
    256 MiB whose HBM traffic is known (256 MiB read + 256 MiB written). The cache
    holds zeros (traffic and time do not depend on its values); every GEMV streams
    its weights from HBM as in the decode loop, since a step reads more than the
    256 MB last-level cache holds. Run it under ``rocprofv3 --pmc FETCH_SIZE`` and
    ``--pmc WRITE_SIZE``, or ``--kernel-trace --stats``."""
    import torch

    from systems_for_llms_amd.config import load_model_config
    from systems_for_llms_amd.engine import DecodeSession
    from systems_for_llms_amd.model import TransformerLM
    from systems_for_llms_amd.weights import seeded_state_dict

    cfg = load_model_config("scale-324m-s4096")
    model = TransformerLM.from_config(cfg, device="cuda", dtype=torch.bfloat16)
    model.load_state_dict(seeded_state_dict(cfg, WEIGHT_SEED))
    session = DecodeSession(model.eval(), BATCH, CONTEXT)
    session.set_position(MEAN_LEN - 1)  # attention length MEAN_LEN at the first step
    for _ in range(steps):
        session.step()
    src = torch.ones(256 << 20, device="cuda", dtype=torch.uint8)
    dst = torch.empty_like(src)
    dst.copy_(src)
    torch.cuda.synchronize()
    log(f"profile target: {steps} eager decode steps (324M, B={BATCH}, attention lengths {MEAN_LEN}.."
        f"{MEAN_LEN + steps - 1}) + one 256 MiB copy")
    return 0


def profile_target_gqa(reps: int = 40) -> int:
    """Kernel-trace target for grouped-query decode attention on the matrix cores.

    The reference's published shape B=8, Hq=32, Hkv=4, N=16384, D=128 (bf16,
    full-capacity caches, the automatic split count): ``reps`` operator calls
    (attention kernel + merge), event-timed as one region, so the rocprof
    per-kernel averages can be checked against the per-call time printed here.
    """
    import torch

    from systems_for_llms_amd.decode import prepare

    b, hq, hkv, n, d = 8, 32, 4, 16384, 128
    g = torch.Generator(device="cuda").manual_seed(11)
    q = torch.randn((b, hq, d), device="cuda", generator=g, dtype=torch.bfloat16)
    k = torch.randn((b, hkv, n, d), device="cuda", generator=g, dtype=torch.bfloat16)
    v = torch.randn_like(k)
    op = prepare(q, k, v, splits=None)
    op()
    torch.cuda.synchronize()
    us = time_events(op, reps) * 1000
    kv = 2 * b * hkv * n * d * 2
    log(f"profile target: {reps} decode_attention calls B={b} Hq={hq} Hkv={hkv} N={n} D={d} splits={op.splits}: "
        f"{us:.1f} us per call (events, eager), K+V {kv} bytes = {kv / us / 1e3:.0f} GB/s")
    return 0

def profile_target_masked(reps: int = 20) -> int:
    """Counter-collection target: the masked prefill attention at BASELINE config 5 and at the
    prefill's causal 16 x 16 x 3072 shape, ``reps`` eager calls each (event-timed per shape)."""
    import torch

    from systems_for_llms_amd.attention import attention
    from systems_for_llms_amd.masks import MaskSpec, compile_mask

    g = torch.Generator(device="cuda").manual_seed(5)
    for name, (b, h, n), spec, impl in (
            ("config 5", (4, 16, 4096), MaskSpec(causal=True, window_left=1023, global_prefix=256), "csr"),
            ("causal 16x16x3072", (16, 16, 3072), MaskSpec(causal=True), "interval")):
        q, k, v = (torch.randn((b, h, n, 64), device="cuda", generator=g, dtype=torch.bfloat16) for _ in range(3))
        sched = compile_mask(n, spec, 64, 64)
        out = torch.empty_like(q)
        call = lambda: attention(q, k, v, sched, spec, implementation=impl, out=out)  # noqa: E731
        call()
        torch.cuda.synchronize()
        log(f"profile target: {reps} masked attention calls, {name}: {time_events(call, reps) * 1000:.1f} us each")
        del q, k, v, out
    return 0


def profile_target_gemm(reps: int = 10) -> int:
    """Counter-collection target: the prefill GEMMs of the 324M model at M = 16 x 3072 tokens
    through the entry points the prefill calls (q/k/v scaled by 1/rms + RoPE + cache write,
    output_proj and w2 adding into x and writing the next norm's input and sums of squares,
    w1/w3 scaled + SwiGLU; then the all-positions lm_head), ``reps`` calls each."""
    import torch

    from systems_for_llms_amd import _lib

    m, d, f, v, h, t = BATCH * PROMPT, 1024, 2752, 10000, 16, PROMPT
    g = torch.Generator(device="cuda").manual_seed(3)
    act = torch.randn((m, d), device="cuda", generator=g, dtype=torch.bfloat16)
    hid = torch.randn((m, f), device="cuda", generator=g, dtype=torch.bfloat16)
    w = {name: torch.randn(shape, device="cuda", generator=g, dtype=torch.bfloat16) * 0.02
         for name, shape in (("qkv", (3 * d, d)), ("o", (d, d)), ("w13", (2 * f, d)), ("w2", (d, f)),
                             ("head", (v, d)))}
    x = torch.zeros((m, d), device="cuda")
    gain = torch.ones((d,), device="cuda", dtype=torch.bfloat16)
    xg = torch.empty((m, d), device="cuda", dtype=torch.bfloat16)  # the next norm's input
    ss = torch.empty((-(-d // 128), m), device="cuda")
    rsc = torch.ones((m,), device="cuda")
    logits = torch.empty((m, v), device="cuda")
    q = torch.empty((BATCH, h, t, d // h), device="cuda", dtype=torch.bfloat16)
    kc = torch.empty((BATCH, h, CONTEXT, d // h), device="cuda", dtype=torch.bfloat16)
    vc = torch.empty_like(kc)
    from systems_for_llms_amd.model import rope_tables
    cos, sin = (c.t().contiguous().cuda() for c in rope_tables(10000.0, d // h, CONTEXT))  # feature-major
    st = _lib.stream_handle()
    calls = {
        "q/k/v": lambda: _lib.call("sfl_gemm_qkv_rope_scaled", act.data_ptr(), w["qkv"].data_ptr(), rsc.data_ptr(),
                                   m, t, d, h, cos.data_ptr(), sin.data_ptr(), q.data_ptr(), kc.data_ptr(),
                                   vc.data_ptr(), CONTEXT, 1, st),
        "output_proj": lambda: _lib.call("sfl_gemm_residual_norm", act.data_ptr(), w["o"].data_ptr(), x.data_ptr(),
                                         m, d, d, gain.data_ptr(), xg.data_ptr(), ss.data_ptr(), 1, st),
        "w1/w3": lambda: _lib.call("sfl_gemm_swiglu_scaled", act.data_ptr(), w["w13"].data_ptr(), rsc.data_ptr(),
                                   hid.data_ptr(), m, f, d, 1, st),
        "w2": lambda: _lib.call("sfl_gemm_residual_norm", hid.data_ptr(), w["w2"].data_ptr(), x.data_ptr(), m, d, f,
                                gain.data_ptr(), xg.data_ptr(), ss.data_ptr(), 1, st),
        "lm_head": lambda: _lib.call("sfl_gemm", act.data_ptr(), w["head"].data_ptr(), logits.data_ptr(), m, v, d, 1, 0, 0, st),
    }
    flops = {"q/k/v": 2 * m * 3 * d * d, "output_proj": 2 * m * d * d, "w1/w3": 2 * m * 2 * f * d,
             "w2": 2 * m * d * f, "lm_head": 2 * m * v * d}
    for name, call in calls.items():
        call()
        torch.cuda.synchronize()
        us = time_events(call, reps) * 1000
        log(f"profile target: {reps} GEMM calls, {name}: {us:.1f} us each, "
            f"{flops[name] / us / 1e6:.0f} TFLOP/s")
    return 0


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=CONTEXT - PROMPT - 1)
    parser.add_argument("--warmup", type=int, default=8)
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-reference-shapes", action="store_true",
                        help="skip timing the reference's published attention shapes")
    parser.add_argument("--attention-reps", type=int, default=50)
    parser.add_argument("--profile-target", choices=["attention", "decode", "gqa", "masked", "gemm"], default=None,
                        help="run only a profiling target (profile_target_attention, _decode, _gqa, _masked, _gemm)")
    args = parser.parse_args()
    if args.profile_target == "attention":
        return profile_target_attention()
    if args.profile_target == "decode":
        return profile_target_decode()
    if args.profile_target == "gqa":
        return profile_target_gqa()
    if args.profile_target == "masked":
        return profile_target_masked()
    if args.profile_target == "gemm":
        return profile_target_gemm()
    if args.gpus != 1:
        print("bench.py measures one GPU: every box in this build has a single MI355X and the decode "
              "path is not sharded across GPUs (data parallel over the batch would need no exchange)",
              file=sys.stderr)
        return 2
    if not 1 <= args.steps <= CONTEXT - PROMPT - 1 or not 0 <= args.warmup <= CONTEXT - PROMPT - 1:
        print(f"--steps and --warmup must be in [1, {CONTEXT - PROMPT - 1}]", file=sys.stderr)
        return 2

    import torch

    from systems_for_llms_amd.config import load_model_config
    from systems_for_llms_amd.decode import prepare
    from systems_for_llms_amd.engine import DecodeSession
    from systems_for_llms_amd.model import TransformerLM
    from systems_for_llms_amd.weights import seeded_prompt, seeded_state_dict

    cfg = load_model_config("scale-324m-s4096")
    t0 = time.perf_counter()
    model = TransformerLM.from_config(cfg, device="cuda", dtype=torch.bfloat16)
    model.load_state_dict(seeded_state_dict(cfg, WEIGHT_SEED))
    model.eval()
    prompt = seeded_prompt(cfg.vocab_size, BATCH, PROMPT, PROMPT_SEED).cuda()
    log(f"model ready in {time.perf_counter() - t0:.1f}s")

    session = DecodeSession(model, BATCH, CONTEXT)
    session.prefill(prompt)  # warm-up: first-call kernel attributes and allocations
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    session.prefill(prompt)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    log(f"prefill of {BATCH}x{PROMPT} tokens in {prefill_s * 1000:.1f} ms "
        f"({BATCH * PROMPT / prefill_s:.0f} tok/s, MFMA GEMMs + masked attention)")
    first = PROMPT  # prefill chose token PROMPT; decode steps run at positions PROMPT ..
    assert int(session.pos[0]) == first and session.position == first
    session.step()  # eager warm-up of every decode kernel before capture
    session.capture(1)
    # Timed steps centred on the mean attention length; untimed real decode
    # steps fill the cache and tokens up to the first timed position.
    start = max(first, min(CONTEXT - 1 - args.steps, MEAN_LEN - (args.steps + 1) // 2))
    warm = min(max(args.warmup, start - session.position), CONTEXT - 1 - session.position)
    for _ in range(warm):
        session.replay()
    torch.cuda.synchronize()
    session.set_position(start)
    torch.cuda.synchronize()
    ms = time_events(session.replay, args.steps)
    ms_per_step = ms
    tokens_per_s = BATCH * 1000.0 / ms_per_step
    mean_len = start + (args.steps + 1) / 2  # attention lengths start+1 .. start+K
    generated = session.tokens[:, PROMPT:start + args.steps + 1]
    assert int(session.pos[0]) == start + args.steps
    assert bool((generated >= 0).all()) and bool((generated < cfg.vocab_size).all())
    log(f"decode {args.steps} steps at positions {start}..{start + args.steps - 1} (mean attention length "
        f"{mean_len}): {ms_per_step:.3f} ms/step, {tokens_per_s:.0f} tok/s")

    # Dominant kernel: decode attention fused with output_proj, at the decode's
    # mean attention length.
    length = MEAN_LEN
    lengths = torch.full((BATCH,), length, device="cuda", dtype=torch.int32)
    q = torch.randn((BATCH, cfg.num_heads, cfg.head_dim), device="cuda", dtype=torch.float32)
    x_scratch = torch.zeros((BATCH, cfg.d_model), device="cuda", dtype=torch.float32)
    from systems_for_llms_amd import _lib

    # Rotate over the 24 layers' caches (5.6 GB in all) so no call re-reads
    # data another left in the 256 MB last-level cache: this is HBM streaming,
    # as in the decode loop.
    layer = [0]
    stream = _lib.stream_handle()

    def fused_call():
        layer[0] = (layer[0] + 1) % cfg.num_layers
        k_l, v_l = session.k_cache[layer[0]], session.v_cache[layer[0]]
        _lib.call("sfl_decode_attention_out_proj", q.data_ptr(), k_l.data_ptr(), v_l.data_ptr(), lengths.data_ptr(),
                  session.p_out[layer[0]].data_ptr(), x_scratch.data_ptr(), BATCH, cfg.num_heads, CONTEXT,
                  cfg.head_dim, cfg.head_dim ** -0.5, 1, stream)

    def attention_call():
        layer[0] = (layer[0] + 1) % cfg.num_layers
        k_l, v_l = session.k_cache[layer[0]], session.v_cache[layer[0]]
        _lib.call("sfl_decode_attention", q.data_ptr(), k_l.data_ptr(), v_l.data_ptr(), lengths.data_ptr(),
                  session.pmax.data_ptr(), session.psum.data_ptr(), session.pout.data_ptr(),
                  session.attn.data_ptr(), BATCH, cfg.num_heads, cfg.num_heads, CONTEXT, cfg.head_dim,
                  session.splits, cfg.head_dim ** -0.5, 1, 0, session.act_code, stream)

    assert session.fused_out_proj, "the 324M decode step runs the fused attention + output_proj kernel"
    for _ in range(3):
        fused_call()
    attn_ms = time_events(fused_call, args.attention_reps)
    attn_bytes = fused_attention_bytes([length] * BATCH, cfg.num_heads, cfg.head_dim, cfg.d_model)
    achieved = attn_bytes / (attn_ms * 1e-3) / 1e9
    log(f"decode attention + output_proj at length {length}: {attn_ms * 1000:.1f} us, {achieved:.0f} GB/s")
    for _ in range(3):
        attention_call()
    op_ms = time_events(attention_call, args.attention_reps)
    op_bytes = attention_bytes([length] * BATCH, cfg.num_heads, cfg.head_dim)
    op_gbs = op_bytes / (op_ms * 1e-3) / 1e9
    log(f"decode attention operator at length {length}: {op_ms * 1000:.1f} us, {op_gbs:.0f} GB/s")

    # BASELINE config 4 decode-attention microbench (ragged 1K..16K, B=64, H=16, D=64).
    g = torch.Generator(device="cuda").manual_seed(4)
    qc = torch.randn((64, 16, 64), device="cuda", generator=g, dtype=torch.bfloat16)
    kc = torch.randn((64, 16, 16384, 64), device="cuda", generator=g, dtype=torch.bfloat16)
    vc = torch.randn((64, 16, 16384, 64), device="cuda", generator=g, dtype=torch.bfloat16)
    lc = torch.randint(1024, 16385, (64,), generator=torch.Generator().manual_seed(4), dtype=torch.int32)
    op = prepare(qc, kc, vc, lc.cuda(), splits=None)
    for _ in range(3):
        op()
    c4_ms = time_events(op, 20)
    c4_bytes = attention_bytes(lc.tolist(), 16, 64, q_elem=2)
    c4_gbs = c4_bytes / (c4_ms * 1e-3) / 1e9
    del qc, kc, vc
    log(f"config-4 decode attention: {c4_ms * 1000:.1f} us, {c4_gbs:.0f} GB/s")

    # BASELINE config 5 masked prefill attention: [4,16,4096,64] bf16, causal,
    # window_left 1023, 4 global prefix blocks of 64 (CSR schedule).
    from systems_for_llms_amd.attention import attention
    from systems_for_llms_amd.masks import MaskSpec, compile_mask

    spec5 = MaskSpec(causal=True, window_left=1023, global_prefix=256)
    g5 = torch.Generator(device="cuda").manual_seed(5)
    q5, k5, v5 = (torch.randn((4, 16, 4096, 64), device="cuda", generator=g5, dtype=torch.bfloat16)
                  for _ in range(3))
    sched5 = compile_mask(4096, spec5, 64, 64)
    pairs5 = sum(min(i, 1023) + 1 + max(0, min(256, i - 1023)) for i in range(4096))
    o5 = torch.empty_like(q5)
    for _ in range(3):
        attention(q5, k5, v5, sched5, spec5, out=o5)
    c5_ms = time_graph(lambda: attention(q5, k5, v5, sched5, spec5, out=o5))
    c5_tflops = 4 * 64 * pairs5 * 4 * 16 / (c5_ms * 1e-3) / 1e12
    del q5, k5, v5, o5
    log(f"config-5 masked attention: {c5_ms * 1000:.1f} us, {c5_tflops:.0f} TFLOP/s (mask-exact)")
    reference_shapes = published_shapes() if not args.no_reference_shapes else None
    gemm_flops, attn_flops = prefill_flops(cfg, BATCH, PROMPT)
    prefill_tflops = (gemm_flops + attn_flops) / prefill_s / 1e12

    # HBM traffic per launch from the committed PMC record of the same launch
    # shape (FETCH_SIZE + WRITE_SIZE, calibrated on a copy of known size).
    traffic = None
    pmc = ROOT / "profiles" / "decode_attention_out_proj_324m_b16_len3584_pmc.json"
    if pmc.exists():
        record = json.loads(pmc.read_text())
        assert record["length"] == length, "the PMC record is for another attention length"
        traffic = record["traffic_bytes"]

    e2e_bytes = step_bytes(cfg, BATCH, mean_len)
    e2e_gbs = e2e_bytes / (ms_per_step * 1e-3) / 1e9
    baseline = reference_semantics = None
    if not args.no_cpu_baseline:
        log("timing the CPU oracle baseline ...")
        baseline = cpu_baseline(cfg)
        log(f"cpu baseline {baseline['value']} tok/s on {baseline['cores']} threads")
        reference_semantics = cpu_reference_semantics(cfg)
        log(f"cpu full-recompute step: {reference_semantics['value']} tok/s")

    record = {
        "metric": "decode tok/s, 324M bf16 ctx4K B=16; decode-attn HBM GB/s as % of peak",
        "value": round(tokens_per_s, 1),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: seeded N(0,0.02) weights, uniform random prompt ids",
        "config": {"workload": "BASELINE config 3: 324.1M llmlab decoder, batch 16, prefill 3072, "
                               "greedy decode to ctx 4096",
                   "d_model": cfg.d_model, "num_layers": cfg.num_layers, "num_heads": cfg.num_heads,
                   "d_ff": cfg.d_ff, "vocab_size": cfg.vocab_size, "global_batch": BATCH,
                   "prompt": PROMPT, "context": CONTEXT, "parallelism": "single GPU",
                   "timed_positions": [start, start + args.steps - 1],
                   "mean_attention_length": mean_len},
        "roofline": {"bound": "hbm",
                     "kernel": "decode_attn_kernel<resid_t> (decode attention + output_proj + residual, one launch)",
                     "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "traffic_source": f"profiles/{pmc.name}" if traffic else None,
                     "bytes_per_launch": attn_bytes, "us_per_launch": round(attn_ms * 1000, 2),
                     "shape": f"B={BATCH} H={cfg.num_heads} D={cfg.head_dim} d_model={cfg.d_model} "
                              f"length={length} (mean attention length of the decode to 4096)"},
        "decode_attention_operator": {"us": round(op_ms * 1000, 2), "achieved_gbs": round(op_gbs, 1),
                                      "frac": round(op_gbs / HBM_PEAK_GBS, 4), "bytes": op_bytes,
                                      "shape": f"sfl_decode_attention, same shape and caches, BF16X2 output"},
        "e2e": {"bytes_per_step": int(e2e_bytes), "achieved_gbs": round(e2e_gbs, 1),
                "frac_of_hbm_peak": round(e2e_gbs / HBM_PEAK_GBS, 4),
                "roofline_tok_s": round(BATCH / (e2e_bytes / (HBM_PEAK_GBS * 1e9)), 1),
                "prefill_s": round(prefill_s, 4), "prefill_tok_s": round(BATCH * PROMPT / prefill_s, 1),
                "prefill_path": "MFMA GEMMs (QKV+RoPE+append, O, SwiGLU, W2) + MFMA causal attention"},
        "prefill": {"ms": round(prefill_s * 1000, 2), "tok_s": round(BATCH * PROMPT / prefill_s, 1),
                    "gemm_tflop": round(gemm_flops / 1e12, 3), "attention_tflop": round(attn_flops / 1e12, 3),
                    "achieved_tflops": round(prefill_tflops, 1), "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                    "frac": round(prefill_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                    "note": "whole prefill (GEMMs, causal attention, norms, embedding) timed end to end"},
        "decode_attention_config4": {"us": round(c4_ms * 1000, 1), "achieved_gbs": round(c4_gbs, 1),
                                     "frac": round(c4_gbs / HBM_PEAK_GBS, 4), "bytes": c4_bytes,
                                     "shape": "B=64 H=16 D=64 bf16 ragged lengths U[1024,16384] seed 4"},
        "masked_attention_config5": {"us": round(c5_ms * 1000, 1), "tflops": round(c5_tflops, 1),
                                     "peak_tflops": MFMA_BF16_PEAK_TFLOPS,
                                     "frac": round(c5_tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                                     "flop": 4 * 64 * pairs5 * 4 * 16,
                                     "shape": "B=4 H=16 N=4096 D=64 bf16, causal, window_left 1023, "
                                              "4 global prefix blocks, CSR schedule; mask-exact flops",
                                     "timing": "median of graph replays of 10 calls (benchmark.py:42-84)"},
        "reference_published_shapes": reference_shapes,
        "cpu_baseline": baseline,
        "cpu_reference_semantics": reference_semantics,
    }
    print(json.dumps(record), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
