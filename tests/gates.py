"""Shared accuracy gates of the bf16 GPU parity tests (imported by the test modules)."""

BF16_ATOL, BF16_AGREE = 2e-2, 0.99  # north-star bf16 gate against fp32
KERNEL_ATOL, KERNEL_AGREE = 2e-3, 0.99  # kernels against the bf16-storage floor
CAP_ATOL, CAP_AGREE = 3.5e-2, 0.95  # absolute cap against the fp32 reference on the seeded weights


def bf16_gate(name, got, ref, floor, targets=None, envelope=None, ref_bf16_weights=None, unfolded_floor=None,
              cap=(CAP_ATOL, CAP_AGREE)):
    """Judge bf16 logits against the fp32 reference and against the bf16-storage floor.

    ``floor`` is the CPU oracle run with the same storage formats as the kernels
    (weights and KV cache rounded to bf16, plus the GEMM inputs a batched
    prefill stores in bf16) and exact fp32 arithmetic otherwise. Two gates:

    * the kernels against the floor, tight (2e-3, 99% agreement): what the HIP
      arithmetic adds on top of the storage formats. Where bf16 activations
      are re-rounded at every stage (the GEMM prefill), two exact computations
      drift apart chaotically -- a 1-ulp flip from fp32 reassociation changes
      the next stage's rounding of its whole row -- so ``envelope``, a pair
      (floor rows, the same rows recomputed with float64 accumulation), sets
      the bound instead: twice that drift, and its agreement less 0.5%. A
      window of fewer than 100 positions cannot resolve 1%, so one pick that
      differs from the floor's is allowed there (its logits still within the
      max-abs bound, i.e. a near-tie; the floor's top-2 margin is printed);
    * the north-star gate against fp32 (max-abs 2e-2, >= 99% greedy agreement).
      It is printed for every config. Where it is missed, the test requires
      that the storage formats alone (the floor) miss it too -- on the flat
      N(0, 0.02) random weights a quarter of the steps have a top-2 gap below
      0.01 -- and that the kernels stay within the kernel-vs-floor bounds of
      the floor's own numbers.

    Two bounds hold with no dependence on the floor:

    * ``ref_bf16_weights``, the fp32 reference forward on the weights the bf16
      model holds (the seeded weights rounded to bf16, exact fp32 arithmetic
      otherwise): the kernels' logits are within max-abs 2e-2 of it, always;
    * against the fp32 reference on the unrounded seeds: max-abs <= 3.5e-2 and
      >= 95% greedy agreement, always (``cap``: a deeper model, whose bf16
      weight rounding alone moves the logits further, states its own).

    ``unfolded_floor`` (a prefill whose norms are folded into its GEMMs): the
    floor of the same prefill with separate norm passes, which stores the
    reference's rounding point bf16(RMSNorm(x) * g) instead of bf16(x * g). The
    folded floor must be no further from ``ref_bf16_weights`` than it (plus the
    kernel tolerance): the fold may move the rounding point, not lose accuracy.
    """
    kernel_atol, kernel_agree, drift_note = KERNEL_ATOL, KERNEL_AGREE, ""
    if envelope is not None:
        base, wide = envelope
        drift = (base - wide).abs().max().item()
        drift_agree = (base.argmax(-1) == wide.argmax(-1)).float().mean().item()
        kernel_atol = max(KERNEL_ATOL, 2.0 * drift)
        kernel_agree = min(KERNEL_AGREE, drift_agree - 0.005)
        drift_note = f" | floor vs float64-accumulated floor: max-abs {drift:.5f} agreement {drift_agree:.4f}"
    samples = got.shape[:-1].numel()
    if samples < 100:  # a window this short cannot resolve 1%: one flip is allowed
        kernel_agree = min(kernel_agree, 1.0 - 1.0 / samples)
    targets = ref.argmax(-1) if targets is None else targets
    err = (got - ref).abs().max().item()
    floor_err = (floor - ref).abs().max().item()
    agree = (got.argmax(-1) == targets).float().mean().item()
    floor_agree = (floor.argmax(-1) == targets).float().mean().item()
    kernel_err = (got - floor).abs().max().item()
    k_agree = (got.argmax(-1) == floor.argmax(-1)).float().mean().item()
    strict = err <= BF16_ATOL and agree >= BF16_AGREE
    floor_strict = floor_err <= BF16_ATOL and floor_agree >= BF16_AGREE
    print(f"{name}: north-star gate (max-abs <= {BF16_ATOL}, agreement >= {BF16_AGREE}) vs fp32: "
          f"max-abs {err:.4f} agreement {agree:.4f} -> {'met' if strict else 'MISSED'} | bf16-storage floor "
          f"vs fp32: max-abs {floor_err:.4f} agreement {floor_agree:.4f} -> "
          f"{'met' if floor_strict else 'MISSED'} | kernels vs floor: max-abs {kernel_err:.5f} "
          f"agreement {k_agree:.4f} (gate {kernel_atol:.5f}, {kernel_agree:.4f})" + drift_note)
    flips = got.argmax(-1) != floor.argmax(-1)
    if flips.any():  # the floor's top-2 gap where the kernels pick another token
        top2 = floor[flips].topk(2, dim=-1).values
        print(f"{name}: {int(flips.sum())} of {samples} picks differ from the floor's, its top-2 margins there: "
              + " ".join(f"{m:.5f}" for m in (top2[:, 0] - top2[:, 1]).tolist()))
    if ref_bf16_weights is not None:
        rw_err = (got - ref_bf16_weights).abs().max().item()
        rw_agree = (got.argmax(-1) == ref_bf16_weights.argmax(-1)).float().mean().item()
        floor_rw = (floor - ref_bf16_weights).abs().max().item()
        print(f"{name}: vs the fp32 reference on the bf16 weights: max-abs {rw_err:.4f} (bound {BF16_ATOL}) "
              f"agreement {rw_agree:.4f}; floor {floor_rw:.4f}")
        assert rw_err <= BF16_ATOL, f"{name}: logits {rw_err} from the fp32 reference on the same bf16 weights"
        if unfolded_floor is not None:
            alt_rw = (unfolded_floor - ref_bf16_weights).abs().max().item()
            alt_agree = (unfolded_floor.argmax(-1) == ref_bf16_weights.argmax(-1)).float().mean().item()
            print(f"{name}: norm fold: folded floor {floor_rw:.4f}, unfolded floor {alt_rw:.4f} (agreement "
                  f"{alt_agree:.4f}) from the fp32 reference on the bf16 weights; kernels vs unfolded floor "
                  f"max-abs {(got - unfolded_floor).abs().max().item():.4f}")
            assert floor_rw <= alt_rw + KERNEL_ATOL, f"{name}: folding the norms costs accuracy"
    cap_atol, cap_agree = cap
    print(f"{name}: absolute cap vs fp32 (max-abs <= {cap_atol}, agreement >= {cap_agree}): {err:.4f}, {agree:.4f}")
    assert err <= cap_atol and agree >= cap_agree, f"{name}: outside the absolute cap against fp32"
    assert kernel_err <= kernel_atol, f"{name}: kernels move the logits {kernel_err} from the storage floor"
    assert k_agree >= kernel_agree, f"{name}: kernels agree with the storage floor on only {k_agree}"
    if not strict:
        assert not floor_strict, f"{name}: bf16 storage alone meets the north-star gate but the kernels miss it"
        assert err <= floor_err + kernel_atol
        assert agree >= floor_agree - (1.0 - kernel_agree)
