"""Host-side contract of the decode operator (no GPU): validation before any launch."""

import pytest
import torch

from systems_for_llms_amd.decode import auto_splits, prepare


def test_cpu_input_rejected_before_launch():
    q = torch.zeros(1, 8, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 17, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="same CUDA"):
        prepare(q, k, k)


def test_invalid_split_count_rejected():
    q = torch.zeros(1, 8, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 17, 64, dtype=torch.float16)
    for splits in (0, 129, True, 2.5):
        with pytest.raises(ValueError, match="splits"):
            prepare(q, k, k, splits=splits)


def test_unknown_variant_and_bad_ratio_rejected():
    q = torch.zeros(1, 8, 64, dtype=torch.float16)
    k = torch.zeros(1, 2, 17, 64, dtype=torch.float16)
    with pytest.raises(ValueError, match="variant"):
        prepare(q, k, k, variant="approximate")
    with pytest.raises(ValueError, match="divisible"):
        prepare(torch.zeros(1, 7, 64, dtype=torch.float16), k, k)
    with pytest.raises(ValueError, match="head dimensions"):
        prepare(torch.zeros(1, 8, 48, dtype=torch.float16), torch.zeros(1, 2, 17, 48, dtype=torch.float16),
                torch.zeros(1, 2, 17, 48, dtype=torch.float16))


def test_split_count_defaults_to_one_as_in_the_reference():
    import inspect

    from systems_for_llms_amd.decode import decode

    for fn in (prepare, decode):  # kernel.py:85,116: splits=1
        assert inspect.signature(fn).parameters["splits"].default == 1


def test_auto_splits_bounds():
    assert auto_splits(64, 16, 16384) == 1   # config 4: 1024 workgroups already
    assert auto_splits(16, 16, 4096) == 1    # 324M decode: one workgroup per (batch, head)
    assert auto_splits(1, 16, 4096) == 4     # single sequence: split the context
    assert auto_splits(1, 4, 1024) == 1
    assert auto_splits(1, 1, 10) == 1
    # Grouped query heads on the VALU kernel: more, shorter splits (about 512 workgroups of >= 512 / G keys).
    assert auto_splits(1, 4, 1024, 8) == 16
    assert auto_splits(1, 4, 4096, 8) == 64
    assert auto_splits(8, 4, 16384, 8) == 16
    assert auto_splits(32, 4, 4096, 8) == 4
    assert auto_splits(1, 8, 4096, 4) == 32
    # On the MFMA kernel: about 256 workgroups of >= 128 keys.
    assert auto_splits(1, 4, 1024, 8, True) == 8
    assert auto_splits(1, 4, 4096, 8, True) == 32
    assert auto_splits(1, 4, 65536, 8, True) == 64
    assert auto_splits(8, 4, 16384, 8, True) == 8
    assert auto_splits(32, 4, 4096, 8, True) == 2
    assert auto_splits(8, 8, 4096, 4, True) == 4


def test_matrix_core_selection():
    from systems_for_llms_amd.decode import uses_matrix_cores

    q = torch.zeros(1, 32, 128, dtype=torch.bfloat16)
    k = torch.zeros(1, 4, 16, 128, dtype=torch.bfloat16)
    assert uses_matrix_cores(q, k)
    assert uses_matrix_cores(q[..., :64].half(), k[..., :64].half())
    assert not uses_matrix_cores(q.float(), k)           # fp32 queries: VALU kernel
    assert not uses_matrix_cores(q[:, :8], k)            # two heads per KV head
    assert not uses_matrix_cores(q[..., :32], k[..., :32])
    assert not uses_matrix_cores(q.float(), k.float())


def test_auto_splits_stay_in_range():
    for b, h, n in ((1, 1, 1), (3, 5, 999), (128, 32, 65536)):
        for g in (1, 2, 4, 8):
            for matrix_cores in (False, True):
                assert 1 <= auto_splits(b, h, n, g, matrix_cores) <= 128
