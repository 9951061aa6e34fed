"""The prismkv.core surface's argument checks and messages
(src/prismkv/core.py), which fire before anything reaches the device."""
import pytest
import torch

from prismkv_amd import core


def test_reference_errors():
    with pytest.raises(ValueError, match="expected a matrix"):
        core.positive_global_topk(torch.zeros(3), 1)
    with pytest.raises(ValueError, match="nonnegative"):
        core.positive_global_topk(torch.zeros(2, 3), -1)
    assert core.positive_global_topk(torch.zeros(2, 3), 0).numel() == 0
    s = core.SharedSAE()
    with pytest.raises(ValueError, match="positive scale"):
        core.build_index(torch.zeros(4, 128), s, 0.0)
    with pytest.raises(ValueError, match="nonempty"):
        core.build_index(torch.zeros(0, 128), s, 1.0)
    with pytest.raises(ValueError, match="head dimensions differ"):
        core.build_index(torch.zeros(4, 64), s, 1.0)
    with pytest.raises(ValueError, match="invalid sparsity"):
        core.SharedSAE(key_mean=0)
    idx = core.FeatureIndex(4, torch.zeros(128), torch.zeros(3000, dtype=torch.long), torch.zeros(3000, 128),
                            torch.zeros(3000, 128), [torch.zeros(0, dtype=torch.long)] * 3000)
    with pytest.raises(ValueError, match="unique_cap must be a fraction"):
        core.select_buckets(torch.zeros(4, 128), idx, unique_cap=2.0)
    with pytest.raises(ValueError, match="specify exact estimator"):
        core.bucket_scores(torch.zeros(4, 128), idx, terms=("count", "bogus"))
    with pytest.raises(ValueError, match="q_activation requires"):
        core.bucket_scores(torch.zeros(4, 128), idx, router="q_activation")
    k = torch.zeros(10, 128)
    with pytest.raises(ValueError, match="invalid KV/history"):
        core.attend(torch.zeros(4, 128), k, torch.zeros(9, 128), torch.zeros(0, dtype=torch.long), 5)
    with pytest.raises(ValueError, match="old history only"):
        core.attend(torch.zeros(4, 128), k, k, torch.tensor([7]), 5)
    with pytest.raises(ValueError, match="deduplicate"):
        core.attend(torch.zeros(4, 128), k, k, torch.tensor([1, 1]), 5)


def test_other_geometries_are_rejected():
    with pytest.raises(NotImplementedError, match="specialised"):
        core.positive_global_topk(torch.zeros(2, 3), 1)  # host tensor, 3 buckets
    with pytest.raises(NotImplementedError, match="specialised"):
        core.build_index(torch.zeros(4, 128), core.SharedSAE(), 1.0)  # host keys
