"""CPU check of plan_batches, the batching loop of runInferenceOnDevice
(internal/embeddings/embeddings.go:704-731), on hand-worked cases."""
import sys

fl = sys.modules["longbow_fletcher_amd"]


def test_token_budget():
    assert fl.plan_batches([5, 5, 5], 512, 10) == [(0, 2), (2, 1)]
    assert fl.plan_batches([5, 5, 5], 512, 15) == [(0, 3)]
    # a sequence longer than the budget runs alone
    assert fl.plan_batches([3, 20, 3, 3], 512, 10) == [(0, 1), (1, 1), (2, 2)]


def test_sequence_cap():
    assert fl.plan_batches([1] * 7, 3, 16384) == [(0, 3), (3, 3), (6, 1)]
    # maxBatchSize <= 0: the loop takes nothing and the reference forces one sequence
    assert fl.plan_batches([4, 4], 0, 100) == [(0, 1), (1, 1)]


def test_empty():
    assert fl.plan_batches([], 512, 16384) == []
