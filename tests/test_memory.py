"""Arena planner: the reference's known answer (tests/test_runtime.py:287-302)."""

from chroma_amd._src.memory import Allocation, plan_memory


def test_inclusive_lifetimes_alignment_and_coalescing():
    allocations = {
        "a": Allocation(64, 0, 1),
        "b": Allocation(128, 1, 2),
        "c": Allocation(64, 2, 3),
        "d": Allocation(192, 4, 5),
    }
    assert plan_memory(allocations) == 192
    assert allocations["a"].offset == allocations["c"].offset
    assert allocations["d"].offset == 0
    for left in allocations.values():
        for right in allocations.values():
            if left is right or left.end < right.start or right.end < left.start:
                continue
            assert left.offset + left.size <= right.offset or right.offset + right.size <= left.offset


def test_best_fit_prefers_the_smallest_hole():
    allocations = {
        "big": Allocation(256, 0, 0),
        "keep1": Allocation(64, 0, 9),
        "small": Allocation(64, 0, 0),
        "keep2": Allocation(64, 0, 9),
        "next": Allocation(64, 1, 1),
    }
    assert plan_memory(allocations) == 448
    # At kernel 1 "big" (256 B at 0) and "small" (64 B at 320) are free and not adjacent: best fit is "small".
    assert allocations["next"].offset == allocations["small"].offset == 320
