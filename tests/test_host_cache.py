"""The derived-operand cache of boundflow_amd.crown (layer-weight transposes, bias
maps and gradient seeds kept across queries): a hit needs the same source tensor
objects at the same versions; an in-place change or a new tensor recomputes."""

import pytest
import torch

from boundflow_amd import crown


def test_hit_requires_same_tensor_and_version():
    calls = []
    W = torch.arange(6.0).reshape(2, 3)

    def make():
        calls.append(1)
        return W.t().contiguous()

    a = crown.derived("t_test", (W,), make)
    b = crown.derived("t_test", (W,), make)
    assert a is b and len(calls) == 1
    W.mul_(2.0)                                   # in-place change bumps the version
    c = crown.derived("t_test", (W,), make)
    assert len(calls) == 2 and torch.equal(c, W.t())


def test_distinct_tensors_and_tags_do_not_collide():
    W1 = torch.ones(2, 2)
    W2 = torch.ones(2, 2) * 3.0
    t1 = crown.transposed(W1)
    t2 = crown.transposed(W2)
    assert torch.equal(t1, W1.t()) and torch.equal(t2, W2.t())
    x = crown.derived("other_tag", (W1,), lambda: W1 + 1.0)
    assert torch.equal(x, W1 + 1.0) and x is not t1


def test_cache_is_bounded():
    keep = [torch.full((1,), float(i)) for i in range(crown._DERIVED_MAX + 8)]
    for t in keep:
        crown.derived("bound_test", (t,), lambda t=t: t * 2.0)
    assert len(crown._DERIVED) <= crown._DERIVED_MAX
    # the newest entries are still there and correct
    last = keep[-1]
    assert torch.equal(crown.derived("bound_test", (last,), lambda: torch.zeros(1)), last * 2.0)


def test_scope_keeps_entries_out_of_the_global_cache():
    """Inside derived_scope (graph capture) entries go to the scope's dict: the
    process-wide cache is neither read nor filled, so the captured work makes
    its operands itself."""
    W = torch.arange(4.0).reshape(2, 2)
    outside = crown.transposed(W)
    n_before = len(crown._DERIVED)
    with crown.derived_scope() as memo:
        inside = crown.transposed(W)
        again = crown.transposed(W)
    assert inside is again and inside is not outside
    assert len(memo) == 1 and len(crown._DERIVED) == n_before
    assert torch.equal(inside, W.t())
    # after the scope the global entry is used again
    assert crown.transposed(W) is outside


def test_call_memo_is_per_call():
    calls = []
    save = {"memo": {}}
    a = crown.call_memo(save, "k", lambda: calls.append(1) or torch.ones(2))
    b = crown.call_memo(save, "k", lambda: calls.append(1) or torch.ones(2))
    assert a is b and len(calls) == 1
    # without a memo (one-off evaluation) the operand is made every time
    crown.call_memo(None, "k", lambda: calls.append(1) or torch.ones(2))
    crown.call_memo({}, "k", lambda: calls.append(1) or torch.ones(2))
    assert len(calls) == 3


@pytest.mark.gpu
def test_box_radius_is_not_cached():
    """The input box radius depends on the query: an in-place change of the box
    is seen by the next query (and by a graph replay, which recomputes it).  The
    radius is one library launch, so this runs on the HIP device."""
    from boundflow_amd.spec import BoxPerturbation
    from tests.gpu_util import device
    dev = device()
    lo = torch.zeros(2, 3, device=dev)
    hi = torch.ones(2, 3, device=dev)
    pert = BoxPerturbation(lower=lo, upper=hi)
    r1, e1 = crown._input_radius(pert, 2, 3)
    r1 = r1.clone()
    pert.upper.copy_(torch.full((2, 3), 3.0, device=dev))   # the perturbation holds its own copy of the box
    r2, _ = crown._input_radius(pert, 2, 3)
    assert e1 == 1.0
    assert torch.equal(r1.cpu(), torch.full((2, 3), 0.5)) and torch.equal(r2.cpu(), torch.full((2, 3), 1.5))
