"""The derived-operand cache of boundflow_amd.crown (layer-weight transposes, bias
maps and gradient seeds kept across queries): a hit needs the same source tensor
objects at the same versions; an in-place change or a new tensor recomputes."""

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
