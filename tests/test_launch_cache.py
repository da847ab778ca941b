"""The prepared-launch cache of kernels.swin_block / kernels.swin_mlp
(host logic, no GPU): an entry serves a call only for the very tensors it was
built from, with unchanged data pointers and sizes, and keeps none of them
alive."""
import gc

import torch

from terra_amd import kernels


def _entry(*given):
    e = kernels._Launch()
    e.watch(given)
    return e


def test_same_tensors_are_served():
    a, b = torch.zeros(4), torch.ones(3)
    e = _entry(a, None, b)
    assert e.serves((a, None, b))
    a.add_(1.0)  # in place: same memory, the kernel reads the new values
    assert e.serves((a, None, b))


def test_other_tensors_or_none_pattern_are_not_served():
    a, b = torch.zeros(4), torch.ones(3)
    e = _entry(a, None, b)
    assert not e.serves((a.clone(), None, b))
    assert not e.serves((a, b, b))
    assert not e.serves((a, None, None))


def test_rebound_data_and_resize_are_not_served():
    a = torch.zeros(8)
    e = _entry(a)
    a.data = torch.zeros(8)  # same tensor object, new memory
    assert not e.serves((a,))
    b = torch.zeros(8)
    e = _entry(b)
    b.resize_(4)  # same memory, fewer elements
    assert not e.serves((b,))


def test_entry_keeps_nothing_alive():
    a = torch.zeros(16)
    ref_count = len(gc.get_referrers(a))
    e = _entry(a)
    assert len(gc.get_referrers(a)) == ref_count
    wr = e.refs[0][0]
    del a
    gc.collect()
    assert wr() is None
