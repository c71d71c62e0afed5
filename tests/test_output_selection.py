"""Host logic of compile_module's output selection (reference compiler.py:843-889): which part
of a module's return value becomes the plan's output."""

from __future__ import annotations

from types import SimpleNamespace

import pytest
import torch

from aotolith_amd.compiler import _select_output


def test_plain_tensor_and_model_outputs():
    t = torch.zeros(2)
    assert _select_output(t, None) is t
    logits = torch.ones(3)
    assert _select_output(SimpleNamespace(logits=logits, past=None), None) is logits
    assert _select_output({"only": t}, None) is t


def test_sequences_flatten_to_tensor_leaves_in_order():
    a, b, c = torch.zeros(1), torch.ones(1), torch.full((1,), 2.0)
    got = _select_output((a, [b, None, (c,)]), None)
    assert isinstance(got, tuple) and len(got) == 3
    assert got[0] is a and got[1] is b and got[2] is c


def test_output_key_selects_from_a_mapping_or_an_attribute():
    a, b = torch.zeros(1), torch.ones(1)
    assert _select_output({"x": a, "y": b}, "y") is b
    assert _select_output(SimpleNamespace(hidden=a, logits=b), "hidden") is a
    with pytest.raises(KeyError):
        _select_output({"x": a}, "y")
    with pytest.raises(ValueError):
        _select_output(SimpleNamespace(x=a), "y")


@pytest.mark.parametrize("bad", [(), [None], (torch.zeros(1), 3), "text", {"a": 1, "b": 2}])
def test_outputs_without_tensors_are_refused(bad):
    with pytest.raises(ValueError):
        _select_output(bad, None)
