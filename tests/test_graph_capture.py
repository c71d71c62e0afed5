"""CPU checks of the graph capture, its legalizations and the oracle interpreter.

Every case of ``tests/graph_cases.py`` is captured on the CPU and interpreted
by the oracle (``oracle/graph.py``); the result must match torch's own CPU
execution of the same function (an independent implementation), which pins
the oracle the GPU lowering is later compared with. The legalizations are
checked structurally (the RMSNorm chains fold, SDPA stays whole).
"""

from __future__ import annotations

import collections

import numpy as np
import pytest
import torch

from oracle.graph import GraphOracle
from tests.graph_cases import CASES, config1_ids, module_case, tiny_llama, tiny_qwen2


def _flat(value):
    if isinstance(value, torch.Tensor):
        return [value]
    out = []
    for item in value:
        out.extend(_flat(item))
    return out


def _np(t):
    t = t.detach()
    return (t.float() if t.dtype == torch.bfloat16 else t).numpy()


def _compare(got, want, tol, name):
    assert len(got) == len(want), name
    for i, (g, w) in enumerate(zip(got, want)):
        w = _np(w)
        g = np.asarray(g)
        assert g.shape == w.shape, (name, i, g.shape, w.shape)
        if w.dtype == np.bool_ or np.issubdtype(w.dtype, np.integer) or tol == 0.0:
            np.testing.assert_array_equal(g.astype(w.dtype), w, err_msg=f"{name}[{i}]")
        else:
            scale = max(1.0, float(np.abs(w).max()))
            np.testing.assert_allclose(g, w, rtol=tol, atol=tol * scale, err_msg=f"{name}[{i}]")


@pytest.mark.parametrize("name,fn,make,tol", CASES, ids=[c[0] for c in CASES])
def test_oracle_interprets_the_captured_graph_like_torch(name, fn, make, tol):
    from aotolith_amd.graph import capture

    inputs = make()
    graph = capture(fn, inputs)
    got = GraphOracle(graph).run(dict(zip(graph.inputs, inputs)))
    _compare(got, _flat(fn(*inputs)), tol, name)


def test_rms_norm_chain_folds_and_sdpa_stays_whole():
    from aotolith_amd.graph import RMS_NORM, capture

    model = module_case(tiny_llama())
    graph = capture(model, (config1_ids(),))
    ops = collections.Counter(n.op for n in graph.nodes)
    # 2 layers x (input, post-attention) + the final norm
    assert ops[RMS_NORM] == 5
    assert ops["aten.scaled_dot_product_attention.default"] == 2
    assert "aten.rsqrt.default" not in ops and "aten._softmax.default" not in ops
    norms = [n for n in graph.nodes if n.op == RMS_NORM]
    assert all(n.args[1] is not None and n.args[2] == pytest.approx(1e-6) for n in norms)
    assert graph.inputs == ["input_ids"] or len(graph.inputs) == 1


@pytest.mark.parametrize("family", ["llama", "qwen2"])
def test_oracle_runs_the_tiny_hf_models_like_torch(family):
    model = module_case(tiny_llama(0) if family == "llama" else tiny_qwen2(1))
    from aotolith_amd.graph import capture

    ids = config1_ids(2) % (128 if family == "llama" else 96)
    graph = capture(model, (ids,))
    (logits,) = GraphOracle(graph).run(dict(zip(graph.inputs, [ids])))
    with torch.no_grad():
        want = model(ids)
    np.testing.assert_allclose(logits, want.numpy(), rtol=2e-5, atol=2e-5)


def test_capture_refuses_data_dependent_control_flow():
    from aotolith_amd.errors import CompilationError
    from aotolith_amd.graph import capture

    def branchy(x):
        if x.sum() > 0:
            return x * 2
        return x

    with pytest.raises(CompilationError):
        capture(branchy, (torch.ones(3),))


def test_graph_encoding_round_trips_through_json():
    """The artifact's graph record (aotolith_amd.artifact.encode_graph) decodes to the same graph."""

    import json

    from aotolith_amd.artifact import decode_graph, encode_graph
    from aotolith_amd.graph import capture

    model = module_case(tiny_llama(11))
    graph = capture(model, (config1_ids(12),))
    text = json.dumps(encode_graph(graph), sort_keys=True)
    again = decode_graph(json.loads(text), graph.state)
    assert again.inputs == graph.inputs and again.input_meta == graph.input_meta
    assert again.state_names == graph.state_names and again.outputs == graph.outputs
    assert [(n.name, n.op, n.args, n.kwargs, n.shape, n.dtype) for n in again.nodes] == \
        [(n.name, n.op, n.args, n.kwargs, n.shape, n.dtype) for n in graph.nodes]
    ids = config1_ids(13)
    np.testing.assert_array_equal(GraphOracle(again).run({graph.inputs[0]: ids})[0],
                                  GraphOracle(graph).run({graph.inputs[0]: ids})[0])
