"""compile_callable / compile_module on the GPU: every node a gfx950 kernel, results like torch.

Each case of ``tests/graph_cases.py`` is compiled for ``target="hip-gfx950"``
and run through the C ABI's generic kernels; outputs are compared with torch's
CPU execution of the same function and with the oracle interpreter of the same
captured graph. Config 1 (the reference's tiny Llama through compile_module,
logits compared elementwise) and a tiny Qwen2 run end to end.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.graph import GraphOracle
from tests.graph_cases import CASES, config1_ids, module_case, tiny_llama, tiny_qwen2
from tests.test_graph_capture import _compare, _flat

pytestmark = pytest.mark.gpu


def _host(values):
    out = []
    for v in values:
        t = v.detach().cpu()
        out.append((t.float() if t.dtype == torch.bfloat16 else t).numpy())
    return out


@pytest.mark.parametrize("name,fn,make,tol", CASES, ids=[c[0] for c in CASES])
def test_compile_callable_matches_torch_and_the_oracle(name, fn, make, tol):
    import aotolith_amd as aoto

    inputs = make()
    print(f"[graph] {name}", flush=True)
    result = aoto.compile_callable(fn, inputs, target="hip-gfx950")
    got = result.plan(*inputs)
    assert all(isinstance(t, torch.Tensor) and t.device.type == "cuda" for t in got)
    assert all(s.is_native and s.device_architecture == "gfx950" for s in result.plan.selections)
    want = _flat(fn(*inputs))
    _compare(_host(got), want, max(tol, 2e-5) if tol else 0.0, name)
    graph = result.lowered_graph
    oracle = GraphOracle(graph).run(dict(zip(graph.inputs, inputs)))
    _compare(_host(got), [torch.from_numpy(np.asarray(o)) for o in oracle], max(tol, 2e-5) if tol else 0.0, name)


def test_config1_tiny_llama_logits_match_hf_eager():
    """Config 1: compile_module(tiny Llama, (input_ids [1, 4],)) -> logits [1, 4, 128], elementwise."""

    import aotolith_amd as aoto

    model = module_case(tiny_llama(0))
    ids = config1_ids(0)
    plan = aoto.compile_module(model, (ids,), target="hip-gfx950")
    (logits,) = plan(ids)
    assert tuple(logits.shape) == (1, 4, 128)
    with torch.no_grad():
        want = model(ids)
    np.testing.assert_allclose(logits.cpu().numpy(), want.numpy(), rtol=1e-4, atol=1e-4)
    kinds = {s.kind for s in plan.selections}
    assert {"rms_norm", "attention", "matmul", "gather", "elementwise"} <= kinds
    assert any(name.endswith("embed_tokens.weight") for name in plan.state_names)
    # new ids, same plan
    ids2 = config1_ids(1)
    (again,) = plan(ids2)
    with torch.no_grad():
        np.testing.assert_allclose(again.cpu().numpy(), model(ids2).numpy(), rtol=1e-4, atol=1e-4)


def test_compile_module_on_the_hf_model_itself_selects_logits():
    import aotolith_amd as aoto

    model = tiny_llama(3)
    ids = config1_ids(4)
    plan = aoto.compile_module(model, (ids,), example_kwargs={"use_cache": False}, target="hip-gfx950")
    (logits,) = plan(ids)
    with torch.no_grad():
        want = model(input_ids=ids, use_cache=False).logits
    np.testing.assert_allclose(logits.cpu().numpy(), want.numpy(), rtol=1e-4, atol=1e-4)


def test_tiny_qwen2_with_qkv_bias():
    import aotolith_amd as aoto

    model = module_case(tiny_qwen2(5))
    ids = config1_ids(6) % 96
    plan = aoto.compile_module(model, (ids,), target="hip-gfx950")
    (logits,) = plan(ids)
    with torch.no_grad():
        want = model(ids)
    np.testing.assert_allclose(logits.cpu().numpy(), want.numpy(), rtol=1e-4, atol=1e-4)


def test_plan_inputs_are_checked_and_index_bounds_verified():
    import aotolith_amd as aoto
    from aotolith_amd.errors import PlanInputError

    model = module_case(tiny_llama(7))
    ids = config1_ids(8)
    plan = aoto.compile_module(model, (ids,), target="hip-gfx950")
    with pytest.raises(PlanInputError):
        plan()
    with pytest.raises(PlanInputError):
        plan(torch.zeros((1, 5), dtype=torch.int64))
    bad = ids.clone()
    bad[0, 2] = 500  # outside the 128-row embedding: the gather flags it, reads nothing
    with pytest.raises(PlanInputError):
        plan(bad)
    plan(bad, verify_index_bounds=False)  # flagged rows read as zeros; no error raised


def test_tensor_keywords_become_named_inputs():
    import aotolith_amd as aoto

    class Scaled(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.w = torch.nn.Parameter(torch.randn(8, 6, generator=torch.Generator().manual_seed(9)))

        def forward(self, x, *, scale, offset=0.0):
            return (x @ self.w.t()) * scale + offset

    module = Scaled().eval()
    x = torch.randn(3, 6)
    scale = torch.rand(8)
    plan = aoto.compile_module(module, (x,), example_kwargs={"scale": scale, "offset": 0.5})
    assert plan.tensor_kwarg_names == ("scale",)
    (y,) = plan(x, scale=scale)
    with torch.no_grad():
        np.testing.assert_allclose(y.cpu().numpy(), module(x, scale=scale, offset=0.5).numpy(), rtol=1e-5,
                                   atol=1e-5)
    from aotolith_amd.errors import PlanInputError

    with pytest.raises(PlanInputError):
        plan(x)


def test_unsupported_targets_and_training_mode_are_refused():
    import aotolith_amd as aoto
    from aotolith_amd.errors import CompilationError

    with pytest.raises(CompilationError):
        aoto.compile_callable(lambda x: x + 1, (torch.ones(2),), target="apple-metal")
    model = tiny_llama(10).train()
    with pytest.raises(CompilationError):
        aoto.compile_module(model, (config1_ids(),))


def test_module_plan_artifact_reloads_here_and_in_a_fresh_process(tmp_path):
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path

    import aotolith_amd as aoto
    from aotolith_amd import load_compiled_module, read_artifact_manifest

    model = module_case(tiny_llama(12))
    ids = config1_ids(13)
    plan = aoto.compile_module(model, (ids,), target="hip-gfx950")
    (logits,) = plan(ids)
    path = plan.save(tmp_path / "tiny.aoto")
    manifest = read_artifact_manifest(path)
    assert manifest["entrypoint"]["kind"] == "graph" and manifest["profile"]["architecture"] == "gfx950"
    loaded = load_compiled_module(path)
    assert loaded.selections == plan.selections and loaded.state_names == plan.state_names
    (again,) = loaded(ids)
    assert torch.equal(again.cpu(), logits.cpu())
    root = Path(__file__).resolve().parents[1]
    script = ("import json, sys, torch\n"
              "from aotolith_amd import load_compiled_module\n"
              "plan = load_compiled_module(sys.argv[1])\n"
              "ids = torch.tensor(json.loads(sys.argv[2]), dtype=torch.int64)\n"
              "(out,) = plan(ids)\n"
              "print(json.dumps(out.cpu().flatten().tolist()))\n")
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(root), env.get("PYTHONPATH", "")])
    print(f"[graph-artifact] fresh process loading {path}", flush=True)
    done = subprocess.run([sys.executable, "-c", script, str(path), json.dumps(ids.tolist())], capture_output=True,
                          text=True, env=env, timeout=240)
    assert done.returncode == 0, done.stderr[-2000:]
    fresh = torch.tensor(json.loads(done.stdout.strip().splitlines()[-1]))
    assert torch.equal(fresh, logits.cpu().flatten())


def test_callable_artifact_round_trip(tmp_path):
    import aotolith_amd as aoto
    from aotolith_amd import load_compiled_module
    from tests.graph_cases import indexing

    inputs = [c for c in CASES if c[0] == "indexing"][0][2]()
    result = aoto.compile_callable(indexing, inputs)
    want = result.plan(*inputs)
    loaded = load_compiled_module(result.save(tmp_path / "indexing.aoto"))
    got = loaded.plan(*inputs)
    assert all(torch.equal(a.cpu(), b.cpu()) for a, b in zip(got, want))
