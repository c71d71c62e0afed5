"""Artifacts on the GPU: save a compiled runtime, reload it (here and in a fresh
process, from the stored gfx950 code object) and get the same results.

The reference's fresh-process test (tests/test_artifact.py:100-131) loads an
artifact in a new interpreter and compares outputs; here the outputs are the
greedy tokens and prefill logits of a random-init decoder, which must be
identical (same state bits, same kernels).
"""

from __future__ import annotations

import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.decoder import DecoderShape
from tests.helpers import random_oracle_state, runtime_spec, state_to_device

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
TINY = DecoderShape(vocab=512, hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64,
                    eps=1e-6, theta=1e6)
PROMPT, NEW = 16, 8


def _runtime(seed=0):
    from aotolith_amd.decoder import compile_decoder_state

    state = state_to_device(random_oracle_state(TINY, seed), TINY.group_size)
    return compile_decoder_state(runtime_spec(TINY), state, prompt_length=PROMPT, max_new_tokens=NEW)


def _ids(seed, n=PROMPT):
    return np.random.default_rng(seed).integers(0, TINY.vocab, n)


def test_saved_runtime_reloads_with_identical_results(tmp_path):
    from aotolith_amd import load_runtime, read_artifact_manifest

    runtime = _runtime(1)
    ids = _ids(2)
    tokens = runtime.greedy_generate(ids).cpu()
    logits, cache = runtime.prefill_ids(ids[None])
    logits, cache = logits.clone(), cache.clone()
    prefill_path, decode_path = runtime.save(tmp_path / "tiny")
    assert prefill_path.name == "tiny.prefill.aoto" and decode_path.name == "tiny.decode.aoto"
    manifest = read_artifact_manifest(decode_path)
    assert manifest["entrypoint"]["kind"] == "decode"
    assert manifest["profile"]["architecture"] == "gfx950"

    loaded = load_runtime(tmp_path / "tiny")
    assert loaded.prefill.selections == runtime.prefill.selections
    assert loaded.decode.selections == runtime.decode.selections
    assert loaded.prompt_length == PROMPT and loaded.max_new_tokens == NEW
    # prefill and decode plans of one runtime share the reloaded state
    assert loaded.prefill.runtime is loaded.decode.runtime
    again_logits, again_cache = loaded.prefill_ids(ids[None])
    assert torch.equal(again_logits.view(torch.int16), logits.view(torch.int16))
    assert torch.equal(again_cache.view(torch.int16), cache.view(torch.int16))
    assert torch.equal(loaded.greedy_generate(ids).cpu(), tokens)


def test_decode_plan_loads_alone(tmp_path):
    from aotolith_amd import load_compiled_module

    runtime = _runtime(3)
    ids = _ids(4)
    logits, compact = runtime.prefill_ids(ids[None])
    cache = runtime.pad_cache(compact)
    token = torch.tensor([[int(torch.argmax(logits.float()))]], device="cuda")
    want_logits, want_cache = runtime.decode(token, cache, PROMPT + 1)
    want_logits, want_cache = want_logits.clone(), want_cache.clone()
    runtime.decode.save(tmp_path / "step.decode.aoto")
    plan = load_compiled_module(tmp_path / "step.decode.aoto")
    assert plan.name == "decode" and plan.selections == runtime.decode.selections
    got_logits, got_cache = plan(token, cache, PROMPT + 1)
    assert torch.equal(got_logits.view(torch.int16), want_logits.view(torch.int16))
    assert torch.equal(got_cache.view(torch.int16), want_cache.view(torch.int16))


def test_artifact_runs_in_a_fresh_process(tmp_path):
    from aotolith_amd.artifact import read_artifact

    runtime = _runtime(5)
    ids = _ids(6)
    tokens = runtime.greedy_generate(ids).cpu().numpy().reshape(-1).tolist()
    runtime.save(tmp_path / "fresh")
    script = (
        "import json, sys\n"
        "import numpy as np\n"
        "from aotolith_amd import load_runtime\n"
        "from aotolith_amd import _lib\n"
        "runtime = load_runtime(sys.argv[1])\n"
        "ids = np.array(json.loads(sys.argv[2]), dtype=np.int64)\n"
        "tokens = runtime.greedy_generate(ids).cpu().numpy().reshape(-1).tolist()\n"
        "print(json.dumps({'tokens': tokens, 'digest': _lib.installed_digest(0)}))\n"
    )
    env = dict(os.environ)
    env["PYTHONPATH"] = os.pathsep.join([str(ROOT), env.get("PYTHONPATH", "")])
    print(f"[fresh-process] loading {tmp_path / 'fresh'}", flush=True)
    done = subprocess.run([sys.executable, "-c", script, str(tmp_path / "fresh"), json.dumps(ids.tolist())],
                          capture_output=True, text=True, env=env, timeout=240)
    assert done.returncode == 0, done.stderr[-2000:]
    result = json.loads(done.stdout.strip().splitlines()[-1])
    assert result["tokens"] == tokens
    # the child ran the code object stored in the artifact
    stored = read_artifact(tmp_path / "fresh.decode.aoto").manifest["payload_digests"]["code_object"]
    assert result["digest"] == stored


def test_bucketed_artifacts_reload_sharing_one_state(tmp_path):
    from aotolith_amd import load_bucketed
    from aotolith_amd.decoder import compile_decoder_bucketed_state

    state = state_to_device(random_oracle_state(TINY, 7), TINY.group_size)
    runtime = compile_decoder_bucketed_state(runtime_spec(TINY), state, prompt_lengths=[8, 16], max_new_tokens=4)
    short, long = _ids(8, 6), _ids(9, 13)
    want = [runtime.greedy_generate(short).cpu(), runtime.greedy_generate(long).cpu()]
    paths = runtime.save(tmp_path / "b")
    assert sorted(p.name for p in paths) == sorted(
        ["b.8.prefill.aoto", "b.8.decode.aoto", "b.16.prefill.aoto", "b.16.decode.aoto"])
    loaded = load_bucketed(tmp_path / "b")
    assert loaded.prompt_lengths == (8, 16) and loaded.max_new_tokens == 4
    assert loaded.buckets[0].engine.state is loaded.buckets[1].engine.state
    assert torch.equal(loaded.greedy_generate(short).cpu(), want[0])
    assert torch.equal(loaded.greedy_generate(long).cpu(), want[1])


def test_strict_device_match_refuses_another_device(tmp_path):
    import zipfile

    from aotolith_amd.artifact import read_artifact
    from aotolith_amd.errors import ArtifactCompatibilityError

    runtime = _runtime(10)
    _, decode_path = runtime.save(tmp_path / "dev")
    read_artifact(decode_path, require_device_match=True)   # this device: accepted
    with zipfile.ZipFile(decode_path) as archive:
        entries = [(i, archive.read(i.filename)) for i in archive.infolist()]
    with zipfile.ZipFile(decode_path, "w") as archive:
        for info, payload in entries:
            if info.filename == "manifest.json":
                manifest = json.loads(payload)
                manifest["profile"]["device_name"] = "another GPU"
                payload = json.dumps(manifest).encode()
            archive.writestr(info, payload)
    read_artifact(decode_path)                                # portable load: accepted
    with pytest.raises(ArtifactCompatibilityError, match="device mismatch"):
        read_artifact(decode_path, require_device_match=True)
