"""Artifact archives on the host: layout, digests, validation (no GPU needed).

Mirrors the reference's artifact tests (tests/test_artifact.py): round trip of
the manifest and payloads, aliased state written once, and refusal of a
tampered kernel table or state payload, an incompatible ABI, an unsupported
target or format version. The GPU side (install the stored code object,
rebuild the plans, generate the same tokens in a fresh process) is in
test_gpu_artifact.py.
"""

from __future__ import annotations

import json
import zipfile
from pathlib import Path

import pytest
import torch

from aotolith_amd import artifact
from aotolith_amd.decoder import DecoderSpec, DecoderState, LayerState, PackedWeight
from aotolith_amd.errors import ArtifactCompatibilityError
from aotolith_amd.selection import KernelSelection

SPEC = DecoderSpec(family="qwen2", vocab=96, hidden=64, intermediate=128, layers=2, heads=4, kv_heads=2,
                   head_dim=16, eps=1e-6, theta=1e6, qkv_bias=True)
GROUP = 32
PROFILE = {"device_name": "AMD Instinct MI355X", "architecture": "gfx950", "arch_features": "gfx950:sramecc+:xnack-"}
CONFIG = {"prompt_length": 8, "max_new_tokens": 4, "cache_capacity": 12, "group_size": GROUP, "memory": "latency",
          "attention_splits": 0}

#: A decode plan's selections as an artifact stores them (the GPU tests record real ones).
SELECTIONS = (
    KernelSelection(0, "embedding", "hidden_0", "hip_kernel", "gather", "bf16 embedding row gather", "aoto_embedding",
                    device_name="AMD Instinct MI355X", device_architecture="gfx950"),
    KernelSelection(1, "addmm", "qkv_0", "hip_kernel", "w4_gemv", "packed W4 GEMV with RMSNorm prologue",
                    "aoto_w4_gemv_r32x1x2_n1_b1", device_name="AMD Instinct MI355X", device_architecture="gfx950"),
    KernelSelection(2, "attention", "attention_0", "hip_kernel", "decode_attention", "single-query GQA",
                    "aoto_decode_attention_d64_w4j2", device_name="AMD Instinct MI355X", device_architecture="gfx950"),
)


def _fake_state(seed: int = 0) -> DecoderState:
    gen = torch.Generator().manual_seed(seed)

    def packed(n, k):
        words = torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k // 8), generator=gen, dtype=torch.int32)
        return PackedWeight(words, torch.rand((n, k // GROUP), generator=gen).to(torch.bfloat16), GROUP)

    def vec(n):
        return torch.randn(n, generator=gen).to(torch.bfloat16)

    h, i, w = SPEC.hidden, SPEC.intermediate, SPEC.qkv_width
    layers = [LayerState(qkv=packed(w, h), o=packed(h, SPEC.attention_width), gate=packed(i, h), up=packed(i, h),
                         down=packed(h, i), input_norm=vec(h), post_norm=vec(h), qkv_bias=vec(w))
              for _ in range(SPEC.layers)]
    embed = torch.randn((SPEC.vocab, h), generator=gen).to(torch.bfloat16)
    return DecoderState(embed=embed, final_norm=vec(h), lm_head=packed(SPEC.vocab, h), layers=layers)


def _write(path: Path, state: DecoderState | None = None, **overrides) -> Path:
    state = _fake_state() if state is None else state
    kwargs = dict(kind="decode", spec=SPEC, config=CONFIG, state=artifact.state_items(state),
                  selections=SELECTIONS, code_object=b"\x7fELF-gfx950-code-object" * 8,
                  profile=PROFILE)
    kwargs.update(overrides)
    return artifact.write_artifact(path, **kwargs)


def _rewrite(path: Path, edit) -> None:
    """Apply ``edit(name, bytes) -> bytes`` to every entry of the archive."""

    with zipfile.ZipFile(path) as archive:
        entries = [(info, archive.read(info.filename)) for info in archive.infolist()]
    with zipfile.ZipFile(path, "w") as archive:
        for info, payload in entries:
            archive.writestr(info, edit(info.filename, payload))


def _edit_manifest(path: Path, change) -> None:
    def edit(name, payload):
        if name != "manifest.json":
            return payload
        manifest = json.loads(payload)
        change(manifest)
        return json.dumps(manifest).encode()

    _rewrite(path, edit)


def test_round_trip_and_manifest(tmp_path):
    state = _fake_state()
    path = _write(tmp_path / "plan.decode.aoto", state)
    manifest = artifact.read_artifact_manifest(path)
    assert manifest["format"] == "aotolith" and manifest["format_version"] == artifact.FORMAT_VERSION
    assert manifest["target"] == "hip-gfx950"
    assert manifest["profile"]["architecture"] == "gfx950"
    assert manifest["entrypoint"]["kind"] == "decode"
    assert manifest["entrypoint"]["config"] == CONFIG
    assert DecoderSpec(**manifest["entrypoint"]["spec"]) == SPEC
    assert manifest["payloads"]["code_object"] == "code/gfx950.hsaco"

    contents = artifact.read_artifact(path)
    assert contents.selections == SELECTIONS
    assert contents.code_object == b"\x7fELF-gfx950-code-object" * 8
    items = artifact.state_items(state)
    assert list(contents.state) == [name for name, _ in items]
    for name, tensor in items:
        raw, dtype, shape = contents.state[name]
        assert shape == tuple(tensor.shape)
        assert raw == tensor.contiguous().reshape(-1).view(torch.uint8).numpy().tobytes()

    # the rebuilt state has the same tensors under the same roles
    named = {}
    for name, (raw, dtype, shape) in contents.state.items():
        host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
        named[name] = host.view(torch.bfloat16 if dtype == "bfloat16" else torch.int32).reshape(shape)
    rebuilt = artifact.state_from_items(SPEC, named, GROUP)
    assert torch.equal(rebuilt.layers[1].down.packed, state.layers[1].down.packed)
    assert torch.equal(rebuilt.layers[0].qkv_bias.view(torch.int16), state.layers[0].qkv_bias.view(torch.int16))
    assert rebuilt.lm_head.group == GROUP


def test_equal_plans_give_equal_bytes(tmp_path):
    a = _write(tmp_path / "a.aoto", _fake_state(3))
    b = _write(tmp_path / "b.aoto", _fake_state(3))
    assert a.read_bytes() == b.read_bytes()


def test_aliased_state_is_written_once(tmp_path):
    state = _fake_state()
    state.layers[1].input_norm = state.layers[0].input_norm   # one tensor, two roles
    path = _write(tmp_path / "alias.aoto", state)
    manifest = artifact.read_artifact_manifest(path)
    entries = {e["name"]: e for e in manifest["entrypoint"]["state"]}
    assert entries["layers.0.input_norm"]["file"] == entries["layers.1.input_norm"]["file"]
    with zipfile.ZipFile(path) as archive:
        files = [n for n in archive.namelist() if n.startswith("state/")]
    assert len(files) == len(entries) - 1
    contents = artifact.read_artifact(path)
    assert contents.state["layers.0.input_norm"][0] == contents.state["layers.1.input_norm"][0]


@pytest.mark.parametrize("target", ["state/00003.bin", "selections.json", "code/gfx950.hsaco"])
def test_tampered_payload_is_refused(tmp_path, target):
    path = _write(tmp_path / "t.aoto")

    def edit(name, payload):
        if name != target:
            return payload
        if name == "selections.json":
            records = json.loads(payload)
            records[1]["artifact_name"] = "some_other_kernel"
            return json.dumps(records, sort_keys=True, separators=(",", ":")).encode()
        return bytes([payload[0] ^ 1]) + payload[1:]

    _rewrite(path, edit)
    with pytest.raises(ArtifactCompatibilityError, match="digest mismatch"):
        artifact.read_artifact(path)


@pytest.mark.parametrize("field,value,message", [
    ("format_version", 5, "format version"),
    ("abi_version", "aoto_hip-1", "ABI mismatch"),
    ("target", "apple-metal", "unsupported artifact target"),
    ("format", "something-else", "unsupported artifact format"),
])
def test_incompatible_manifest_is_refused(tmp_path, field, value, message):
    path = _write(tmp_path / "m.aoto")
    _edit_manifest(path, lambda m: m.__setitem__(field, value))
    with pytest.raises(ArtifactCompatibilityError, match=message):
        artifact.read_artifact_manifest(path)


def test_other_architecture_and_missing_fields_are_refused(tmp_path):
    path = _write(tmp_path / "arch.aoto", profile={**PROFILE, "architecture": "gfx942"})
    with pytest.raises(ArtifactCompatibilityError, match="gfx942"):
        artifact.read_artifact(path)
    path = _write(tmp_path / "fields.aoto")
    _edit_manifest(path, lambda m: m.pop("payload_digests"))
    with pytest.raises(ArtifactCompatibilityError, match="missing fields"):
        artifact.read_artifact_manifest(path)


def test_state_entry_that_does_not_match_its_bytes_is_refused(tmp_path):
    path = _write(tmp_path / "shape.aoto")

    def change(manifest):
        entry = manifest["entrypoint"]["state"][0]
        entry["shape"] = [entry["shape"][0] + 1, entry["shape"][1]]

    _edit_manifest(path, change)
    with pytest.raises(ArtifactCompatibilityError, match="do not hold"):
        artifact.read_artifact(path)


def test_payload_names_must_stay_inside_the_archive(tmp_path):
    path = _write(tmp_path / "name.aoto")
    _edit_manifest(path, lambda m: m["payloads"].__setitem__("code_object", "../outside.hsaco"))
    with pytest.raises(ArtifactCompatibilityError, match="relative archive path"):
        artifact.read_artifact(path)


def test_not_an_archive_is_refused(tmp_path):
    path = tmp_path / "junk.aoto"
    path.write_bytes(b"not a zip file")
    with pytest.raises(ArtifactCompatibilityError, match="not an aotolith artifact"):
        artifact.read_artifact_manifest(path)
