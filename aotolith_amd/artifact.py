"""Artifacts of the hip-gfx950 target: a compiled plan's gfx950 code object,
kernel selections and packed state in one archive, reloadable in a fresh process.

Counterpart of the reference's ``artifact.py`` (``save_compiled`` /
``load_compiled_module`` / ``read_artifact_manifest``, src/aotolith/artifact.py:
82-520) for the static-cache decoder plans this target compiles:

* the archive is a zip with the reference's layout conventions - a canonical
  JSON ``manifest.json`` (sorted keys, fixed entry timestamps, so equal plans
  give equal bytes), payload files named in ``payloads`` with sha256 digests in
  ``payload_digests``, and the plan state as ``state/NNNNN.bin`` entries, an
  aliased tensor written once (artifact.py:150-180);
* the manifest keeps the reference's validation order - format, format
  version, ABI, target, required fields, then the device profile when asked
  (artifact.py:437-512);
* what is new for this target: the gfx950 code object is a payload
  (``code/gfx950.hsaco``, digest in ``payload_digests["code_object"]``) that the
  loader installs instead of re-emitting kernel source (the reference rebuilds
  Metal kernels from the stored graph, artifact.py:367-384), the profile records
  ``architecture = "gfx950"`` and the loader refuses any other architecture, the
  ABI is the C ABI of ``include/aoto_hip.h`` the code object's kernels were
  built against, and ``FORMAT_VERSION`` is 7 (the reference's is 5; 7: selections name the
  exact kernel symbols each node launches).

A static-cache runtime saves as the reference's does (models/decoder.py:953-958):
``prefix.prefill.aoto`` and ``prefix.decode.aoto``, each a complete artifact of
one plan; a bucketed runtime saves each bucket under ``prefix.<width>``
(models/decoder.py:1395-1404). Loading rebuilds the plans over the stored state
and checks that the rebuilt selections equal the stored ones
(artifact.py:685-726); runtimes loaded together share one device state
(``share_plan_state``, buckets.py:183-218).
"""

from __future__ import annotations

import dataclasses
import glob
import hashlib
import json
import os
import re
import tempfile
import zipfile
from collections.abc import Mapping, Sequence
from pathlib import Path, PurePosixPath
from typing import Any

import numpy as np

from ._version import __version__
from .errors import ArtifactCompatibilityError, ArtifactError
from .plan import ARCHITECTURE, TARGET
from .selection import KernelBenchmark, KernelSelection

ARTIFACT_FORMAT = "aotolith"
FORMAT_VERSION = 7
_SUPPORTED_FORMAT_VERSIONS = (7,)
KINDS = ("prefill", "decode", "graph")
CODE_OBJECT_ENTRY = "code/gfx950.hsaco"
_ZIP_TIMESTAMP = (1980, 1, 1, 0, 0, 0)
_DTYPES = {"bfloat16": 2, "int32": 4, "int64": 8, "float32": 4, "bool": 1, "uint8": 1, "int8": 1}
_REQUIRED = ("entrypoint", "compile_options", "profile", "payload_digests", "payloads")


def abi_version() -> str:
    """The C-ABI version of the loaded library, as stored in manifests."""

    from . import _lib

    return f"aoto_hip-{int(_lib.library().aoto_hip_abi_version())}"


# ----------------------------------------------------------------------------- encoding
def _canonical_json(payload: object) -> bytes:
    return json.dumps(payload, sort_keys=True, separators=(",", ":"), ensure_ascii=True).encode("ascii")


def _digest(payload: bytes) -> str:
    return hashlib.sha256(payload).hexdigest()


def _encode_selection(s: KernelSelection) -> dict[str, object]:
    return {
        "op_index": s.op_index, "op": s.op, "output_id": s.output_id, "implementation": s.implementation,
        "kind": s.kind, "reason": s.reason, "artifact_name": s.artifact_name,
        "benchmarks": [dataclasses.asdict(b) for b in s.benchmarks], "autotuned": s.autotuned,
        "device_name": s.device_name, "device_architecture": s.device_architecture,
    }


def _decode_selection(d: Mapping[str, Any]) -> KernelSelection:
    try:
        benchmarks = tuple(
            KernelBenchmark(**{**b, "samples_seconds": tuple(b["samples_seconds"])}) for b in d["benchmarks"]
        )
        return KernelSelection(
            op_index=int(d["op_index"]), op=str(d["op"]), output_id=str(d["output_id"]),
            implementation=str(d["implementation"]), kind=str(d["kind"]), reason=str(d["reason"]),
            artifact_name=d["artifact_name"], benchmarks=benchmarks, autotuned=bool(d["autotuned"]),
            device_name=d["device_name"], device_architecture=d["device_architecture"],
        )
    except (KeyError, TypeError, ValueError) as error:
        raise ArtifactCompatibilityError(f"artifact selection record is malformed: {error}") from error


def _tensor_bytes(tensor) -> tuple[bytes, str, list[int]]:
    import torch

    names = {torch.bfloat16: "bfloat16", torch.int32: "int32", torch.int64: "int64", torch.float32: "float32",
             torch.bool: "bool", torch.uint8: "uint8", torch.int8: "int8"}
    if tensor.dtype not in names:
        raise ArtifactError(f"cannot store a {tensor.dtype} state tensor")
    host = tensor.detach().to("cpu").contiguous()
    raw = host.reshape(-1).view(torch.uint8).numpy().tobytes()
    return raw, names[tensor.dtype], [int(d) for d in host.shape]


def _write_entry(archive: zipfile.ZipFile, name: str, payload: bytes, *, compress: bool) -> None:
    info = zipfile.ZipInfo(name, date_time=_ZIP_TIMESTAMP)
    info.compress_type = zipfile.ZIP_DEFLATED if compress else zipfile.ZIP_STORED
    info.external_attr = 0o644 << 16
    archive.writestr(info, payload)


# ----------------------------------------------------------------------------- state naming
def state_items(state) -> list[tuple[str, Any]]:
    """``(name, tensor)`` of a DecoderState in a fixed order."""

    items = [("embed", state.embed), ("final_norm", state.final_norm),
             ("lm_head.packed", state.lm_head.packed), ("lm_head.scales", state.lm_head.scales)]
    for i, layer in enumerate(state.layers):
        for key in ("qkv", "o", "gate", "up", "down"):
            weight = getattr(layer, key)
            items += [(f"layers.{i}.{key}.packed", weight.packed), (f"layers.{i}.{key}.scales", weight.scales)]
        items += [(f"layers.{i}.input_norm", layer.input_norm), (f"layers.{i}.post_norm", layer.post_norm)]
        if layer.qkv_bias is not None:
            items.append((f"layers.{i}.qkv_bias", layer.qkv_bias))
    return items


def state_from_items(spec, named: Mapping[str, Any], group: int, bits: int = 4):
    """Rebuild a DecoderState from ``state_items`` names (tensors already on the device)."""

    from .decoder import DecoderState, LayerState, PackedWeight

    def take(name):
        if name not in named:
            raise ArtifactCompatibilityError(f"artifact state has no entry {name!r}")
        return named[name]

    def packed(prefix):
        return PackedWeight(take(f"{prefix}.packed"), take(f"{prefix}.scales"), group, bits)

    layers = []
    for i in range(spec.layers):
        layers.append(LayerState(
            qkv=packed(f"layers.{i}.qkv"), o=packed(f"layers.{i}.o"), gate=packed(f"layers.{i}.gate"),
            up=packed(f"layers.{i}.up"), down=packed(f"layers.{i}.down"),
            input_norm=take(f"layers.{i}.input_norm"), post_norm=take(f"layers.{i}.post_norm"),
            qkv_bias=named.get(f"layers.{i}.qkv_bias") if spec.qkv_bias else None,
        ))
    return DecoderState(embed=take("embed"), final_norm=take("final_norm"), lm_head=packed("lm_head"),
                        layers=layers)


# ----------------------------------------------------------------------------- writing
def write_artifact(
    path: str | os.PathLike[str],
    *,
    kind: str,
    spec,
    config: Mapping[str, Any],
    state: Sequence[tuple[str, Any]],
    selections: Sequence[KernelSelection],
    code_object: bytes,
    profile: Mapping[str, Any],
    graph: Mapping[str, Any] | None = None,
) -> Path:
    """Write one plan's archive. ``state`` is ``(name, tensor)`` pairs (any device).

    Decoder plans carry their ``spec`` and ``config``; a graph plan (``kind``
    ``"graph"``) carries its encoded lowered graph instead of a spec.
    """

    if kind not in KINDS:
        raise ArtifactError(f"unknown plan kind {kind!r}; expected one of {KINDS}")
    if not code_object:
        raise ArtifactError("an artifact needs the gfx950 code object its plan runs")
    selections_bytes = _canonical_json([_encode_selection(s) for s in selections])
    entries: list[dict[str, object]] = []
    payloads: list[tuple[str, bytes]] = []
    shared: dict[tuple, tuple[str, str]] = {}
    for index, (name, tensor) in enumerate(state):
        key = (tensor.device.type, tensor.device.index, tensor.data_ptr(), tensor.numel(), str(tensor.dtype),
               tuple(tensor.shape), tuple(tensor.stride()))
        raw, dtype, shape = _tensor_bytes(tensor)
        file = shared.get(key)
        if file is None:
            file = (f"state/{index:05d}.bin", _digest(raw))
            shared[key] = file
            payloads.append((file[0], raw))
        entries.append({"name": name, "shape": shape, "dtype": dtype, "nbytes": len(raw), "file": file[0],
                        "digest": file[1]})
    manifest = {
        "format": ARTIFACT_FORMAT,
        "format_version": FORMAT_VERSION,
        "abi_version": abi_version(),
        "compiler_version": __version__,
        "target": TARGET,
        "entrypoint": {
            "kind": kind,
            "plan": "graph" if kind == "graph" else "static_cache_decoder",
            "spec": None if spec is None else dataclasses.asdict(spec),
            "config": dict(config),
            "state": entries,
            **({"graph": dict(graph)} if graph is not None else {}),
        },
        "compile_options": {"codegen_matmul": True, "codegen_attention": True, "autotune": False,
                            "quantize": config.get("group_size"),
                            "quantize_bits": int(config.get("quantize_bits", 4))},
        "profile": dict(profile),
        "payload_digests": {"selections": _digest(selections_bytes), "code_object": _digest(code_object)},
        "payloads": {"selections": "selections.json", "code_object": CODE_OBJECT_ENTRY},
    }
    destination = Path(path)
    destination.parent.mkdir(parents=True, exist_ok=True)
    with tempfile.NamedTemporaryFile(mode="wb", dir=destination.parent, delete=False) as temporary:
        temporary_path = Path(temporary.name)
    try:
        with zipfile.ZipFile(temporary_path, "w") as archive:
            _write_entry(archive, "manifest.json", _canonical_json(manifest), compress=True)
            _write_entry(archive, "selections.json", selections_bytes, compress=True)
            _write_entry(archive, CODE_OBJECT_ENTRY, code_object, compress=True)
            for name, raw in payloads:
                # packed int4 words do not compress; store state as is
                _write_entry(archive, name, raw, compress=False)
        temporary_path.replace(destination)
    finally:
        temporary_path.unlink(missing_ok=True)
    return destination


def device_profile(device) -> dict[str, object]:
    import torch

    props = torch.cuda.get_device_properties(device)
    arch = str(getattr(props, "gcnArchName", "") or "")
    return {"device_name": props.name, "architecture": arch.split(":", 1)[0] or None, "arch_features": arch}


def save_plan(runtime, kind: str, path: str | os.PathLike[str]) -> Path:
    """Save ``runtime.prefill`` or ``runtime.decode`` as one artifact."""

    from . import _lib

    engine = runtime.engine
    device = engine.device.index if engine.device.index is not None else 0
    image = _lib.installed_image(device)
    if image is None:
        _lib.ensure_code_object(device)
        image = _lib.installed_image(device)
    plan = runtime.prefill if kind == "prefill" else runtime.decode
    config = {"prompt_length": runtime.prompt_length, "max_new_tokens": runtime.max_new_tokens,
              "cache_capacity": runtime.cache_capacity, "group_size": runtime.group_size,
              "quantize_bits": runtime.quantize_bits, "memory": runtime.memory,
              "attention_splits": engine.attention_splits}
    return write_artifact(path, kind=kind, spec=runtime.spec, config=config, state=state_items(engine.state),
                          selections=plan.selections, code_object=image, profile=device_profile(engine.device))


def save_runtime(runtime, prefix: str | os.PathLike[str]) -> tuple[Path, Path]:
    """``prefix.prefill.aoto`` and ``prefix.decode.aoto`` (models/decoder.py:953-958)."""

    path = Path(prefix)
    return (save_plan(runtime, "prefill", path.with_name(path.name + ".prefill.aoto")),
            save_plan(runtime, "decode", path.with_name(path.name + ".decode.aoto")))


# ----------------------------------------------------------------------------- reading
def _open(path: Path) -> zipfile.ZipFile:
    try:
        return zipfile.ZipFile(path, "r")
    except FileNotFoundError:
        raise
    except (zipfile.BadZipFile, OSError) as error:
        raise ArtifactCompatibilityError(f"{path} is not an aotolith artifact: {error}") from error


def _safe_name(name: object) -> str:
    text = str(name)
    pure = PurePosixPath(text)
    if pure.is_absolute() or ".." in pure.parts or not text:
        raise ArtifactCompatibilityError(f"artifact payload name {text!r} is not a relative archive path")
    return text


def _read(archive: zipfile.ZipFile, name: object, digest: object, label: str) -> bytes:
    name = _safe_name(name)
    try:
        payload = archive.read(name)
    except KeyError as error:
        raise ArtifactCompatibilityError(f"artifact has no {label} payload {name!r}") from error
    actual = _digest(payload)
    if actual != digest:
        raise ArtifactCompatibilityError(f"{label} digest mismatch: expected {digest!r}, got {actual}")
    return payload


def _validate_manifest(manifest: Mapping[str, Any], *, require_device_match: bool, device=None) -> None:
    if not isinstance(manifest, Mapping) or manifest.get("format") != ARTIFACT_FORMAT:
        raise ArtifactCompatibilityError(f"unsupported artifact format: {manifest.get('format')!r}")
    version = manifest.get("format_version")
    if version not in _SUPPORTED_FORMAT_VERSIONS:
        raise ArtifactCompatibilityError(
            f"artifact format version mismatch: expected one of {list(_SUPPORTED_FORMAT_VERSIONS)}, got {version!r}"
        )
    current_abi = abi_version()
    if manifest.get("abi_version") != current_abi:
        raise ArtifactCompatibilityError(
            f"artifact ABI mismatch: built against {manifest.get('abi_version')!r}, this library is {current_abi!r}",
            hint="the stored code object's kernel arguments must match the host launchers; recompile the plan",
        )
    if manifest.get("target") != TARGET:
        raise ArtifactCompatibilityError(f"unsupported artifact target: {manifest.get('target')!r}",
                                         hint=f"this package loads {TARGET!r} artifacts")
    missing = [key for key in _REQUIRED if key not in manifest]
    if missing:
        raise ArtifactCompatibilityError(f"artifact manifest is missing fields: {sorted(missing)}")
    entry = manifest["entrypoint"]
    if not isinstance(entry, Mapping) or entry.get("kind") not in KINDS:
        raise ArtifactCompatibilityError(f"artifact entrypoint kind must be one of {KINDS}")
    profile = manifest["profile"]
    if not isinstance(profile, Mapping) or profile.get("architecture") != ARCHITECTURE:
        raise ArtifactCompatibilityError(
            f"artifact code object is for {profile.get('architecture') if isinstance(profile, Mapping) else None!r}, "
            f"not {ARCHITECTURE!r}"
        )
    if require_device_match:
        _validate_device_profile(profile, device)


def _validate_device_profile(profile: Mapping[str, Any], device=None) -> None:
    import torch

    if not profile.get("device_name") or not profile.get("architecture"):
        raise ArtifactCompatibilityError("artifact has no device profile for strict device matching")
    if not torch.cuda.is_available():
        raise ArtifactCompatibilityError("cannot query the current GPU for artifact validation")
    current = device_profile(torch.cuda.current_device() if device is None else device)
    if (current["device_name"], current["architecture"]) != (profile["device_name"], profile["architecture"]):
        raise ArtifactCompatibilityError(
            f"artifact device mismatch: compiled for {profile['device_name']!r} ({profile['architecture']!r}), "
            f"running on {current['device_name']!r} ({current['architecture']!r})"
        )


def read_artifact_manifest(path: str | os.PathLike[str], *, require_device_match: bool = False) -> dict[str, Any]:
    """Read and validate a manifest without touching the GPU (artifact.py:424-434)."""

    with _open(Path(path)) as archive:
        try:
            manifest = json.loads(archive.read("manifest.json"))
        except (KeyError, ValueError) as error:
            raise ArtifactCompatibilityError(f"{path}: unreadable manifest: {error}") from error
    _validate_manifest(manifest, require_device_match=require_device_match)
    return dict(manifest)


@dataclasses.dataclass
class ArtifactContents:
    """A validated archive on the host: manifest, selections, code object and state bytes."""

    manifest: dict[str, Any]
    selections: tuple[KernelSelection, ...]
    code_object: bytes
    state: dict[str, tuple[bytes, str, tuple[int, ...]]]  # name -> (raw, dtype, shape)

    @property
    def kind(self) -> str:
        return self.manifest["entrypoint"]["kind"]

    def state_digest(self) -> str:
        """One digest over every state entry (names, shapes, dtypes, payload digests)."""

        entries = [(e["name"], e["shape"], e["dtype"], e["digest"]) for e in self.manifest["entrypoint"]["state"]]
        return _digest(_canonical_json(entries))


def read_artifact(path: str | os.PathLike[str], *, require_device_match: bool = False) -> ArtifactContents:
    """Validate every digest of an archive and return its contents on the host."""

    path = Path(path)
    with _open(path) as archive:
        try:
            manifest = json.loads(archive.read("manifest.json"))
        except (KeyError, ValueError) as error:
            raise ArtifactCompatibilityError(f"{path}: unreadable manifest: {error}") from error
        _validate_manifest(manifest, require_device_match=require_device_match)
        payloads, digests = manifest["payloads"], manifest["payload_digests"]
        selections_raw = _read(archive, payloads.get("selections"), digests.get("selections"), "kernel selections")
        code_object = _read(archive, payloads.get("code_object"), digests.get("code_object"), "code object")
        try:
            records = json.loads(selections_raw)
        except ValueError as error:
            raise ArtifactCompatibilityError(f"artifact selections are not JSON: {error}") from error
        if not isinstance(records, list):
            raise ArtifactCompatibilityError("artifact selections must be a list")
        selections = tuple(_decode_selection(r) for r in records)
        state: dict[str, tuple[bytes, str, tuple[int, ...]]] = {}
        cache: dict[str, bytes] = {}
        for entry in manifest["entrypoint"].get("state", []):
            try:
                name, file, digest = str(entry["name"]), str(entry["file"]), entry["digest"]
                dtype, shape = str(entry["dtype"]), tuple(int(d) for d in entry["shape"])
            except (KeyError, TypeError, ValueError) as error:
                raise ArtifactCompatibilityError(f"artifact state entry is malformed: {error}") from error
            if dtype not in _DTYPES:
                raise ArtifactCompatibilityError(f"state {name!r} has unsupported dtype {dtype!r}")
            raw = cache.get(file)
            if raw is None:
                raw = _read(archive, file, digest, f"state {name!r}")
                cache[file] = raw
            elif _digest(raw) != digest:
                raise ArtifactCompatibilityError(f"state {name!r} digest mismatch")
            if len(raw) != int(np.prod(shape, dtype=np.int64)) * _DTYPES[dtype] or len(raw) != entry.get("nbytes"):
                raise ArtifactCompatibilityError(
                    f"state {name!r}: {len(raw)} bytes do not hold a {dtype} tensor of shape {list(shape)}"
                )
            state[name] = (raw, dtype, shape)
    return ArtifactContents(manifest=manifest, selections=selections, code_object=code_object, state=state)


# ----------------------------------------------------------------------------- loading on the GPU
def _install_code_object(image: bytes, device: int) -> None:
    from . import _lib

    digest = _lib.code_object_digest(image)
    current = _lib.installed_digest(device)
    if current is None:
        _lib.install_code_object(image, device)
    elif current != digest:
        raise ArtifactCompatibilityError(
            f"device {device} already runs a different gfx950 code object ({current[:12]}...) than the "
            f"artifact's ({digest[:12]}...)",
            hint="load the artifact in a fresh process; live plans keep their kernels",
        )


def _device_state(contents: ArtifactContents, device) -> dict[str, Any]:
    import torch

    dtypes = {"bfloat16": torch.bfloat16, "int32": torch.int32, "int64": torch.int64, "float32": torch.float32,
              "bool": torch.bool, "uint8": torch.uint8, "int8": torch.int8}
    tensors: dict[str, Any] = {}
    by_file: dict[str, Any] = {}
    files = {e["name"]: e["file"] for e in contents.manifest["entrypoint"]["state"]}
    for name, (raw, dtype, shape) in contents.state.items():
        tensor = by_file.get(files[name])
        if tensor is None:
            host = torch.frombuffer(bytearray(raw), dtype=torch.uint8)
            tensor = host.view(dtypes[dtype]).reshape(shape).to(device)
            by_file[files[name]] = tensor  # aliased entries stay aliased on the device
        tensors[name] = tensor
    return tensors


def _spec(contents: ArtifactContents):
    from .decoder import DecoderSpec

    try:
        return DecoderSpec(**contents.manifest["entrypoint"]["spec"])
    except TypeError as error:
        raise ArtifactCompatibilityError(f"artifact decoder spec is malformed: {error}") from error


def _build(contents_list: Sequence[ArtifactContents], device, state_cache: dict):
    """One runtime from the artifacts of its plans (same spec, config and state)."""

    from .decoder import compile_decoder_state

    first = contents_list[0]
    spec = _spec(first)
    config = first.manifest["entrypoint"]["config"]
    for other in contents_list[1:]:
        if (other.manifest["entrypoint"]["spec"] != first.manifest["entrypoint"]["spec"]
                or other.manifest["entrypoint"]["config"] != config):
            raise ArtifactCompatibilityError("the prefill and decode artifacts describe different plans")
        if other.state_digest() != first.state_digest():
            raise ArtifactCompatibilityError("the prefill and decode artifacts hold different state")
        if other.code_object != first.code_object:
            raise ArtifactCompatibilityError("the prefill and decode artifacts hold different code objects")
    device_index = device.index if device.index is not None else 0
    _install_code_object(first.code_object, device_index)
    bits = int(config.get("quantize_bits", 4))
    if bits not in (4, 8):
        raise ArtifactCompatibilityError(f"artifact records quantize_bits={bits}; this package packs 4 or 8 bits")
    key = (first.state_digest(), int(config["group_size"]), bits)
    state = state_cache.get(key)
    if state is None:
        state = state_from_items(spec, _device_state(first, device), int(config["group_size"]), bits)
        state_cache[key] = state
    runtime = compile_decoder_state(
        spec, state, prompt_length=int(config["prompt_length"]), max_new_tokens=int(config["max_new_tokens"]),
        group_size=int(config["group_size"]), memory=str(config.get("memory", "latency")),
        attention_splits=int(config.get("attention_splits", 0)),
    )
    for contents in contents_list:
        plan = runtime.prefill if contents.kind == "prefill" else runtime.decode
        rebuilt = [_encode_selection(s) for s in plan.selections]
        stored = [_encode_selection(s) for s in contents.selections]
        if rebuilt != stored:
            raise ArtifactCompatibilityError(
                f"the rebuilt {contents.kind} plan selects different kernels than the artifact records",
                hint="the artifact was written by another version of this package; recompile it",
            )
    return runtime


def _torch_device(device):
    import torch

    if not torch.cuda.is_available():
        from .errors import DeviceError

        raise DeviceError("loading a hip-gfx950 artifact needs a ROCm GPU")
    return torch.device("cuda", torch.cuda.current_device() if device is None else device)


def load_compiled_module(path: str | os.PathLike[str], *, require_device_match: bool = False, device=None):
    """Load one plan artifact; returns its ``CompiledPlan`` (``.runtime`` is the runtime built around it)."""

    dev = _torch_device(device)
    contents = read_artifact(path, require_device_match=require_device_match)
    if contents.kind == "graph":
        return _load_graph(contents, dev)
    runtime = _build([contents], dev, {})
    plan = runtime.prefill if contents.kind == "prefill" else runtime.decode
    plan._keepalive = runtime  # the caller holds only the plan
    return plan


def _pair_paths(prefix) -> tuple[Path, Path]:
    path = Path(prefix)
    return path.with_name(path.name + ".prefill.aoto"), path.with_name(path.name + ".decode.aoto")


def load_runtime(prefix: str | os.PathLike[str] | None = None, *, prefill: str | os.PathLike[str] | None = None,
                 decode: str | os.PathLike[str] | None = None, require_device_match: bool = False, device=None):
    """A static-cache runtime from ``prefix.prefill.aoto`` + ``prefix.decode.aoto`` (or explicit paths)."""

    if prefix is not None:
        prefill_path, decode_path = _pair_paths(prefix)
    else:
        if prefill is None or decode is None:
            raise ArtifactError("load_runtime needs a prefix or both the prefill and decode paths")
        prefill_path, decode_path = Path(prefill), Path(decode)
    dev = _torch_device(device)
    contents = [read_artifact(prefill_path, require_device_match=require_device_match),
                read_artifact(decode_path, require_device_match=require_device_match)]
    if [c.kind for c in contents] != ["prefill", "decode"]:
        raise ArtifactCompatibilityError("expected a prefill artifact and a decode artifact")
    return _build(contents, dev, {})


def load_bucketed(prefix: str | os.PathLike[str], *, prompt_lengths: Sequence[int] | None = None,
                  require_device_match: bool = False, device=None):
    """The buckets saved by ``DecoderBucketedRuntime.save(prefix)``, sharing one state (buckets.py:682-740)."""

    from .decoder import DecoderBucketedRuntime

    base = Path(prefix)
    if prompt_lengths is None:
        pattern = re.compile(re.escape(base.name) + r"\.(\d+)\.prefill\.aoto$")
        found = sorted(int(m.group(1)) for f in glob.glob(str(base.with_name(base.name + ".*.prefill.aoto")))
                       if (m := pattern.search(os.path.basename(f))))
        widths = found
    else:
        widths = sorted(int(w) for w in prompt_lengths)
    if not widths:
        raise ArtifactError(f"no bucket artifacts found for prefix {str(base)!r}")
    dev = _torch_device(device)
    cache: dict = {}
    runtimes = []
    for width in widths:
        p, d = _pair_paths(base.with_name(f"{base.name}.{width}"))
        contents = [read_artifact(p, require_device_match=require_device_match),
                    read_artifact(d, require_device_match=require_device_match)]
        runtimes.append(_build(contents, dev, cache))
    steps = {r.max_new_tokens for r in runtimes}
    if len(steps) != 1:
        raise ArtifactCompatibilityError(f"bucket artifacts disagree on max_new_tokens: {sorted(steps)}")
    return DecoderBucketedRuntime(buckets=tuple(runtimes), max_new_tokens=steps.pop())


def save_compiled(compiled, path: str | os.PathLike[str]) -> Path:
    """Save a compiled plan as one artifact (artifact.py:82-269).

    Takes ``runtime.prefill`` / ``runtime.decode`` of a static-cache runtime, or
    the result of ``compile_callable`` / ``compile_module``.
    """

    from .compiler import CompilationResult, CompiledModulePlan

    if isinstance(compiled, (CompilationResult, CompiledModulePlan)):
        return save_graph_plan(compiled, path)
    runtime = getattr(compiled, "runtime", None)
    if runtime is None or getattr(compiled, "name", None) not in KINDS:
        raise ArtifactError("save_compiled takes the prefill or decode plan of a compiled static-cache runtime")
    return save_plan(runtime, compiled.name, path)


# ----------------------------------------------------------------------------- graph plans
def _encode_value(value):
    import torch

    from .graph import Ref

    if isinstance(value, Ref):
        return {"ref": value.name}
    if isinstance(value, torch.dtype):
        return {"dtype": str(value)}
    if isinstance(value, torch.device):
        return {"device": str(value)}
    if isinstance(value, (torch.layout, torch.memory_format)):
        return {"torch": str(value)}
    if isinstance(value, tuple):
        return {"tuple": [_encode_value(v) for v in value]}
    if isinstance(value, list):
        return [_encode_value(v) for v in value]
    if isinstance(value, dict):
        return {"map": {str(k): _encode_value(v) for k, v in value.items()}}
    if value is None or isinstance(value, (bool, int, float, str)):
        return value
    raise ArtifactError(f"cannot store a graph argument of type {type(value).__name__}")


def _torch_attr(text: str):
    import torch

    name = text.removeprefix("torch.")
    value = getattr(torch, name, None)
    if value is None:
        raise ArtifactCompatibilityError(f"unknown torch constant {text!r} in the stored graph")
    return value


def _decode_value(value):
    import torch

    from .graph import Ref

    if isinstance(value, list):
        return [_decode_value(v) for v in value]
    if isinstance(value, dict):
        if "ref" in value:
            return Ref(str(value["ref"]))
        if "dtype" in value:
            return _torch_attr(value["dtype"])
        if "device" in value:
            return torch.device(value["device"])
        if "torch" in value:
            return _torch_attr(value["torch"])
        if "tuple" in value:
            return tuple(_decode_value(v) for v in value["tuple"])
        if "map" in value:
            return {k: _decode_value(v) for k, v in value["map"].items()}
        raise ArtifactCompatibilityError(f"malformed stored graph value {value!r}")
    return value


def encode_graph(graph) -> dict[str, Any]:
    """The lowered graph as JSON-safe data (node records, inputs, outputs; state goes to payloads)."""

    return {
        "inputs": list(graph.inputs),
        "input_meta": {k: {"shape": list(shape), "dtype": str(dtype)} for k, (shape, dtype) in
                       graph.input_meta.items()},
        "state_names": list(graph.state_names),
        "state_labels": dict(graph.state_labels),
        "nodes": [{"name": n.name, "op": n.op, "args": _encode_value(tuple(n.args)),
                   "kwargs": _encode_value(dict(n.kwargs)), "shape": None if n.shape is None else list(n.shape),
                   "dtype": None if n.dtype is None else str(n.dtype)} for n in graph.nodes],
        "outputs": _encode_value(list(graph.outputs)),
    }


def decode_graph(data: Mapping[str, Any], state: Mapping[str, Any]):
    from .graph import LoweredGraph, Node

    try:
        nodes = [Node(str(n["name"]), str(n["op"]), tuple(_decode_value(n["args"])), dict(_decode_value(n["kwargs"])),
                      None if n["shape"] is None else tuple(int(d) for d in n["shape"]),
                      None if n["dtype"] is None else _torch_attr(n["dtype"])) for n in data["nodes"]]
        meta = {k: (tuple(int(d) for d in v["shape"]), _torch_attr(v["dtype"])) for k, v in data["input_meta"].items()}
        names = [str(n) for n in data["state_names"]]
        return LoweredGraph(inputs=[str(i) for i in data["inputs"]], input_meta=meta, state_names=names,
                            state={n: state[n] for n in names}, nodes=nodes, outputs=list(_decode_value(data["outputs"])),
                            state_labels={str(k): str(v) for k, v in data.get("state_labels", {}).items()})
    except (KeyError, TypeError, ValueError) as error:
        raise ArtifactCompatibilityError(f"stored graph is malformed: {error}") from error


def save_graph_plan(compiled, path: str | os.PathLike[str]) -> Path:
    """Save a ``compile_callable`` / ``compile_module`` result (artifact.py:82-269 for graph plans)."""

    import torch

    from . import _lib
    from .compiler import CompiledModulePlan

    result = compiled.compilation if isinstance(compiled, CompiledModulePlan) else compiled
    graph = result.lowered_graph
    runner = result.plan._keepalive
    device = runner.device
    image = _lib.installed_image(device.index if device.index is not None else 0)
    if image is None:
        _lib.ensure_code_object(device.index)
        image = _lib.installed_image(device.index)
    config: dict[str, Any] = {"entry": "module" if isinstance(compiled, CompiledModulePlan) else "callable",
                              "name": result.plan.name}
    if isinstance(compiled, CompiledModulePlan):
        config.update({"input_count": compiled.input_count, "state_names": list(compiled.state_names),
                       "tensor_kwarg_names": list(compiled.tensor_kwarg_names)})
    state = [(name, runner.state[name] if isinstance(runner.state[name], torch.Tensor)
              else torch.as_tensor(runner.state[name])) for name in graph.state_names]
    return write_artifact(path, kind="graph", spec=None, config=config, state=state,
                          selections=result.plan.selections, code_object=image, profile=device_profile(device),
                          graph=encode_graph(graph))


def _load_graph(contents: ArtifactContents, device):
    from .compiler import CompilationResult, CompiledModulePlan
    from .graph_ops import build_graph_plan

    _install_code_object(contents.code_object, device.index if device.index is not None else 0)
    entry = contents.manifest["entrypoint"]
    state = _device_state(contents, device)
    graph = decode_graph(entry.get("graph") or {}, state)
    config = entry["config"]
    plan, runner = build_graph_plan(graph, name=str(config.get("name", "graph")))
    plan._keepalive = runner
    rebuilt = [_encode_selection(s) for s in plan.selections]
    stored = [_encode_selection(s) for s in contents.selections]
    if rebuilt != stored:
        raise ArtifactCompatibilityError("the rebuilt graph plan selects different kernels than the artifact records",
                                         hint="the artifact was written by another version of this package")
    result = CompilationResult(plan=plan, input_graph=graph, lowered_graph=graph)
    if config.get("entry") != "module":
        return result
    return CompiledModulePlan(compilation=result, input_count=int(config["input_count"]),
                              state_names=tuple(config.get("state_names", ())),
                              tensor_kwarg_names=tuple(config.get("tensor_kwarg_names", ())), _runner=runner)


__all__ = [
    "ARTIFACT_FORMAT",
    "ArtifactContents",
    "FORMAT_VERSION",
    "load_bucketed",
    "load_compiled_module",
    "load_runtime",
    "read_artifact",
    "read_artifact_manifest",
    "save_compiled",
    "save_graph_plan",
    "save_plan",
    "save_runtime",
    "write_artifact",
]
