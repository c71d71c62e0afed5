"""Static-KV-cache W4 (and W8) decoder runtime for the hip-gfx950 target.

The host-side mirror of the reference's static-cache adapter
(``models/decoder.py``): the same cache ABI, the same plan pair per prompt
bucket and the same runtime methods (``prefill_ids``, ``prefill_padded``,
``pad_cache``, ``decode_token``, ``decode_mask``, ``greedy_generate``,
``memory_footprint``, ``check_memory_budget``, ``save``), with every node of
both plans a gfx950 kernel:

prefill (per layer)   rms_norm -> W4 GEMM (+q/k/v bias) -> fused RoPE + cache fill
                      -> MFMA flash attention -> W4 GEMM (+residual) -> rms_norm
                      -> W4 GEMM (gate) -> W4 GEMM (up, silu_mul) -> W4 GEMM (down, +residual);
                      the final norm is the LM-head GEMV's prologue on the last row.
decode  (per layer)   W4 GEMV (norm prologue, bias) -> RoPE + KV append
                      -> split-K decode attention -> W4 GEMV (+residual)
                      -> paired gate/up W4 GEMV (norm, silu) -> W4 GEMV (+residual);
                      LM-head GEMV (norm), argmax.

With ``quantize_bits=8`` every W4 kernel above is its eight-bit counterpart
(int8 packer, GEMV and GEMM) and the LM head's argmax runs as its own kernel.

``decode_token`` keeps the reference's functional contract (the cache it
returns is the input window rolled by one slot). ``greedy_generate`` runs the
same kernels on a ring-buffer cache with device-resident step state, captured
once as a HIP graph and replayed per token with no host work in between.
"""

from __future__ import annotations

import contextlib
import gc
import os
from collections.abc import Sequence
from dataclasses import dataclass, field

import numpy as np
import torch

from . import _lib, ops
from .errors import (
    BucketRangeError,
    CompilationError,
    DeviceError,
    DynamicShapeError,
    MemoryBudgetError,
    PlanInputError,
    UnsupportedDTypeError,
    UnsupportedModelError,
)
from .plan import ARCHITECTURE, TARGET, CompiledPlan, PlanNode, require_native
from .selection import KernelSelection

BF16 = torch.bfloat16

#: Family name -> accepted ``config.model_type`` values (models/decoder.py:65-89).
FAMILIES: dict[str, tuple[str, ...]] = {"qwen2": ("qwen2",), "llama": ("llama",)}
_LABELS = {"qwen2": "Qwen2/Qwen2.5", "llama": "Llama"}

#: Targets this package compiles for; the reference's own two are named so the
#: error for them can say where they live.
TARGETS: tuple[str, ...] = (TARGET,)
MEMORY_POLICIES: tuple[str, ...] = ("latency", "balanced", "minimal")


# ----------------------------------------------------------------------------- spec
@dataclass(frozen=True)
class DecoderSpec:
    """The shape of a decoder the adapter compiles (read from a model config)."""

    family: str
    vocab: int
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    theta: float
    qkv_bias: bool
    tied: bool = False
    max_position: int = 1 << 20

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim

    @property
    def attention_width(self) -> int:
        return self.heads * self.head_dim


def family_for(model: torch.nn.Module, *, require: str | None = None) -> str:
    """The family of ``model``; refuse others (models/decoder.py:92-133)."""

    model_type = str(getattr(model.config, "model_type", None))
    family = next((name for name, types in FAMILIES.items() if model_type in types), None)
    if family is None:
        supported = ", ".join(f"{_LABELS[n]} ({'/'.join(t)})" for n, t in FAMILIES.items())
        raise UnsupportedModelError(
            f"the static-cache adapter does not cover model_type {model_type!r}; it covers {supported}",
            hint="add the family once its module tree and causal mask have been checked",
        )
    if require is not None and family != require:
        raise UnsupportedModelError(
            f"this entry point compiles {require} and the model is {_LABELS[family]} ({model_type!r})",
            hint=f"call compile_{family}_static_cache instead",
        )
    return family


def _rope_theta(config) -> float:
    """RoPE base from either config generation.

    transformers < 5 stores ``rope_theta``; transformers 5 moves it into
    ``rope_parameters`` (``{"rope_theta": ..., "rope_type": "default"}``) and
    leaves ``rope_scaling`` as that same dict. Only the default (unscaled) type
    is accepted, as the reference refuses RoPE scaling (models/decoder.py:299-306).
    """

    params = getattr(config, "rope_parameters", None)
    scaling = getattr(config, "rope_scaling", None)
    for block in (params, scaling):
        if isinstance(block, dict):
            kind = block.get("rope_type", block.get("type", "default"))
            if kind not in (None, "default"):
                raise UnsupportedModelError(
                    f"RoPE scaling {kind!r} is not supported yet",
                    hint="the adapter builds one rotary table from rope_theta",
                )
    theta = getattr(config, "rope_theta", None)
    if theta is None and isinstance(params, dict):
        theta = params.get("rope_theta")
    if theta is None and isinstance(scaling, dict):
        theta = scaling.get("rope_theta")
    return float(theta if theta is not None else 10000.0)


def spec_from_model(model: torch.nn.Module, *, require: str | None = None) -> DecoderSpec:
    family = family_for(model, require=require)
    config = model.config
    layer_types = getattr(config, "layer_types", None)
    if getattr(model.model, "has_sliding_layers", False) or (
        isinstance(layer_types, (list, tuple)) and any(t == "sliding_attention" for t in layer_types)
    ):
        raise UnsupportedModelError(
            "sliding-window attention is not supported: the static-cache adapter builds a plain causal mask"
        )
    hidden = int(config.hidden_size)
    heads = int(config.num_attention_heads)
    attention = model.model.layers[0].self_attn
    biases = [getattr(attention, name).bias for name in ("q_proj", "k_proj", "v_proj")]
    if any(b is None for b in biases) and not all(b is None for b in biases):
        raise UnsupportedModelError("the attention has a bias on some of q/k/v and not others")
    act = str(getattr(config, "hidden_act", "silu"))
    if act != "silu":
        raise UnsupportedModelError(
            f"MLP activation {act!r}: the fused gate/up kernels implement silu_mul only",
            hint="the W4 path fuses silu(gate) * up into the projection epilogue",
        )
    return DecoderSpec(
        family=family,
        vocab=int(config.vocab_size),
        hidden=hidden,
        intermediate=int(config.intermediate_size),
        layers=int(config.num_hidden_layers),
        heads=heads,
        kv_heads=int(config.num_key_value_heads),
        head_dim=int(getattr(config, "head_dim", None) or hidden // heads),
        eps=float(config.rms_norm_eps),
        theta=_rope_theta(config),
        qkv_bias=biases[0] is not None,
        tied=bool(getattr(config, "tie_word_embeddings", False)),
        max_position=int(getattr(config, "max_position_embeddings", 1 << 20)),
    )


# ----------------------------------------------------------------------------- state
@dataclass
class PackedWeight:
    """A packed weight in the reference's format: int32 words [N, K/8] (``bits=8``:
    [N, K/4]), bf16 scales [N, K/g]."""

    packed: torch.Tensor
    scales: torch.Tensor
    group: int
    bits: int = 4

    @property
    def out_features(self) -> int:
        return int(self.packed.shape[0])

    @property
    def in_features(self) -> int:
        return int(self.packed.shape[1]) * ops.CODES_PER_WORD[self.bits]

    @property
    def nbytes(self) -> int:
        return self.packed.numel() * 4 + self.scales.numel() * 2


@dataclass
class LayerState:
    qkv: PackedWeight
    o: PackedWeight
    gate: PackedWeight
    up: PackedWeight
    down: PackedWeight
    input_norm: torch.Tensor
    post_norm: torch.Tensor
    qkv_bias: torch.Tensor | None = None


@dataclass
class DecoderState:
    """Device-resident plan state: the packed weights and the bf16 tensors."""

    embed: torch.Tensor
    final_norm: torch.Tensor
    lm_head: PackedWeight
    layers: list[LayerState]

    def tensors(self) -> list[torch.Tensor]:
        out = [self.embed, self.final_norm, self.lm_head.packed, self.lm_head.scales]
        for layer in self.layers:
            for weight in (layer.qkv, layer.o, layer.gate, layer.up, layer.down):
                out += [weight.packed, weight.scales]
            out += [layer.input_norm, layer.post_norm]
            if layer.qkv_bias is not None:
                out.append(layer.qkv_bias)
        return out

    @property
    def weights(self) -> list[PackedWeight]:
        out = [self.lm_head]
        for layer in self.layers:
            out += [layer.qkv, layer.o, layer.gate, layer.up, layer.down]
        return out

    @property
    def bits(self) -> int:
        """The code width of every packed weight (4 or 8); mixed widths are refused."""

        widths = {w.bits for w in self.weights}
        if len(widths) != 1:
            raise CompilationError(f"a decoder state packs every weight at one width, found {sorted(widths)}")
        return widths.pop()

    @property
    def nbytes(self) -> int:
        seen = {}
        for tensor in self.tensors():
            seen[tensor.data_ptr()] = tensor.numel() * tensor.element_size()
        return sum(seen.values())


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise DeviceError(
            f"the {TARGET} target needs a ROCm GPU (MI355X, gfx950); none is visible",
            hint="run on the GPU host, or use the CPU oracle for reference numbers",
        )
    return torch.device("cuda", torch.cuda.current_device())


def _pack(weight: torch.Tensor, group: int, device, bits: int = 4) -> PackedWeight:
    w = weight.detach().to(device=device)
    if w.dtype not in (BF16, torch.float32):
        w = w.to(BF16)
    packed, scales = ops.quantize(w.contiguous(), group, bits)
    return PackedWeight(packed, scales, group, bits)


def pack_model_state(model: torch.nn.Module, spec: DecoderSpec, group: int, bits: int = 4) -> DecoderState:
    """Pack an HF model's projections on the GPU (models/decoder.py:640-698).

    The packer is the bit-exact gfx950 quantizer (symmetric int4, or int8 with
    ``bits=8`` as models/decoder.py:651 picks pack_weight_int8; bf16 scales);
    the q/k/v projections are concatenated into one packed weight, the embedding
    and norms stay bf16, and any bias besides q/k/v is refused.
    """

    device = _device()
    dtype = next(model.parameters()).dtype
    if dtype != BF16:
        raise UnsupportedDTypeError(
            f"the {TARGET} W4 path computes in bf16; the model is {dtype}",
            hint="load the checkpoint with torch_dtype=torch.bfloat16",
        )

    def dev(t: torch.Tensor) -> torch.Tensor:
        return t.detach().to(device=device, dtype=BF16).contiguous()

    layers = []
    for index, layer in enumerate(model.model.layers):
        attention, mlp = layer.self_attn, layer.mlp
        for owner, name in ((attention, "o_proj"), (mlp, "gate_proj"), (mlp, "up_proj"), (mlp, "down_proj")):
            if getattr(owner, name).bias is not None:
                raise UnsupportedModelError(
                    f"packed compilation cannot pack the {name} bias of layer {index}",
                    hint="the quantized plan holds only the packed q/k/v bias",
                )
        qkv = torch.cat((attention.q_proj.weight, attention.k_proj.weight, attention.v_proj.weight), dim=0)
        bias = None
        if spec.qkv_bias:
            bias = dev(torch.cat((attention.q_proj.bias, attention.k_proj.bias, attention.v_proj.bias), dim=0))
        layers.append(
            LayerState(
                qkv=_pack(qkv, group, device, bits),
                o=_pack(attention.o_proj.weight, group, device, bits),
                gate=_pack(mlp.gate_proj.weight, group, device, bits),
                up=_pack(mlp.up_proj.weight, group, device, bits),
                down=_pack(mlp.down_proj.weight, group, device, bits),
                input_norm=dev(layer.input_layernorm.weight),
                post_norm=dev(layer.post_attention_layernorm.weight),
                qkv_bias=bias,
            )
        )
    head = getattr(model, "lm_head", None)
    if head is not None and getattr(head, "bias", None) is not None:
        raise UnsupportedModelError("packed compilation cannot pack an lm_head bias")
    return DecoderState(
        embed=dev(model.model.embed_tokens.weight),
        final_norm=dev(model.model.norm.weight),
        lm_head=_pack(model.lm_head.weight, group, device, bits),
        layers=layers,
    )


def random_state(spec: DecoderSpec, group: int = 64, *, seed: int = 0, std: float = 0.02,
                 norm_std: float = 0.0, bits: int = 4) -> DecoderState:
    """A seeded random-init state built directly on the GPU, one tensor at a time.

    Weights and biases ~ N(0, std) in bf16 (q/k/v biases seeded, unlike HF's
    zero init), norms 1 + N(0, norm_std). No fp32 model is ever materialized, so
    an 8B-shape state needs only its packed size plus one bf16 projection.
    """

    device = _device()
    generator = torch.Generator(device=device)
    generator.manual_seed(seed)

    def normal(*shape, scale=std):
        return (torch.randn(*shape, generator=generator, device=device, dtype=torch.float32) * scale).to(BF16)

    def norm(n):
        if norm_std == 0.0:
            return torch.ones(n, device=device, dtype=BF16)
        return (1.0 + torch.randn(n, generator=generator, device=device) * norm_std).to(BF16)

    def packed(n, k):
        w = normal(n, k)
        out = _pack(w, group, device, bits)
        del w
        return out

    h, i = spec.hidden, spec.intermediate
    layers = []
    for _ in range(spec.layers):
        layers.append(
            LayerState(
                qkv=packed(spec.qkv_width, h),
                o=packed(h, spec.attention_width),
                gate=packed(i, h),
                up=packed(i, h),
                down=packed(h, i),
                input_norm=norm(h),
                post_norm=norm(h),
                qkv_bias=normal(spec.qkv_width) if spec.qkv_bias else None,
            )
        )
    embed = normal(spec.vocab, h)
    lm_head = _pack(embed, group, device, bits) if spec.tied else packed(spec.vocab, h)
    return DecoderState(embed=embed, final_norm=norm(h), lm_head=lm_head, layers=layers)


# ----------------------------------------------------------------------------- tables
def rope_tables(capacity: int, head_dim: int, theta: float, device) -> tuple[torch.Tensor, torch.Tensor]:
    """bf16 cos/sin tables [capacity, head_dim], built as the reference builds them.

    models/decoder.py:323-334: the angle ``pos / theta^(2i/D)`` is formed in
    f32 by torch on the host, duplicated over the two halves, cast to the model
    dtype (bf16) *before* ``cos``/``sin``, and the bf16 results are the tables.
    The same torch CPU ops are used here so the tables match bit for bit; they
    are built once per plan and uploaded.
    """

    frequencies = torch.arange(capacity, dtype=torch.float32)[:, None] / torch.pow(
        torch.tensor(theta, dtype=torch.float32),
        torch.arange(0, head_dim, 2, dtype=torch.float32)[None, :] / head_dim,
    )
    frequencies = torch.cat((frequencies, frequencies), dim=-1).to(BF16)
    return frequencies.cos().to(device).contiguous(), frequencies.sin().to(device).contiguous()


def prefill_mask(length: int, bucket: int) -> np.ndarray:
    """``[1, 1, bucket, bucket]`` keep-mask, causal and not a left pad (models/decoder.py:226-247)."""

    if bucket <= 0 or length <= 0:
        raise PlanInputError(f"need 0 < length <= bucket, got length={length}, bucket={bucket}")
    if length > bucket:
        raise BucketRangeError(f"a {length}-token prompt does not fit a {bucket}-token bucket")
    query = np.arange(bucket)[:, None]
    key = np.arange(bucket)[None, :]
    return ((key <= query) & (key >= bucket - length))[None, None]


# ----------------------------------------------------------------------------- selections
def _sel(index: int, op: str, output: str, kind: str, reason: str, artifact: str) -> KernelSelection:
    name = None
    if torch.cuda.is_available():
        try:
            name = torch.cuda.get_device_name()
        except Exception:  # noqa: BLE001 - the name is informational
            name = None
    return KernelSelection(
        op_index=index,
        op=op,
        output_id=output,
        implementation="hip_kernel",
        kind=kind,
        reason=reason,
        artifact_name=artifact,
        device_name=name,
        device_architecture=ARCHITECTURE,
    )


def kernel_refusals(spec: DecoderSpec, group: int) -> tuple[KernelSelection, ...]:
    """Per-node refusals of a decoder shape outside the kernels' limits.

    The reference refuses an unsupported shape per node at candidate time and
    records the reason in that node's selection (``backends/apple.py:719-740``).
    This target has no fallback to send such a node to, so each refused node gets a
    ``KernelSelection`` with implementation ``"unsupported"`` and the reason; a
    non-empty result stops the compile (:func:`_check_kernel_limits`).
    """

    out: list[KernelSelection] = []

    def refuse(op: str, output: str, kind: str, reason: str) -> None:
        out.append(KernelSelection(op_index=len(out), op=op, output_id=output, implementation="unsupported",
                                   kind=kind, reason=reason, device_architecture=ARCHITECTURE))

    layers = range(spec.layers)
    attention = []
    if spec.head_dim not in (64, 128):
        attention.append(f"head_dim {spec.head_dim}: the decode and flash attention kernels take 64 or 128")
    if spec.heads % spec.kv_heads:
        attention.append(f"{spec.heads} query heads are not a multiple of {spec.kv_heads} kv heads")
    for reason in attention:
        for layer in layers:
            refuse("attention", f"attention_{layer}", "attention", reason)

    # (node, output features N, reduction K) of every packed projection
    projections = [("qkv", spec.qkv_width, spec.hidden), ("hidden_{}a", spec.hidden, spec.attention_width),
                   ("mlp", spec.intermediate, spec.hidden), ("hidden_{}b", spec.hidden, spec.intermediate)]
    for node, n, k in projections:
        reasons = []
        if k % 64:
            reasons.append(f"reduction length {k} is not a multiple of 64")
        if n % 16:
            reasons.append(f"{n} output features are not a multiple of 16")
        if group % 32 or k % group:
            reasons.append(f"group size {group} is not a multiple of 32 dividing the reduction length {k}")
        for reason in reasons:
            for layer in layers:
                output = node.format(layer) if "{}" in node else f"{node}_{layer}"
                refuse("matmul", output, "packed_matmul", reason)
    if group % 32 or spec.hidden % group:
        refuse("matmul", "logits", "packed_matmul",
               f"group size {group} is not a multiple of 32 dividing the hidden size {spec.hidden}")
    return tuple(out)


def _check_kernel_limits(spec: DecoderSpec, group: int) -> None:
    refused = kernel_refusals(spec, group)
    if refused:
        reasons = sorted({s.reason for s in refused})
        error = CompilationError(
            f"{TARGET} cannot compile this decoder: {len(refused)} node(s) refused: " + "; ".join(reasons),
            hint="every node must run as a gfx950 kernel; there is no fallback (the error's `refused` "
                 "attribute holds each node's selection record)",
        )
        error.refused = refused
        raise error


def _prefill_pairs_gate_up(tokens: int, spec: DecoderSpec) -> bool:
    """Whether a prefill of ``tokens`` rows runs the MLP's gate and up projections as
    one paired GEMM (one pass over x, one launch) instead of the reference's two.

    Paired at every length, measured on MI355X: the Qwen2-0.5B 128-token prefill
    (58.5k -> 69.6k tok/s when introduced) and the Llama-3-8B 512 / 2048-token
    buckets (37.6k / 41.2k tok/s paired against 36.7k / 40.2k with two GEMMs).
    ``AOTOLITH_PREFILL_GATE_UP=0`` keeps the two GEMMs.
    """

    if os.environ.get("AOTOLITH_PREFILL_GATE_UP", "1") == "0":
        return False
    return tokens > 0


def _prefill_fuses_norms(spec: DecoderSpec) -> bool:
    """Whether the prefill runs each RMSNorm after a residual projection (o, and
    the previous layer's down) through :func:`ops.matmul_residual_norm`: rows up
    to 4096 wide, a multiple of 8."""

    return spec.hidden % 8 == 0 and spec.hidden <= 4096


class _LaunchRecorder:
    """Node-by-node record of the kernels one pass of a sequence launches.

    ``node(...)`` opens a node; the kernel symbols the C ABI reports launched
    until the next node (``ops.take_launches``) are that node's. Each launched
    kernel becomes one ``KernelSelection`` whose ``artifact_name`` is the exact
    symbol (the reference's selection names the kernel the node emitted,
    ``selection.py:19-34``); a node that launches two kernels (a split-K GEMM and
    its sum) gives two records, the second with output id ``<node>.1``.
    """

    def __init__(self, take) -> None:
        self._take = take
        self._open: tuple[str, str, str, str] | None = None
        self.nodes: list[tuple[str, str, str, str, list[str]]] = []
        take()  # drop anything recorded before the first node

    def node(self, op: str, output: str, kind: str, reason: str) -> None:
        self._close()
        self._open = (op, output, kind, reason)

    def _close(self) -> None:
        names = self._take()
        if self._open is not None:
            self.nodes.append((*self._open, names))
        elif names:
            raise CompilationError(f"kernels launched outside a plan node: {names}")
        self._open = None

    def selections(self) -> tuple[KernelSelection, ...]:
        self._close()
        out: list[KernelSelection] = []
        for op, output, kind, reason, names in self.nodes:
            if not names:
                raise CompilationError(f"plan node {output} ({op}) launched no kernel")
            for index, name in enumerate(names):
                out.append(_sel(len(out), op, output if index == 0 else f"{output}.{index}", kind, reason, name))
        return tuple(out)


def _mark(rec: _LaunchRecorder | None, op: str, output: str, kind: str, reason: str) -> None:
    if rec is not None:
        rec.node(op, output, kind, reason)


# ----------------------------------------------------------------------------- engine
@contextlib.contextmanager
def _graph_capture(graph, pool=None):
    """``torch.cuda.graph`` with the Python GC run first and held off until the end.

    A dead reference cycle that owns another captured graph, collected while a
    capture is underway, destroys that graph mid-capture and aborts the
    process; torch's capture context no longer collects on entry.
    """

    gc.collect()
    enabled = gc.isenabled()
    gc.disable()
    try:
        with torch.cuda.graph(graph, pool=pool):
            yield
    finally:
        if enabled:
            gc.enable()


# ----------------------------------------------------------------------------- engine
@dataclass
class _Engine:
    """Kernel sequences of one bucket over one shared state."""

    spec: DecoderSpec
    state: DecoderState
    prompt_length: int
    capacity: int
    device: torch.device
    attention_splits: int = 0
    cos: torch.Tensor = field(init=False)
    sin: torch.Tensor = field(init=False)

    def __post_init__(self) -> None:
        s = self.spec
        dev = self.device
        self.cos, self.sin = rope_tables(self.capacity, s.head_dim, s.theta, dev)
        self.scale = float(np.float32(s.head_dim ** -0.5))
        # decode buffers
        self.hidden = torch.empty(s.hidden, dtype=BF16, device=dev)
        self.qkv = torch.empty(s.qkv_width, dtype=BF16, device=dev)
        self.q = torch.empty((1, s.heads, s.head_dim), dtype=BF16, device=dev)
        self.attn = torch.empty((1, s.heads, s.head_dim), dtype=BF16, device=dev)
        self.act = torch.empty(s.intermediate, dtype=BF16, device=dev)
        self.logits = torch.empty((1, 1, s.vocab), dtype=BF16, device=dev)
        self.token = torch.zeros((1,), dtype=torch.int64, device=dev)
        self.step_state = torch.zeros((4,), dtype=torch.int32, device=dev)
        self.workspace = ops.decode_attention_workspace(
            1, s.heads, s.kv_heads, self.capacity, s.head_dim, self.attention_splits, device=dev
        )
        self.ring = torch.zeros((s.layers, 2, 1, s.kv_heads, self.capacity, s.head_dim), dtype=BF16, device=dev)
        self.history = torch.zeros((self.capacity + 1,), dtype=torch.int64, device=dev)
        self.history_len = torch.zeros((1,), dtype=torch.int32, device=dev)
        # Greedy loop tail: the LM-head GEMV writes per-wave argmax keys and one
        # finish kernel turns them into the token, its history entry, the next
        # step state and the next step's embedding row (2 launches instead of
        # GEMV + argmax + step advance + embedding), when the LM-head shape has
        # the fused form.
        head = self.state.lm_head
        self.key_count = (ops.argmax_key_count(s.hidden, head.packed.shape[0], head.group)
                          if head.bits == 4 else 0)
        self.keys = (torch.empty((self.key_count,), dtype=torch.int64, device=dev) if self.key_count else None)
        # cos/sin rows of the current decode position, kept by the finish kernel,
        # so attention does not wait for the step state before its table loads
        self.rope_rows = torch.zeros((2, s.head_dim), dtype=BF16, device=dev)
        # The graph loop folds each step's finish into the next step's first
        # q/k/v GEMV (ops.w4_gemv_finish: one launch fewer per token) where that
        # GEMV's shape has the fused form; the last token's finish runs alone.
        qkv0 = self.state.layers[0].qkv if self.state.layers else None
        self.fold_finish = bool(
            self.keys is not None and qkv0 is not None and qkv0.bits == 4
            and tuple(self.state.embed.shape[1:]) == (s.hidden,)
            and ops.gemv_finish_supported(s.hidden, qkv0.packed.shape[0], qkv0.group, self.key_count)
            and os.environ.get("AOTOLITH_FOLD_FINISH", "1") != "0"
        )
        # ring prefill inputs (captured prefill graphs read these) and the graphs,
        # one per left-pad width (the attention's key start), sharing one pool
        self.prefill_ids = torch.zeros((1, self.prompt_length), dtype=torch.int64, device=dev)
        self.prefill_positions = torch.zeros((1, self.prompt_length), dtype=torch.int64, device=dev)
        self._prefill_graphs: dict[int, tuple] = {}
        self._prefill_pool = None
        self.prefill_graph_error: str | None = None
        self._graph = None
        self._graphs: dict[int, object] = {}
        self._first_graph = None
        self.graph_error: str | None = None

    #: longest run of decode steps captured in one graph (AOTOLITH_GRAPH_STEPS
    #: overrides). Measured on MI355X, one-step graphs replayed back to back beat
    #: 4- and 32-step graphs by ~25 us per token, so 1 is the default.
    MAX_GRAPH_STEPS = 1

    # -- decode -----------------------------------------------------------------
    def _gemv(self, x, w: PackedWeight, out, **kwargs):
        gemv = ops.w4_gemv if w.bits == 4 else ops.w8_gemv
        return gemv(x, w.packed, w.scales, w.group, out=out, **kwargs)

    @staticmethod
    def _matmul(x, w: PackedWeight, **kwargs):
        matmul = ops.w4_matmul if w.bits == 4 else ops.w8_matmul
        return matmul(x, w.packed, w.scales, w.group, **kwargs)

    def _decode_layers(self, cache_in, cache_out, *, valid=None, ring: bool, lm_head: bool = True, rec=None,
                       finish: bool = False):
        """Run the per-layer decode kernels (and the LM head); ``hidden`` holds the embedded token.

        ``finish``: the previous step's argmax finish runs in layer 0's q/k/v GEMV
        (``ops.w4_gemv_finish``), which embeds the token into ``hidden`` itself.
        """

        s = self.spec
        qd, kd = s.heads * s.head_dim, s.kv_heads * s.head_dim
        bits = self.state.bits
        gemv = f"w{bits}_gemv"
        for index, layer in enumerate(self.state.layers):
            if finish and index == 0:
                _mark(rec, "addmm", f"qkv_{index}", gemv,
                      "the previous step's argmax finish (token, history, step state, RoPE rows, embedding) in "
                      "the prologue of the packed W4 GEMV (M=1) with RMSNorm prologue"
                      + (" and q/k/v bias epilogue" if s.qkv_bias else ""))
                ops.w4_gemv_finish(self.keys, self.key_count, self.state.embed, layer.qkv.packed, layer.qkv.scales,
                                   layer.qkv.group, norm_weight=layer.input_norm, eps=s.eps, bias=layer.qkv_bias,
                                   out=self.qkv, token_out=self.token, hidden_out=self.hidden,
                                   history=self.history, history_len=self.history_len, step_state=self.step_state,
                                   capacity=self.capacity, rope_tables=(self.cos, self.sin), rope_rows=self.rope_rows)
            else:
                _mark(rec, "addmm", f"qkv_{index}", gemv,
                      f"packed W{bits} GEMV (M=1) with RMSNorm prologue"
                      + (" and q/k/v bias epilogue" if s.qkv_bias else ""))
                self._gemv(self.hidden, layer.qkv, self.qkv, norm_weight=layer.input_norm, eps=s.eps,
                           bias=layer.qkv_bias)
            pair_out = cache_out[index]
            if ring:
                _mark(rec, "attention", f"attention_{index}", "decode_attention",
                      "ring step: RoPE of q/k, in-place KV write at the step's slot and single-query GQA attention "
                      "(long windows split, then merged)")
                ops.decode_rope_attention(self.qkv.view(1, -1), self.cos, self.sin, pair_out, query_heads=s.heads,
                                          query_start=0, key_start=qd, value_start=qd + kd,
                                          step_state=self.step_state, scale=self.scale, workspace=self.workspace,
                                          splits=self.attention_splits,
                                          rope_rows=self.rope_rows if self.keys is not None else None,
                                          out=self.attn)
            else:
                position = valid - 1
                _mark(rec, "rope_kv_cache_append", f"query_{index}", "rope_kv_append",
                      "rotates q/k and appends (k, v) to the rolled cache window")
                ops.rope_kv_cache_append(self.qkv.view(1, -1), self.cos, self.sin, position, pair_out,
                                         pair_in=cache_in[index], query_heads=s.heads, query_start=0,
                                         key_start=qd, value_start=qd + kd, q_out=self.q)
                _mark(rec, "attention", f"attention_{index}", "decode_attention",
                      f"single-query GQA ({s.heads // s.kv_heads} query heads per kv head) over the last "
                      f"{valid} slots (long windows split, then merged)")
                ops.decode_attention(self.q, pair_out[0], pair_out[1], valid=valid, scale=self.scale,
                                     workspace=self.workspace, splits=self.attention_splits, out=self.attn)
            _mark(rec, "addmm", f"hidden_{index}a", gemv, f"packed W{bits} GEMV with residual epilogue")
            self._gemv(self.attn.view(-1), layer.o, self.hidden, bias=self.hidden)
            _mark(rec, "matmul", f"mlp_{index}", gemv,
                  f"paired gate/up W{bits} GEMV with RMSNorm prologue and silu_mul_paired epilogue")
            self._gemv(self.hidden, layer.gate, self.act, norm_weight=layer.post_norm, eps=s.eps,
                       up=(layer.up.packed, layer.up.scales))
            _mark(rec, "addmm", f"hidden_{index}b", gemv, f"packed W{bits} GEMV with residual epilogue")
            self._gemv(self.act, layer.down, self.hidden, bias=self.hidden)
        if lm_head:
            _mark(rec, "matmul", "logits", gemv, f"LM-head W{bits} GEMV with final RMSNorm prologue")
            self._gemv(self.hidden, self.state.lm_head, self.logits.view(-1), norm_weight=self.state.final_norm,
                       eps=s.eps)

    def decode_functional(self, token: torch.Tensor, cache: torch.Tensor, valid: int, rec=None):
        """The reference decode plan: fresh logits and the rolled next cache."""

        _mark(rec, "embedding", "hidden_0", "gather", "bf16 embedding row gather by device token")
        ops.embedding(self.state.embed, token.reshape(-1)[:1], out=self.hidden.view(1, -1))
        next_cache = torch.empty_like(cache)
        self._decode_layers(cache, next_cache, valid=valid, ring=False, rec=rec)
        return self.logits.clone(), next_cache

    def _ring_step(self, rec=None) -> None:
        """One captured-loop step: token -> logits -> token, cache/step state advanced on device.

        With the fused tail ``hidden`` must hold the token's embedding on entry
        (``_enter_loop``), and holds the next token's on exit; ``rope_rows`` likewise.
        """

        if self.keys is None:
            _mark(rec, "embedding", "hidden_0", "gather", "bf16 embedding row gather by device token")
            ops.embedding(self.state.embed, self.token, out=self.hidden.view(1, -1))
            self._decode_layers(None, self.ring, ring=True, rec=rec)
            _mark(rec, "argmax", "token", "argmax", "first-index greedy argmax, appended to the token history")
            ops.argmax(self.logits.view(1, -1), out=self.token, history=self.history,
                       history_len=self.history_len)
            _mark(rec, "step_advance", "step_state", "step_state", "advances {position, valid, ring offset, slot}")
            ops.step_advance(self.step_state, self.capacity)
            return
        head = self.state.lm_head
        self._decode_layers(None, self.ring, ring=True, lm_head=False, rec=rec)
        _mark(rec, "matmul", "logits", "w4_gemv",
              "LM-head W4 GEMV with final RMSNorm prologue, writing per-wave greedy-argmax keys")
        ops.w4_gemv_argmax(self.hidden, head.packed, head.scales, head.group, self.keys,
                           norm_weight=self.state.final_norm, eps=self.spec.eps, out=self.logits.view(-1))
        _mark(rec, "argmax", "token", "argmax",
              "reduces the argmax keys to the token; appends it to the history, advances the step state, "
              "copies the next position's RoPE rows and gathers the next token's embedding")
        ops.argmax_finish(self.keys, self.key_count, out=self.token, history=self.history,
                          history_len=self.history_len, step_state=self.step_state, capacity=self.capacity,
                          embedding=self.state.embed, hidden_out=self.hidden, rope_tables=(self.cos, self.sin),
                          rope_rows=self.rope_rows)

    def _ring_step_folded(self, first: bool, rec=None) -> None:
        """One step of the folded graph loop: [finish of the previous keys + layer-0 q/k/v, ..., LM-head keys].

        ``first``: the loop's first step, whose token ``_enter_loop`` embedded, runs
        the plain q/k/v GEMV. After the last step ``_finish_keys`` turns the keys
        into the final token.
        """

        head = self.state.lm_head
        self._decode_layers(None, self.ring, ring=True, lm_head=False, rec=rec, finish=not first)
        _mark(rec, "matmul", "logits", "w4_gemv",
              "LM-head W4 GEMV with final RMSNorm prologue, writing per-wave greedy-argmax keys")
        ops.w4_gemv_argmax(self.hidden, head.packed, head.scales, head.group, self.keys,
                           norm_weight=self.state.final_norm, eps=self.spec.eps, out=self.logits.view(-1))

    def _finish_keys(self, rec=None) -> None:
        """The standalone argmax finish of the last LM-head keys (the folded loop's last token)."""

        _mark(rec, "argmax", "token", "argmax",
              "reduces the last step's argmax keys to the token; appends it to the history, advances the step "
              "state, copies the next position's RoPE rows and gathers the next token's embedding")
        ops.argmax_finish(self.keys, self.key_count, out=self.token, history=self.history,
                          history_len=self.history_len, step_state=self.step_state, capacity=self.capacity,
                          embedding=self.state.embed, hidden_out=self.hidden, rope_tables=(self.cos, self.sin),
                          rope_rows=self.rope_rows)

    def _enter_loop(self, position: int) -> None:
        """The loop's entry condition: the RoPE rows of ``position`` and (fused tail) ``token``'s embedding."""

        self.rope_rows[0].copy_(self.cos[position])
        self.rope_rows[1].copy_(self.sin[position])
        if self.keys is not None:
            ops.embedding(self.state.embed, self.token, out=self.hidden.view(1, -1))

    def _ensure_graph(self) -> None:
        if self._graph is not None or self.graph_error is not None:
            return
        if os.environ.get("AOTOLITH_HIP_GRAPH", "1") == "0":
            self.graph_error = "disabled by AOTOLITH_HIP_GRAPH=0"
            return
        # Warm up once on dummy state (kernel lookup happens on first launch),
        # then restore the buffers a real loop initializes anyway.
        self.token.zero_()
        self.step_state.copy_(torch.tensor([0, 1, 1 % self.capacity, 0], dtype=torch.int32))
        self.history_len.zero_()
        self._enter_loop(0)
        self._ring_step()
        if self.fold_finish:
            self._ring_step_folded(first=True)
            self._ring_step_folded(first=False)
            self._finish_keys()
        torch.cuda.synchronize()
        try:
            # Graphs of 1, 2, 4, ... consecutive steps: a loop of n steps replays
            # the binary decomposition of n, so back-to-back graph launches
            # (each with its own launch cost) are few. With the folded finish the
            # loop's first step has a graph of its own (plain q/k/v GEMV) and the
            # others fold the previous step's finish into theirs.
            longest = int(os.environ.get("AOTOLITH_GRAPH_STEPS", self.MAX_GRAPH_STEPS))
            limit = min(max(1, longest), max(1, self.capacity - self.prompt_length - 1))
            step = (lambda: self._ring_step_folded(first=False)) if self.fold_finish else self._ring_step
            graphs = {}
            size = 1
            while size <= limit:
                graph = torch.cuda.CUDAGraph()
                with _graph_capture(graph):
                    for _ in range(size):
                        step()
                _lib.hold_graph(graph)
                graphs[size] = graph
                size *= 2
            if self.fold_finish:
                graph = torch.cuda.CUDAGraph()
                with _graph_capture(graph):
                    self._ring_step_folded(first=True)
                _lib.hold_graph(graph)
                self._first_graph = graph
            self._graphs = graphs
            self._graph = graphs[1]
        except Exception as error:  # noqa: BLE001 - fall back to eager replay, recorded
            self.graph_error = f"{type(error).__name__}: {error}"
            self._graph = None
            self._graphs = {}
            self._first_graph = None
        torch.cuda.synchronize()

    def ring_loop(self, steps: int, start_valid: int, first_token: torch.Tensor, *, sync_each_step: bool,
                  use_graph: bool = True) -> torch.Tensor:
        """``steps`` device-driven decode steps after a prefill that filled ``self.ring``."""

        if use_graph:
            self._ensure_graph()
        self.token.copy_(first_token.reshape(-1)[:1])
        # state = {position, valid, ring_offset, slot} of the first decode step
        self.step_state.copy_(
            torch.tensor([start_valid, start_valid + 1, 1 % self.capacity, 0], dtype=torch.int32)
        )
        self._enter_loop(start_valid)
        graphs = use_graph and bool(self._graphs)
        remaining = steps
        if self.fold_finish and remaining > 0:
            # the loop's first step (its token embedded on entry), then the folded steps
            if graphs and self._first_graph is not None:
                self._first_graph.replay()
            else:
                self._ring_step_folded(first=True)
            remaining -= 1
            if sync_each_step:
                torch.cuda.synchronize()
        while remaining > 0:
            if graphs:
                size = 1
                if not sync_each_step:
                    while size * 2 in self._graphs and size * 2 <= remaining:
                        size *= 2
                self._graphs[size].replay()
            else:
                size = 1
                if self.fold_finish:
                    self._ring_step_folded(first=False)
                else:
                    self._ring_step()
            remaining -= size
            if sync_each_step:
                torch.cuda.synchronize()
        if self.fold_finish and steps > 0:
            self._finish_keys()  # the last step's token
            if sync_each_step:
                torch.cuda.synchronize()
        return self.history

    # -- prefill ----------------------------------------------------------------
    #: captured ring-prefill graphs kept per engine (one per left-pad width)
    MAX_PREFILL_GRAPHS = 8

    def _ring_prefill_body(self, key_start: int) -> torch.Tensor:
        """Prefill of ``prefill_ids`` into the ring, then the first greedy token (token, history[0])."""

        slot0 = self.capacity - self.prompt_length
        logits = self.prefill_into(self.prefill_ids, self.prefill_positions, lambda i: self.ring[i], slot0,
                                   self.capacity, key_start=key_start)
        self.history_len.zero_()
        ops.argmax(logits.view(1, -1), out=self.token, history=self.history, history_len=self.history_len)
        return logits

    def _prefill_graphs_enabled(self, use_graph: bool) -> bool:
        return (use_graph and self.prefill_graph_error is None
                and os.environ.get("AOTOLITH_HIP_GRAPH", "1") != "0"
                and os.environ.get("AOTOLITH_PREFILL_GRAPH", "1") != "0")

    def ensure_prefill_graph(self, key_start: int, *, use_graph: bool = True) -> None:
        """Capture the ring prefill of one left-pad width (an eager warm-up pass first).

        The warm-up and the capture use whatever ``prefill_ids`` holds and
        overwrite the ring cache and token history; a caller fills both anew.
        """

        if not self._prefill_graphs_enabled(use_graph) or key_start in self._prefill_graphs:
            return
        if len(self._prefill_graphs) >= self.MAX_PREFILL_GRAPHS:
            self._prefill_graphs.pop(next(iter(self._prefill_graphs)))
        self._ring_prefill_body(key_start)
        torch.cuda.synchronize()
        try:
            if self._prefill_pool is None:
                self._prefill_pool = torch.cuda.graph_pool_handle()
            graph = torch.cuda.CUDAGraph()
            with _graph_capture(graph, pool=self._prefill_pool):
                captured = self._ring_prefill_body(key_start)
            _lib.hold_graph(graph)
            self._prefill_graphs[key_start] = (graph, captured)
        except Exception as error:  # noqa: BLE001 - eager prefill stays correct, recorded
            self.prefill_graph_error = f"{type(error).__name__}: {error}"
        torch.cuda.synchronize()

    def ring_prefill(self, ids: torch.Tensor, positions: torch.Tensor, key_start: int, *,
                     use_graph: bool = True) -> torch.Tensor:
        """Prefill ``ids`` (left-padded to the bucket) into the ring cache and pick the first token.

        With ``use_graph`` the kernel sequence of each left-pad width is captured
        once as a HIP graph (``ensure_prefill_graph``) and replayed, so a prefill
        costs device time only.
        """

        self.ensure_prefill_graph(key_start, use_graph=use_graph)
        self.prefill_ids.copy_(ids)
        self.prefill_positions.copy_(positions)
        entry = self._prefill_graphs.get(key_start) if self._prefill_graphs_enabled(use_graph) else None
        if entry is None:
            return self._ring_prefill_body(key_start)
        graph, logits = entry
        graph.replay()
        return logits

    def prefill_into(self, ids: torch.Tensor, positions: torch.Tensor, pair_of, slot0: int, window: int, *,
                     key_start: int, mask: torch.Tensor | None = None, rec=None) -> torch.Tensor:
        """Run the prefill kernels; layer ``i``'s keys/values go to ``pair_of(i)`` at ``slot0``.

        Returns logits ``[1, 1, V]`` of the last token.
        """

        s = self.spec
        m = ids.numel()
        dev = self.device
        bits = self.state.bits
        gemm = f"w{bits}_gemm"
        x = torch.empty((m, s.hidden), dtype=BF16, device=dev)
        xn = torch.empty_like(x)
        qkv = torch.empty((1, m, s.qkv_width), dtype=BF16, device=dev)
        q = torch.empty((1, s.heads, m, s.head_dim), dtype=BF16, device=dev)
        attn = torch.empty((1, m, s.attention_width), dtype=BF16, device=dev)
        act = torch.empty((m, s.intermediate), dtype=BF16, device=dev)
        paired = _prefill_pairs_gate_up(m, s)
        gate = None if paired else torch.empty_like(act)
        _mark(rec, "embedding", "hidden_0", "gather", "bf16 embedding row gather")
        ops.embedding(self.state.embed, ids.reshape(-1), out=x)
        layers = self.state.layers
        fuse = _prefill_fuses_norms(s)
        for index, layer in enumerate(layers):
            if index == 0 or not fuse:
                _mark(rec, "rms_norm", f"norm_{index}a", "rms_norm", "row RMSNorm")
                ops.rms_norm(x, layer.input_norm, s.eps, out=xn)
            pair = pair_of(index)
            _mark(rec, "addmm" if s.qkv_bias else "matmul", f"qkv_{index}", gemm,
                  (f"dequant-once W{bits} GEMM (packed tiles expanded once per 256-row block into LDS) on "
                   "32x32x16 bf16 MFMA"
                   if ops.lds_plan(m, s.qkv_width, s.hidden, group_size=layer.qkv.group, bits=bits, rope=True)
                   is not None
                   else f"wide-tile fused-dequant W{bits} GEMM on 32x32x16 bf16 MFMA"
                   if ops.wide_plan(m, s.qkv_width, s.hidden) is not None
                   else f"fused-dequant W{bits} GEMM on bf16 MFMA") + (" with q/k/v bias" if s.qkv_bias else "")
                  + ", RoPE of q/k and the layer's cache fill (with the split-K sum when the plan splits)")
            # q/k/v projection, RoPE and the cache fill (one launch fewer when the plan splits K)
            ops.matmul_qkv_rope(xn, layer.qkv.packed, layer.qkv.scales, layer.qkv.group, positions.reshape(-1),
                                self.cos, self.sin, pair, query_heads=s.heads, kv_heads=s.kv_heads,
                                head_dim=s.head_dim, slot0=slot0, bias=layer.qkv_bias, bits=layer.qkv.bits,
                                out=qkv.view(m, -1), q_out=q)
            keys = pair[0][:, :, slot0:slot0 + m]
            values = pair[1][:, :, slot0:slot0 + m]
            _mark(rec, "attention", f"attention_{index}", "flash_attention",
                  "masked GQA flash attention on MFMA" if mask is not None
                  else "causal + left-pad masked GQA flash attention on MFMA")
            if mask is not None:
                ops.prefill_attention(q, keys, values, mask=mask, scale=self.scale, out=attn)
            else:
                ops.prefill_attention(q, keys, values, causal=True, key_start=key_start, scale=self.scale, out=attn)
            if fuse:
                _mark(rec, "addmm", f"hidden_{index}a", gemm,
                      f"W{bits} GEMM with residual epilogue, then the next RMSNorm (one launch with the split-K sum "
                      "when the plan splits)")
                ops.matmul_residual_norm(attn.view(m, -1), layer.o.packed, layer.o.scales, layer.o.group, x,
                                         layer.post_norm, s.eps, bits=layer.o.bits, out=x, norm_out=xn)
            else:
                _mark(rec, "addmm", f"hidden_{index}a", gemm, f"W{bits} GEMM with residual epilogue")
                self._matmul(attn.view(m, -1), layer.o, residual=x, out=x)
                _mark(rec, "rms_norm", f"norm_{index}b", "rms_norm", "row RMSNorm")
                ops.rms_norm(x, layer.post_norm, s.eps, out=xn)
            if paired:
                _mark(rec, "matmul", f"mlp_{index}", gemm,
                      f"paired gate/up W{bits} GEMM (one pass over x) with silu_mul epilogue")
                gate_up = ops.w4_matmul_gate_up if layer.gate.bits == 4 else ops.w8_matmul_gate_up
                gate_up(xn, layer.gate.packed, layer.gate.scales, layer.up.packed, layer.up.scales,
                        layer.gate.group, out=act)
            else:
                _mark(rec, "matmul", f"gate_{index}", gemm, f"W{bits} GEMM")
                self._matmul(xn, layer.gate, out=gate)
                _mark(rec, "matmul", f"up_{index}", gemm, f"W{bits} GEMM with silu_mul epilogue")
                self._matmul(xn, layer.up, gate=gate, out=act)
            if fuse and index + 1 < len(layers):
                _mark(rec, "addmm", f"hidden_{index}b", gemm,
                      f"W{bits} GEMM with residual epilogue, then the next layer's input RMSNorm (one launch with "
                      "the split-K sum when the plan splits)")
                # the next layer's input norm with this projection's split-K sum
                ops.matmul_residual_norm(act, layer.down.packed, layer.down.scales, layer.down.group, x,
                                         layers[index + 1].input_norm, s.eps, bits=layer.down.bits, out=x,
                                         norm_out=xn)
            else:
                _mark(rec, "addmm", f"hidden_{index}b", gemm, f"W{bits} GEMM with residual epilogue")
                self._matmul(act, layer.down, residual=x, out=x)
        logits = torch.empty((1, 1, s.vocab), dtype=BF16, device=dev)
        _mark(rec, "matmul", "logits", f"w{bits}_gemv",
              f"LM-head W{bits} GEMV on the last row with final RMSNorm prologue")
        self._gemv(x[m - 1], self.state.lm_head, logits.view(-1), norm_weight=self.state.final_norm, eps=s.eps)
        return logits

    # -- selections ---------------------------------------------------------------
    def record_selections(self) -> dict[str, tuple[KernelSelection, ...]]:
        """The kernels each plan launches, node by node, from one real pass of each sequence.

        Run at compile time on placeholder inputs (the reference's selections are
        likewise made when the plan is built): the functional prefill of a zero
        prompt, one functional decode step, and the greedy loop's first-token
        argmax and one ring step. The loop's buffers are left for the first
        ``greedy_generate`` to initialize, as a warm-up pass does.
        """

        s = self.spec
        dev = self.device
        out = {}
        with ops.recording_launches() as take:
            ids = torch.zeros((1, self.prompt_length), dtype=torch.int64, device=dev)
            positions = torch.arange(self.prompt_length, dtype=torch.int64, device=dev)[None, :]
            compact = torch.empty((s.layers, 2, 1, s.kv_heads, self.prompt_length, s.head_dim), dtype=BF16,
                                  device=dev)
            rec = _LaunchRecorder(take)
            logits = self.prefill_into(ids, positions, lambda i: compact[i], 0, self.prompt_length, key_start=0,
                                       rec=rec)
            out["prefill"] = rec.selections()
            del compact
            rec = _LaunchRecorder(take)
            cache = torch.zeros((s.layers, 2, 1, s.kv_heads, self.capacity, s.head_dim), dtype=BF16, device=dev)
            valid = min(self.prompt_length + 1, self.capacity)
            self.decode_functional(torch.zeros((1,), dtype=torch.int64, device=dev), cache, valid, rec=rec)
            out["decode"] = rec.selections()
            del cache
            rec = _LaunchRecorder(take)
            self.history_len.zero_()
            _mark(rec, "argmax", "first_token", "argmax",
                  "first-index greedy argmax of the prefill logits, the first entry of the token history")
            ops.argmax(logits.view(1, -1), out=self.token, history=self.history, history_len=self.history_len)
            self.token.zero_()
            self.step_state.copy_(torch.tensor([0, 1, 1 % self.capacity, 0], dtype=torch.int32))
            if self.keys is not None:
                _mark(rec, "embedding", "hidden_0", "gather",
                      "the first token's embedding row, gathered once when the loop starts (each step's finish "
                      "gathers the next one)")
            if self.fold_finish:
                # the loop's first step runs the plain q/k/v GEMV (recorded below as
                # layer 1's); a token's step is the folded one, the last token's
                # finish runs alone
                self._enter_loop(0)
                self._ring_step_folded(first=True)
                self._ring_step_folded(first=False, rec=rec)
                self._finish_keys(rec=rec)
            else:
                self._enter_loop(0)
                self._ring_step(rec=rec)
            out["decode_loop"] = rec.selections()
        torch.cuda.synchronize()
        return out


# ----------------------------------------------------------------------------- runtime
@dataclass(frozen=True)
class DecoderMemoryFootprint:
    """Resident and per-step bytes of one bucket (models/decoder.py:745-780)."""

    weights_bytes: int
    cache_bytes: int
    scratch_bytes: int
    masks_bytes: int
    step_peak_bytes: int

    def describe(self) -> str:
        def mb(v):
            return f"{v / (1 << 20):.1f} MiB"

        return (f"weights {mb(self.weights_bytes)}, cache {mb(self.cache_bytes)}, masks {mb(self.masks_bytes)}, "
                f"scratch {mb(self.scratch_bytes)}, step peak {mb(self.step_peak_bytes)}")


def _as_ids(input_ids, device) -> torch.Tensor:
    if isinstance(input_ids, torch.Tensor):
        ids = input_ids.to(device=device, dtype=torch.int64)
    else:
        ids = torch.from_numpy(np.asarray(input_ids, dtype=np.int64)).to(device)
    if ids.dim() == 1:
        ids = ids[None, :]
    return ids.contiguous()


@dataclass(frozen=True)
class DecoderStaticCacheRuntime:
    """Executable prefill/decode plans of one bucket plus the host cache helpers."""

    prefill: CompiledPlan
    decode: CompiledPlan
    prompt_length: int
    max_new_tokens: int
    cache_capacity: int
    num_layers: int
    num_key_value_heads: int
    head_dim: int
    family: str
    memory: str
    spec: DecoderSpec
    engine: _Engine
    group_size: int
    quantize_bits: int = 4
    #: the greedy loop's plan (first-token argmax + one ring step), set at compile time
    decode_loop: CompiledPlan | None = None

    # -- reference API -----------------------------------------------------------
    def prefill_ids(self, input_ids):
        ids = _as_ids(input_ids, self.engine.device)
        if tuple(ids.shape) != (1, self.prompt_length):
            raise PlanInputError(f"expected prompt shape (1, {self.prompt_length}), got {tuple(ids.shape)}")
        positions = torch.arange(self.prompt_length, dtype=torch.int64, device=ids.device)[None, :]
        return self.prefill(ids, positions, None)

    def prefill_padded(self, input_ids):
        ids = _as_ids(input_ids, self.engine.device)
        if ids.shape[0] != 1:
            raise PlanInputError(f"expected batch size 1, got {ids.shape[0]}")
        length = int(ids.shape[1])
        if length < 1:
            raise PlanInputError(f"prompt length must be positive, got {length}")
        if length > self.prompt_length:
            raise BucketRangeError(f"a {length}-token prompt does not fit the {self.prompt_length}-token plan")
        if length == self.prompt_length:
            return self.prefill_ids(ids)
        padding = self.prompt_length - length
        zeros = torch.zeros((1, padding), dtype=torch.int64, device=ids.device)
        padded_ids = torch.cat((zeros, ids), dim=1)
        positions = torch.cat((zeros, torch.arange(length, dtype=torch.int64, device=ids.device)[None, :]), dim=1)
        return self.prefill(padded_ids, positions, length)

    def pad_cache(self, compact_cache: torch.Tensor) -> torch.Tensor:
        expected = (self.num_layers, 2, 1, self.num_key_value_heads, self.prompt_length, self.head_dim)
        if tuple(compact_cache.shape) != expected:
            raise PlanInputError(f"expected compact cache shape {expected}, got {tuple(compact_cache.shape)}")
        pad = torch.zeros(expected[:4] + (self.cache_capacity - self.prompt_length,) + expected[5:],
                          dtype=compact_cache.dtype, device=compact_cache.device)
        return torch.cat((pad, compact_cache), dim=4)

    def decode_mask(self, valid_length: int) -> torch.Tensor:
        if not 1 <= valid_length <= self.cache_capacity:
            raise PlanInputError(f"valid_length must be in [1, {self.cache_capacity}], got {valid_length}")
        window = torch.arange(self.cache_capacity) >= self.cache_capacity - valid_length
        return window.reshape(1, 1, 1, self.cache_capacity)

    def decode_token(self, token, cache: torch.Tensor, valid_length: int, *, verify_token: bool = True):
        """One decode step ``(logits [1,1,V], rolled cache)`` (models/decoder.py:889-932)."""

        if valid_length < 1 or valid_length >= self.cache_capacity:
            raise PlanInputError(f"valid_length must be in [1, {self.cache_capacity}), got {valid_length}")
        token = _as_ids(token, self.engine.device).reshape(-1)[:1]
        if verify_token:
            value = int(token.item())
            if not 0 <= value < self.spec.vocab:
                from .errors import IndexBoundsError

                raise IndexBoundsError(f"token {value} is outside the vocabulary [0, {self.spec.vocab})")
        return self.decode(token, cache, valid_length)

    def greedy_generate(self, input_ids, *, max_new_tokens: int | None = None, sync_each_step: bool = False,
                        use_graph: bool = True, events: dict | None = None) -> torch.Tensor:
        """Greedy tokens ``[1, steps]`` (models/decoder.py:934-951, 1054-1087).

        Prefill fills the ring cache in place; the first token is the argmax of
        its logits; the remaining ``steps - 1`` tokens come from device-driven
        decode steps (HIP graph replays unless ``use_graph`` is False).
        ``events``, when given, receives ``torch.cuda.Event`` marks recorded on
        the current stream at ``"start"``, ``"prefill"`` (first token ready) and
        ``"end"``.
        """

        steps = self.max_new_tokens if max_new_tokens is None else max_new_tokens
        if steps < 0 or steps > self.max_new_tokens:
            raise PlanInputError(f"max_new_tokens must be in [0, {self.max_new_tokens}], got {steps}")
        engine = self.engine
        if steps == 0:
            return torch.zeros((1, 0), dtype=torch.int64, device=engine.device)
        ids = _as_ids(input_ids, engine.device)
        if ids.shape[0] != 1:
            raise PlanInputError(f"expected batch size 1, got {ids.shape[0]}")
        length = int(ids.shape[1])
        if length > self.prompt_length:
            raise BucketRangeError(f"a {length}-token prompt does not fit the {self.prompt_length}-token plan")
        if use_graph:
            # Captures (and their warm-up passes on stale inputs) precede the
            # prefill: the warm-ups write the ring cache and the token history.
            engine.ensure_prefill_graph(self.prompt_length - length)
            engine._ensure_graph()
        marks = {}
        if events is not None:
            for key in ("start", "prefill", "end"):
                marks[key] = torch.cuda.Event(enable_timing=True)
            marks["start"].record()
        self._prefill_ring(ids, use_graph=use_graph)
        first = engine.token.clone()
        if events is not None:
            marks["prefill"].record()
        if sync_each_step:
            torch.cuda.synchronize()
        engine.ring_loop(steps - 1, length, first, sync_each_step=sync_each_step, use_graph=use_graph)
        tokens = engine.history[:steps].clone().view(1, steps)
        if events is not None:
            marks["end"].record()
            events.update(marks)
        return tokens

    def save(self, prefix):
        from .artifact import save_runtime

        return save_runtime(self, prefix)

    def memory_footprint(self) -> DecoderMemoryFootprint:
        s = self.spec
        cache = s.layers * 2 * s.kv_heads * self.cache_capacity * s.head_dim * 2
        m = self.prompt_length
        scratch = 2 * (m * s.hidden * 2 + m * s.qkv_width + s.heads * m * s.head_dim + m * s.attention_width
                       + 2 * m * s.intermediate) + s.vocab * 2
        masks = m * m + self.cache_capacity
        weights = self.engine.state.nbytes
        return DecoderMemoryFootprint(weights, cache, scratch, masks, weights + 2 * cache + masks + scratch)

    def check_memory_budget(self, budget_bytes: int) -> DecoderMemoryFootprint:
        footprint = self.memory_footprint()
        if footprint.step_peak_bytes > budget_bytes:
            raise MemoryBudgetError(
                f"one step needs {footprint.step_peak_bytes} bytes but the budget is {budget_bytes} "
                f"({footprint.describe()})",
                hint="shorten prompt_length + max_new_tokens or raise the budget",
            )
        return footprint

    # -- internals ---------------------------------------------------------------
    def _prefill_ring(self, ids: torch.Tensor, *, use_graph: bool = True) -> torch.Tensor:
        """Ring prefill of a left-padded prompt; the first token lands in ``engine.token``/``history``."""

        engine = self.engine
        length = int(ids.shape[1])
        padding = self.prompt_length - length
        if padding:
            zeros = torch.zeros((1, padding), dtype=torch.int64, device=ids.device)
            ids = torch.cat((zeros, ids), dim=1)
            positions = torch.cat((zeros, torch.arange(length, dtype=torch.int64, device=ids.device)[None, :]), 1)
        else:
            positions = torch.arange(length, dtype=torch.int64, device=ids.device)[None, :]
        return engine.ring_prefill(ids, positions, padding, use_graph=use_graph)


def _build_plans(spec: DecoderSpec, engine: _Engine, prompt_length: int):
    capacity = engine.capacity

    def run_prefill(ids, positions, mask_or_length=None):
        """(ids [1,P], positions [1,P], mask [1,1,P,P] | real length | None) -> (logits, compact cache)."""

        ids = _as_ids(ids, engine.device)
        if tuple(ids.shape) != (1, prompt_length):
            raise PlanInputError(f"expected ids of shape (1, {prompt_length}), got {tuple(ids.shape)}")
        positions = _as_ids(positions, engine.device)
        if int(positions.max()) >= capacity or int(positions.min()) < 0:
            raise PlanInputError(f"positions must lie in [0, {capacity})")
        compact = torch.empty((spec.layers, 2, 1, spec.kv_heads, prompt_length, spec.head_dim), dtype=BF16,
                              device=engine.device)
        mask = None
        key_start = 0
        if isinstance(mask_or_length, int):
            key_start = prompt_length - mask_or_length
        elif mask_or_length is not None:
            mask = torch.as_tensor(np.asarray(mask_or_length) if not isinstance(mask_or_length, torch.Tensor)
                                   else mask_or_length).to(device=engine.device, dtype=torch.bool)
            mask = mask.reshape(1, prompt_length, prompt_length)
        logits = engine.prefill_into(ids, positions, lambda i: compact[i], 0, prompt_length, key_start=key_start,
                                     mask=mask)
        return logits, compact

    def run_decode(token, cache, valid_length):
        expected = (spec.layers, 2, 1, spec.kv_heads, capacity, spec.head_dim)
        if tuple(cache.shape) != expected or cache.dtype != BF16 or cache.device.type != "cuda":
            raise PlanInputError(f"expected a bf16 device cache of shape {expected}, got {tuple(cache.shape)}")
        return engine.decode_functional(token, cache.contiguous(), int(valid_length))

    recorded = engine.record_selections()
    for name, selections in recorded.items():
        require_native(selections, f"{name} plan")
    prefill = CompiledPlan("prefill", tuple(PlanNode(s) for s in recorded["prefill"]), run_prefill,
                           input_names=("input_ids", "positions", "attention_mask"),
                           output_names=("logits", "cache"))
    decode = CompiledPlan("decode", tuple(PlanNode(s) for s in recorded["decode"]), run_decode,
                          input_names=("input_ids", "cache", "valid_length"), output_names=("logits", "cache"))
    return prefill, decode, recorded["decode_loop"]


def _check_target(target: str) -> None:
    if target != TARGET:
        raise CompilationError(
            f"unknown target {target!r} for this package",
            hint=f"this package implements {TARGET!r}; the reference's 'apple-metal' and 'mlx-reference' "
                 "targets run on Apple silicon",
        )


def compile_decoder_state(
    spec: DecoderSpec,
    state: DecoderState,
    *,
    prompt_length: int,
    max_new_tokens: int,
    group_size: int = 64,
    memory: str = "latency",
    attention_splits: int = 0,
) -> DecoderStaticCacheRuntime:
    """Compile one bucket over an already-packed device state (shared across buckets)."""

    if memory not in MEMORY_POLICIES:
        raise CompilationError(f"unknown memory policy {memory!r}", hint="choose one of: " + ", ".join(MEMORY_POLICIES))
    if prompt_length <= 0 or max_new_tokens < 0:
        raise CompilationError("prompt_length must be positive and max_new_tokens non-negative")
    capacity = prompt_length + max_new_tokens
    if capacity > spec.max_position:
        raise DynamicShapeError(
            f"prompt_length + max_new_tokens exceeds the model's maximum position embeddings ({spec.max_position})"
        )
    _check_kernel_limits(spec, group_size)
    bits = state.bits
    if any(w.group != group_size for w in state.weights):
        raise CompilationError(f"the state's packed weights are not all grouped by {group_size}")
    engine = _Engine(spec, state, prompt_length, capacity, _device(), attention_splits)
    prefill, decode, loop_selections = _build_plans(spec, engine, prompt_length)
    runtime = DecoderStaticCacheRuntime(
        prefill=prefill, decode=decode, prompt_length=prompt_length, max_new_tokens=max_new_tokens,
        cache_capacity=capacity, num_layers=spec.layers, num_key_value_heads=spec.kv_heads,
        head_dim=spec.head_dim, family=spec.family, memory=memory, spec=spec, engine=engine,
        group_size=group_size, quantize_bits=bits,
    )
    # The greedy loop's own plan: the first token's argmax over the prefill logits and
    # one device-driven ring step (replayed per token); its run is greedy_generate.
    loop = CompiledPlan("decode_loop", tuple(PlanNode(s) for s in loop_selections), runtime.greedy_generate,
                        input_names=("input_ids",), output_names=("tokens",))
    object.__setattr__(runtime, "decode_loop", loop)
    prefill.runtime = runtime
    decode.runtime = runtime
    loop.runtime = runtime
    return runtime


def _check_quantize(quantize: int | None, quantize_bits: int) -> int:
    """``quantize`` is the group size and ``quantize_bits`` the width (models/decoder.py:1406-1425)."""

    if quantize_bits not in (4, 8):
        raise CompilationError(f"quantize_bits must be 4 or 8, got {quantize_bits!r}",
                               hint="four bits packs eight codes a word, eight bits packs four")
    if quantize is None:
        raise CompilationError(
            f"the {TARGET} target compiles the weight-only packed path: pass quantize=<group size> (e.g. 64)",
            hint="dense bf16 projections are not part of this backend",
        )
    return int(quantize)


def compile_decoder_static_cache(
    model: torch.nn.Module,
    *,
    prompt_length: int,
    max_new_tokens: int,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
    quantize: int | None = None,
    quantize_bits: int = 4,
    family: str | None = None,
    target: str = TARGET,
    memory: str = "latency",
) -> DecoderStaticCacheRuntime:
    """Compile a supported causal LM for greedy single-request generation (models/decoder.py:1090-1146)."""

    _check_target(target)
    group = _check_quantize(quantize, quantize_bits)
    if getattr(model, "training", False):
        raise CompilationError("compile_decoder_static_cache requires model.eval()")
    spec = spec_from_model(model, require=family)
    if prompt_length + max_new_tokens > spec.max_position:
        raise DynamicShapeError(
            "prompt_length + max_new_tokens exceeds the model's maximum position embeddings "
            f"({spec.max_position})"
        )
    _check_kernel_limits(spec, group)
    state = pack_model_state(model, spec, group, quantize_bits)
    return compile_decoder_state(spec, state, prompt_length=prompt_length, max_new_tokens=max_new_tokens,
                                 group_size=group, memory=memory)


@dataclass(frozen=True)
class DecoderBucketedRuntime:
    """One runtime per prompt-length bucket over one shared state (models/decoder.py:1292-1400)."""

    buckets: tuple[DecoderStaticCacheRuntime, ...]
    max_new_tokens: int

    def __post_init__(self) -> None:
        if not self.buckets:
            raise CompilationError("at least one bucket is required")
        widths = [b.prompt_length for b in self.buckets]
        if widths != sorted(set(widths)):
            raise CompilationError(f"buckets must be strictly increasing, got {widths}")

    @property
    def prompt_lengths(self) -> tuple[int, ...]:
        return tuple(b.prompt_length for b in self.buckets)

    @property
    def family(self) -> str:
        return self.buckets[0].family

    @property
    def max_prompt_length(self) -> int:
        return self.buckets[-1].prompt_length

    def bucket_for(self, prompt_length: int) -> DecoderStaticCacheRuntime:
        for bucket in self.buckets:
            if prompt_length <= bucket.prompt_length:
                return bucket
        raise BucketRangeError(
            f"prompt length {prompt_length} exceeds the largest bucket ({self.max_prompt_length})"
        )

    def prefill_ids(self, input_ids):
        ids = _as_ids(input_ids, self.buckets[0].engine.device)
        if ids.shape[0] != 1:
            raise PlanInputError(f"expected batch size 1, got {ids.shape[0]}")
        bucket = self.bucket_for(int(ids.shape[1]))
        logits, compact = bucket.prefill_padded(ids)
        return logits, bucket.pad_cache(compact)

    def greedy_generate(self, input_ids, *, max_new_tokens: int | None = None, sync_each_step: bool = False,
                        use_graph: bool = True, events: dict | None = None) -> torch.Tensor:
        ids = _as_ids(input_ids, self.buckets[0].engine.device)
        bucket = self.bucket_for(int(ids.shape[1]))
        return bucket.greedy_generate(ids, max_new_tokens=max_new_tokens, sync_each_step=sync_each_step,
                                      use_graph=use_graph, events=events)

    def save(self, prefix):
        from .artifact import save_runtime

        paths = []
        for bucket in self.buckets:
            paths.extend(save_runtime(bucket, f"{prefix}.{bucket.prompt_length}"))
        return tuple(paths)


def compile_decoder_bucketed_state(
    spec: DecoderSpec,
    state: DecoderState,
    *,
    prompt_lengths: Sequence[int],
    max_new_tokens: int,
    group_size: int = 64,
) -> DecoderBucketedRuntime:
    widths = [int(w) for w in prompt_lengths]
    if not widths:
        raise CompilationError("prompt_lengths must name at least one bucket")
    if any(w <= 0 for w in widths):
        raise CompilationError(f"bucket widths must be positive, got {widths}")
    if widths != sorted(set(widths)):
        raise CompilationError(f"bucket widths must be strictly increasing, got {widths}")
    runtimes = tuple(
        compile_decoder_state(spec, state, prompt_length=w, max_new_tokens=max_new_tokens, group_size=group_size)
        for w in widths
    )
    return DecoderBucketedRuntime(buckets=runtimes, max_new_tokens=max_new_tokens)


def compile_decoder_bucketed(
    model: torch.nn.Module,
    *,
    prompt_lengths: Sequence[int],
    max_new_tokens: int,
    codegen_matmul: bool = False,
    codegen_attention: bool = False,
    autotune: bool = False,
    quantize: int | None = None,
    quantize_bits: int = 4,
    family: str | None = None,
    target: str = TARGET,
) -> DecoderBucketedRuntime:
    """One plan pair per bucket over one packed state (models/decoder.py:1413-1478)."""

    _check_target(target)
    group = _check_quantize(quantize, quantize_bits)
    spec = spec_from_model(model, require=family)
    _check_kernel_limits(spec, group)
    widths = [int(w) for w in prompt_lengths]
    if widths and widths[-1] + max_new_tokens > spec.max_position:
        raise DynamicShapeError("the largest bucket + max_new_tokens exceeds the maximum position embeddings")
    state = pack_model_state(model, spec, group, quantize_bits)
    return compile_decoder_bucketed_state(spec, state, prompt_lengths=widths, max_new_tokens=max_new_tokens,
                                          group_size=group)
