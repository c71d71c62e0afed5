"""Shared test helpers: seeded bf16 data, parity metrics, GPU gating."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.bf16 import from_bf16_bits, round_bf16, to_bf16_bits


def gpu_available() -> bool:
    return torch.cuda.is_available()


requires_gpu = pytest.mark.skipif(not gpu_available(), reason="needs an MI355X")


def bf16_normal(rng: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    """bf16-representable N(0, std) values as f32."""

    return round_bf16(rng.standard_normal(shape).astype(np.float32) * np.float32(std))


def to_gpu_bf16(values: np.ndarray) -> torch.Tensor:
    bits = to_bf16_bits(values)
    return torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).cuda()


def to_gpu_bits(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16).copy()).view(torch.bfloat16).cuda()


def from_gpu_bf16(tensor: torch.Tensor) -> np.ndarray:
    return from_bf16_bits(tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16))


def bf16_bits_of(tensor: torch.Tensor) -> np.ndarray:
    return tensor.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)


def parity(actual: np.ndarray, expected: np.ndarray) -> dict:
    a = np.asarray(actual, dtype=np.float64).reshape(-1)
    e = np.asarray(expected, dtype=np.float64).reshape(-1)
    diff = np.abs(a - e)
    denom = np.linalg.norm(a) * np.linalg.norm(e)
    cosine = float(a @ e / denom) if denom > 0 else (1.0 if np.all(a == e) else 0.0)
    # Distance in bf16 ulps (1 ulp = 2^-7 relative to the leading bit) of the larger
    # of the two values: an f32 sum that lands on the other side of a binade edge
    # rounds to a neighbour one ulp away in the wider binade. Values far below the
    # row's scale (cancellation) are measured against 2^-10 of the largest value,
    # where f32 accumulation noise, not the final rounding, sets the error.
    floor = max(float(np.abs(e).max()) * 2.0 ** -10 if e.size else 0.0, 2.0 ** -126)
    scale = np.maximum(np.maximum(np.abs(e), np.abs(a)), floor)
    ulp = 2.0 ** (np.floor(np.log2(scale)) - 7)
    return {
        "max_abs": float(diff.max()) if diff.size else 0.0,
        "cosine": cosine,
        "max_ulp": float((diff / ulp).max()) if diff.size else 0.0,
        "mismatch": int((diff > 0).sum()),
    }


def assert_bf16_parity(
    actual, expected, *, max_ulp: float | None = 1.0, atol: float = 2e-2, min_cos: float = 0.999
) -> dict:
    """North-star bars (max abs <= 2e-2, cosine >= 0.999) plus an ulp bound (None: no ulp bound)."""

    stats = parity(actual, expected)
    assert stats["max_abs"] <= atol, stats
    assert stats["cosine"] >= min_cos, stats
    if max_ulp is not None:
        assert stats["max_ulp"] <= max_ulp, stats
    return stats


def random_oracle_state(shape, seed: int = 0, *, std: float = 0.02, norm_std: float = 0.1, bias: bool = True) -> dict:
    """A seeded decoder state in the oracle's format (f32 arrays of bf16 values, packed W4).

    Norm weights are 1 + N(0, norm_std) and q/k/v biases N(0, std) so that a
    dropped or misplaced term changes the outputs (HF's init would zero them).
    """

    from oracle.quant import pack_weight_bits_bf16

    rng = np.random.default_rng(seed)
    g = shape.group_size
    bits = getattr(shape, "bits", 4)
    h, i, w = shape.hidden, shape.intermediate, shape.qkv_width
    hd = shape.heads * shape.head_dim

    def packed(n, k):
        return pack_weight_bits_bf16(bf16_normal(rng, (n, k), std), g, bits)

    def norm(n):
        return round_bf16(np.float32(1.0) + rng.standard_normal(n).astype(np.float32) * np.float32(norm_std))

    layers = []
    for _ in range(shape.layers):
        layers.append(
            {
                "qkv": packed(w, h),
                "o": packed(h, hd),
                "gate": packed(i, h),
                "up": packed(i, h),
                "down": packed(h, i),
                "qkv_bias": bf16_normal(rng, (w,), std) if bias else None,
                "input_norm": norm(h),
                "post_norm": norm(h),
            }
        )
    embed = bf16_normal(rng, (shape.vocab, h), std * 50)
    return {"embed": embed, "final_norm": norm(h), "lm_head": packed(shape.vocab, h), "layers": layers}


def state_to_device(ostate: dict, group: int, bits: int = 4):
    """Upload an oracle-format state as the runtime's device state (same bits)."""

    from aotolith_amd.decoder import DecoderState, LayerState, PackedWeight

    def pw(pair):
        return PackedWeight(torch.from_numpy(pair[0]).cuda(), to_gpu_bits(pair[1]), group, bits)

    layers = [
        LayerState(
            qkv=pw(l["qkv"]), o=pw(l["o"]), gate=pw(l["gate"]), up=pw(l["up"]), down=pw(l["down"]),
            input_norm=to_gpu_bf16(l["input_norm"]), post_norm=to_gpu_bf16(l["post_norm"]),
            qkv_bias=None if l["qkv_bias"] is None else to_gpu_bf16(l["qkv_bias"]),
        )
        for l in ostate["layers"]
    ]
    return DecoderState(embed=to_gpu_bf16(ostate["embed"]), final_norm=to_gpu_bf16(ostate["final_norm"]),
                        lm_head=pw(ostate["lm_head"]), layers=layers)


def runtime_spec(shape, family: str = "qwen2", bias: bool = True, max_position: int = 1 << 20):
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family=family, vocab=shape.vocab, hidden=shape.hidden, intermediate=shape.intermediate,
                       layers=shape.layers, heads=shape.heads, kv_heads=shape.kv_heads, head_dim=shape.head_dim,
                       eps=shape.eps, theta=shape.theta, qkv_bias=bias, max_position=max_position)


def first_divergence(tokens, reference, logits_history) -> dict | None:
    """None when the token streams agree, else the first differing step and the reference's top-2 margin."""

    tokens = np.asarray(tokens).reshape(-1)
    reference = np.asarray(reference).reshape(-1)
    for step, (a, b) in enumerate(zip(tokens, reference)):
        if a != b:
            logits = np.asarray(logits_history[step], dtype=np.float64).reshape(-1)
            top = np.sort(logits)[-2:]
            return {"step": step, "got": int(a), "want": int(b), "margin": float(top[1] - top[0]),
                    "got_logit": float(logits[a]), "want_logit": float(logits[b])}
    return None


def state_to_oracle(state) -> dict:
    """Download a runtime device state into the oracle's format (same bits)."""

    def bits(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    def f32(t):
        return t.detach().cpu().float().numpy()

    def pair(w):
        return (w.packed.cpu().numpy(), bits(w.scales))

    return {
        "embed": f32(state.embed),
        "final_norm": f32(state.final_norm),
        "lm_head": pair(state.lm_head),
        "layers": [
            {"qkv": pair(l.qkv), "o": pair(l.o), "gate": pair(l.gate), "up": pair(l.up), "down": pair(l.down),
             "qkv_bias": None if l.qkv_bias is None else f32(l.qkv_bias), "input_norm": f32(l.input_norm),
             "post_norm": f32(l.post_norm)}
            for l in state.layers
        ],
    }


def near_tie(divergence: dict, logits_history) -> bool:
    """Whether a token flip sits on a near-tie of the oracle's logits.

    The oracle's top two logits must be within two bf16 ulps of their magnitude
    (floored at 1/16 of the step's largest logit): there the order in which the
    GPU's f32 accumulators sum decides which of the two rounds higher.
    """

    scale = float(np.abs(np.asarray(logits_history[divergence["step"]], dtype=np.float64)).max())
    return divergence["margin"] <= 2 * 2.0 ** -7 * max(abs(divergence["want_logit"]), scale * 2.0 ** -4)


def teacher_forced_logits(runtime, prompt_ids, forced_tokens) -> tuple[list[np.ndarray], list[int]]:
    """GPU logits of every greedy step when the loop is fed ``forced_tokens`` instead of its own picks.

    The ring prefill, then the ring loop's step kernels launched eagerly one step
    at a time (the same kernels the captured graph replays); after each step the
    loop's next input token (and, with the fused argmax tail, the embedding row it
    gathered) is overwritten with the forced one. Returns the per-step logits and
    the GPU's own argmax at each step (the pattern of the reference's agreement
    check, ``examples/qwen_quantized_agreement.py``: teacher-forced after a flip).
    """

    from aotolith_amd import ops

    engine = runtime.engine
    ids = torch.as_tensor(np.asarray(prompt_ids, dtype=np.int64)).reshape(1, -1).cuda()
    length = int(ids.shape[1])
    assert length == runtime.prompt_length, "teacher forcing runs unpadded prompts"
    logits = runtime._prefill_ring(ids, use_graph=False)
    out = [from_gpu_bf16(logits).reshape(-1)]
    picks = [int(engine.token.item())]
    device = engine.token.device
    engine.token.fill_(int(forced_tokens[0]))
    engine.step_state.copy_(torch.tensor([length, length + 1, 1 % engine.capacity, 0], dtype=torch.int32))
    engine._enter_loop(length)
    for step in range(1, len(forced_tokens)):
        engine._ring_step()
        out.append(from_gpu_bf16(engine.logits).reshape(-1))
        picks.append(int(engine.token.item()))
        engine.token.copy_(torch.tensor([int(forced_tokens[step])], dtype=torch.int64, device=device))
        if engine.keys is not None:
            ops.embedding(engine.state.embed, engine.token, out=engine.hidden.view(1, -1))
    torch.cuda.synchronize()
    return out, picks
