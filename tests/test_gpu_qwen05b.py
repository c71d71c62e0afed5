"""Config 4 end to end: the Qwen2.5-0.5B-shape W4g64 model, 128-token prompt, 64 greedy tokens.

24 layers, hidden 896, intermediate 4864, 14/2 heads, head_dim 64, vocab 151936, q/k/v bias,
tied embeddings, rope_theta 1e6, bf16, batch 1 (reference ``compile_qwen2_static_cache``,
``models/qwen2.py:70-98``). The state is random-init on the GPU with non-trivial norms
(1 + N(0, 0.1)), seeded q/k/v biases and weights N(0, 0.03): at this width the stream of
greedy tokens then moves (with N(0, 0.02) weights a random model falls onto one repeated
token within a few steps, which would leave the check without power).

Agreement criterion (reference ``examples/qwen_quantized_agreement.py:1-24, 150-165`` and
``tests/test_quantized_qwen2.py:107-123``):

* the captured-graph greedy loop gives the oracle's 64 tokens, or the first divergence is
  reported with its top-2 margin;
* teacher-forced on the oracle's stream, the GPU's logits stay within the bar at every one of
  the 64 steps (per-step max|logit difference|, cosine and top-2 gap are printed), and every
  step where the two argmaxes differ is reported;
* the first divergence and every teacher-forced flip sit on a near-tie of the oracle's
  logits: a top-2 margin of at most twice that step's max|logit difference| (itself bounded
  by the cosine bar), so a flip on a wide margin fails however small the cosine gap (whether
  the margin is also within two bf16 ulps of the logit is printed);
* the prefill's K/V cache stays within ten times the oracle's own f32-vs-f64 deviation,
  layer by layer (ten, not five: the GPU's flash attention also rounds P to bf16 where the
  reference's flash kernel does, ``codegen/attention.py:367-371``, which the oracle's
  mlx-reference attention does not - measured at 1.6-5.3 times the f64 deviation), a bar
  that a planted mistake (one layer's input norm dropped) must fail.

The bar on the logits is set by the model's own sensitivity to rounding: 24 layers amplify a
one-ulp difference in any intermediate (the per-layer cache deviation grows geometrically with
depth). The oracle evaluated twice - its GEMMs accumulated in f32 BLAS and in f64, nothing
else changed - differs by a measured ``1 - cos``; the GPU may differ by at most five times
that. To show the bar has power, the same check is applied to the oracle with one planted
mistake (the final RMSNorm weight dropped), which must fail it.
"""

from __future__ import annotations

import numpy as np
import pytest

from oracle.bf16 import round_bf16
from oracle.decoder import DecoderShape, OracleDecoder
from tests.helpers import (
    first_divergence,
    from_gpu_bf16,
    near_tie,
    parity,
    state_to_oracle,
    teacher_forced_logits,
)

pytestmark = pytest.mark.gpu

PROMPT, NEW = 128, 64


def qwen05b_spec():
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family="qwen2", vocab=151936, hidden=896, intermediate=4864, layers=24, heads=14,
                       kv_heads=2, head_dim=64, eps=1e-6, theta=1e6, qkv_bias=True, tied=True,
                       max_position=32768)


class _F64Oracle(OracleDecoder):
    """The oracle with its prefill GEMMs accumulated in f64 instead of f32 BLAS: the same
    rounding points, a different summation order (the measure of the model's sensitivity)."""

    def _matmul(self, x, pair, *, bias=None, residual=None, gate=None):
        acc = np.asarray(x, dtype=np.float64) @ self._w_rounded(pair).T.astype(np.float64)
        if bias is not None:
            acc = acc + bias[None, :]
        if residual is not None:
            acc = acc + residual
        if gate is not None:
            g = gate.astype(np.float64)
            acc = acc.astype(np.float32).astype(np.float64) * (g / (1.0 + np.exp(-g)))
        return round_bf16(acc)


@pytest.mark.timeout(900)
def test_qwen05b_64_greedy_tokens_match_the_oracle():
    from aotolith_amd.decoder import compile_decoder_state, random_state

    spec = qwen05b_spec()
    state = random_state(spec, 64, seed=11, std=0.03, norm_std=0.1)
    runtime = compile_decoder_state(spec, state, prompt_length=PROMPT, max_new_tokens=NEW)
    shape = DecoderShape(vocab=spec.vocab, hidden=spec.hidden, intermediate=spec.intermediate, layers=spec.layers,
                         heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim, eps=spec.eps,
                         theta=spec.theta)
    ostate = state_to_oracle(state)
    oracle = OracleDecoder(shape, ostate, PROMPT + NEW)
    ids = np.random.default_rng(12).integers(0, spec.vocab, PROMPT)

    want, history = oracle.greedy_generate(ids, NEW, record_logits=True)
    distinct = len(set(want.tolist()))
    print(f"oracle stream: {distinct} distinct of {NEW}: {want.tolist()}")
    assert distinct >= 16, "the oracle's stream must move for the check to have power"

    # The bar: five times the oracle's own rounding sensitivity at the prefill logits.
    ref0 = np.asarray(history[0], dtype=np.float64).reshape(-1)
    f64_logits, f64_cache = _F64Oracle(shape, ostate, PROMPT + NEW).prefill(ids)
    noise = 1.0 - parity(f64_logits, ref0)["cosine"]
    bar = max(5.0 * noise, 1e-5)
    planted = OracleDecoder(shape, {**ostate, "final_norm": np.ones_like(ostate["final_norm"])}, PROMPT + NEW)
    planted_gap = 1.0 - parity(planted.prefill(ids)[0], ref0)["cosine"]
    print(f"oracle f32-vs-f64 noise 1-cos {noise:.3g}; bar {bar:.3g}; dropped final norm 1-cos {planted_gap:.3g}")
    assert planted_gap > bar, "the bar must reject a dropped norm weight"

    _, ref_cache = oracle.prefill(ids)
    _, cache = runtime.prefill_ids(ids)
    got_cache = from_gpu_bf16(cache)
    over, bars = [], []
    for layer in range(spec.layers):
        stats = parity(got_cache[layer], ref_cache[layer])
        layer_noise = 1.0 - parity(f64_cache[layer], ref_cache[layer])["cosine"]
        layer_bar = max(10.0 * layer_noise, 1e-5)
        bars.append(layer_bar)
        print(f"prefill cache layer {layer:2d}: max|d| {stats['max_abs']:.4f} 1-cos {1 - stats['cosine']:.3g} "
              f"(f64 noise {layer_noise:.3g}, bar {layer_bar:.3g})")
        if 1.0 - stats["cosine"] > layer_bar:
            over.append((layer, 1.0 - stats["cosine"], layer_bar))
    assert not over, over
    # the cache bar has power: one layer's input RMSNorm weight dropped moves that layer's cache past it
    layers = [dict(l) for l in ostate["layers"]]
    layers[12]["input_norm"] = np.ones_like(layers[12]["input_norm"])
    _, planted_cache = OracleDecoder(shape, {**ostate, "layers": layers}, PROMPT + NEW).prefill(ids)
    planted_layer = 1.0 - parity(planted_cache[12], ref_cache[12])["cosine"]
    print(f"dropped layer-12 input norm: cache 1-cos {planted_layer:.3g} (bar {bars[12]:.3g})")
    assert planted_layer > bars[12], "the cache bar must reject a dropped norm weight"

    tokens = runtime.greedy_generate(ids).cpu().numpy().reshape(-1)
    assert runtime.engine.graph_error is None, runtime.engine.graph_error
    divergence = first_divergence(tokens, want, history)
    agree = NEW if divergence is None else divergence["step"]
    print(f"graph loop: identical prefix {agree}/{NEW}; first divergence {divergence}")

    forced, picks = teacher_forced_logits(runtime, ids, want)
    if divergence is not None:
        # Up to the divergence the loop saw the oracle's tokens, so its logits there are the
        # teacher-forced ones: its pick must be the forced run's pick.
        assert picks[divergence["step"]] == divergence["got"], (picks[divergence["step"]], divergence)
    flips = []
    worst = 0.0
    for step, (got, ref) in enumerate(zip(forced, history)):
        ref = np.asarray(ref, dtype=np.float64).reshape(-1)
        stats = parity(got, ref)
        top = np.sort(ref)[-2:]
        print(f"step {step:2d}: max|dlogit| {stats['max_abs']:.4f} 1-cos {1 - stats['cosine']:.3g} "
              f"top-2 gap {top[1] - top[0]:.4f} max|logit| {np.abs(ref).max():.2f}")
        worst = max(worst, 1.0 - stats["cosine"])
        if picks[step] != int(want[step]):
            flips.append({"step": step, "got": picks[step], "want": int(want[step]),
                          "margin": float(top[1] - top[0]), "want_logit": float(ref[int(want[step])]),
                          "max_dlogit": stats["max_abs"]})
    print(f"teacher-forced: worst 1-cos {worst:.3g} (bar {bar:.3g}); argmax flips {flips}")
    assert worst <= bar
    for flip in flips:
        print(f"flip at step {flip['step']}: margin {flip['margin']:.4f}, two-ulp near-tie {near_tie(flip, history)}")
        assert flip["margin"] <= 2.0 * flip["max_dlogit"], flip
    if divergence is not None:
        # the loop's first divergence is the teacher-forced flip at that step
        assert any(flip["step"] == divergence["step"] for flip in flips), (divergence, flips)
