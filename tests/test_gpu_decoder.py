"""End-to-end parity of the hip-gfx950 static-cache runtime against the CPU oracle decoder.

The runtime and the oracle run the same packed state (uploaded bit for bit).
Prefill logits/cache and one functional decode step must meet the per-op bf16
bars; greedy tokens must be identical, or the first divergence must sit on a
near-tie of the oracle's logits (the reference's own agreement criterion,
examples/qwen_quantized_agreement.py: flips only at top-2 ties).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle.decoder import DecoderShape, OracleDecoder
from tests.helpers import (
    assert_bf16_parity,
    bf16_bits_of,
    first_divergence,
    from_gpu_bf16,
    random_oracle_state,
    runtime_spec,
    state_to_device,
    to_gpu_bf16,
)

pytestmark = pytest.mark.gpu

TINY = DecoderShape(vocab=512, hidden=256, intermediate=512, layers=2, heads=4, kv_heads=2, head_dim=64,
                    eps=1e-6, theta=1e6)
PROMPT, NEW = 16, 10


def _pair(shape=TINY, seed=0, bias=True, prompt=PROMPT, new=NEW, family="qwen2"):
    from aotolith_amd.decoder import compile_decoder_state

    ostate = random_oracle_state(shape, seed, bias=bias)
    state = state_to_device(ostate, shape.group_size)
    runtime = compile_decoder_state(runtime_spec(shape, family, bias), state, prompt_length=prompt,
                                    max_new_tokens=new)
    oracle = OracleDecoder(shape, ostate, prompt + new)
    return runtime, oracle


def _margin_ok(divergence, logits_scale: float) -> bool:
    # A flip is a tie when the oracle's top two logits are within two bf16 ulps
    # of their magnitude (the GPU's f32 accumulation order decides the tie).
    return divergence["margin"] <= 2 * 2.0 ** -7 * max(abs(divergence["want_logit"]), logits_scale * 2.0 ** -4)


@pytest.mark.parametrize("bias", [True, False])
def test_prefill_logits_and_cache(bias):
    runtime, oracle = _pair(bias=bias, seed=1 + bias)
    ids = np.random.default_rng(3).integers(0, TINY.vocab, PROMPT)
    logits, cache = runtime.prefill_ids(ids)
    ref_logits, ref_cache = oracle.prefill(ids)
    assert tuple(logits.shape) == (1, 1, TINY.vocab)
    assert tuple(cache.shape) == ref_cache.shape
    assert_bf16_parity(from_gpu_bf16(logits), ref_logits, max_ulp=None, atol=2e-2, min_cos=0.999)
    assert_bf16_parity(from_gpu_bf16(cache), ref_cache, max_ulp=None, atol=2e-2, min_cos=0.999)


def test_decode_token_matches_the_oracle_and_rolls_the_cache():
    runtime, oracle = _pair(seed=4)
    ids = np.random.default_rng(5).integers(0, TINY.vocab, PROMPT)
    ref_logits, ref_compact = oracle.prefill(ids)
    ref_cache = oracle.pad_cache(ref_compact)
    cache = runtime.pad_cache(to_gpu_bf16(ref_compact))
    np.testing.assert_array_equal(from_gpu_bf16(cache), ref_cache)
    token = int(np.argmax(ref_logits))
    logits, next_cache = runtime.decode_token(torch.tensor([[token]]), cache, PROMPT + 1)
    want_logits, want_cache = oracle.decode(token, PROMPT + 1, ref_cache)
    assert_bf16_parity(from_gpu_bf16(logits), want_logits, max_ulp=None)
    got = from_gpu_bf16(next_cache)
    cap = PROMPT + NEW
    # the roll is a copy: bit-exact; the appended key/value meets the bf16 bars
    np.testing.assert_array_equal(got[..., : cap - 1, :], ref_cache[..., 1:, :])
    assert_bf16_parity(got[..., cap - 1, :], want_cache[..., cap - 1, :], max_ulp=None)
    # the input cache is not modified (functional contract)
    np.testing.assert_array_equal(from_gpu_bf16(cache), ref_cache)


@pytest.mark.parametrize("use_graph", [True, False])
def test_greedy_tokens_match_the_oracle(use_graph):
    runtime, oracle = _pair(seed=7)
    ids = np.random.default_rng(8).integers(0, TINY.vocab, PROMPT)
    tokens = runtime.greedy_generate(ids, use_graph=use_graph).cpu().numpy()
    want, history = oracle.greedy_generate(ids, NEW, record_logits=True)
    assert tokens.shape == (1, NEW)
    divergence = first_divergence(tokens, want, history)
    if divergence is not None:
        scale = float(np.abs(history[divergence["step"]]).max())
        assert _margin_ok(divergence, scale), divergence
    if use_graph:
        assert runtime.engine.graph_error is None, runtime.engine.graph_error


def test_graph_and_eager_loops_agree_and_repeat():
    runtime, _ = _pair(seed=9)
    ids = np.random.default_rng(10).integers(0, TINY.vocab, PROMPT)
    first = runtime.greedy_generate(ids).cpu().numpy()
    eager = runtime.greedy_generate(ids, use_graph=False).cpu().numpy()
    again = runtime.greedy_generate(ids).cpu().numpy()
    synced = runtime.greedy_generate(ids, sync_each_step=True).cpu().numpy()
    np.testing.assert_array_equal(first, eager)
    np.testing.assert_array_equal(first, again)
    np.testing.assert_array_equal(first, synced)
    short = runtime.greedy_generate(ids, max_new_tokens=3).cpu().numpy()
    np.testing.assert_array_equal(short[0], first[0, :3])


def test_graphs_captured_before_a_code_object_install_still_replay():
    """Installing a code object (an artifact load does) keeps the replaced module
    loaded: a runtime whose decode loop was captured over it replays its graph and
    gets the same tokens (an unload there would run freed kernel code)."""
    from aotolith_amd import _lib

    runtime, _ = _pair(seed=11)
    ids = np.random.default_rng(12).integers(0, TINY.vocab, PROMPT)
    first = runtime.greedy_generate(ids).cpu().numpy()
    _lib.install_code_object(_lib.default_code_object())
    again = runtime.greedy_generate(ids).cpu().numpy()
    torch.cuda.synchronize()
    np.testing.assert_array_equal(first, again)


def test_prefill_graph_replays_match_eager():
    """Captured ring prefills (one graph per left-pad width) replay with new ids and match eager runs."""

    runtime, _ = _pair(seed=21)
    rng = np.random.default_rng(22)
    prompts = [rng.integers(0, TINY.vocab, n) for n in (PROMPT, PROMPT - 4, PROMPT, PROMPT - 4, PROMPT - 9)]
    prompts.append(prompts[1])
    for ids in prompts:
        graphed = runtime.greedy_generate(ids).cpu().numpy()
        torch.cuda.synchronize()
        eager = runtime.greedy_generate(ids, use_graph=False).cpu().numpy()
        np.testing.assert_array_equal(graphed, eager)
    engine = runtime.engine
    assert engine.prefill_graph_error is None
    assert sorted(engine._prefill_graphs) == [0, 4, 9]


def test_ring_loop_matches_the_functional_roll():
    """The ring-buffer greedy loop gives the same tokens as chaining decode_token."""

    runtime, _ = _pair(seed=11)
    ids = np.random.default_rng(12).integers(0, TINY.vocab, PROMPT)
    ring_tokens = runtime.greedy_generate(ids, max_new_tokens=6).cpu().numpy()[0]
    logits, compact = runtime.prefill_ids(ids)
    cache = runtime.pad_cache(compact)
    tokens = [int(torch.argmax(logits.float().view(-1)))]
    valid = PROMPT
    for _ in range(5):
        valid += 1
        logits, cache = runtime.decode_token(torch.tensor([[tokens[-1]]]), cache, valid)
        tokens.append(int(torch.argmax(logits.float().view(-1))))
    # The two paths run the same kernels; only the attention's key order differs
    # (ring vs rolled window), so a flip needs a near-tie - none at this seed.
    np.testing.assert_array_equal(ring_tokens, np.array(tokens))


def test_padded_prefill_uses_the_left_pad_mask():
    runtime, oracle = _pair(seed=13, prompt=24, new=8)
    ids = np.random.default_rng(14).integers(0, TINY.vocab, 17)
    logits, compact = runtime.prefill_padded(ids)
    ref_logits, ref_compact = oracle.prefill(
        np.concatenate([np.zeros(7, dtype=np.int64), ids]),
        positions=np.concatenate([np.zeros(7, dtype=np.int64), np.arange(17)]),
        mask=oracle_mask(17, 24),
    )
    assert_bf16_parity(from_gpu_bf16(logits), ref_logits, max_ulp=None)
    assert_bf16_parity(from_gpu_bf16(compact)[..., 7:, :], ref_compact[..., 7:, :], max_ulp=None)
    # explicit-mask plan call gives the same bits as the implicit left-pad path
    from aotolith_amd.decoder import prefill_mask

    padded = torch.cat((torch.zeros(7, dtype=torch.int64), torch.from_numpy(ids)))[None]
    positions = torch.cat((torch.zeros(7, dtype=torch.int64), torch.arange(17)))[None]
    logits2, compact2 = runtime.prefill(padded, positions, prefill_mask(17, 24))
    np.testing.assert_array_equal(bf16_bits_of(logits2), bf16_bits_of(logits))
    np.testing.assert_array_equal(bf16_bits_of(compact2), bf16_bits_of(compact))


def oracle_mask(length, bucket):
    from oracle.ops import prefill_mask

    return prefill_mask(length, bucket)[0, 0]


def test_bucketed_runtime_dispatches_by_length():
    from aotolith_amd.decoder import compile_decoder_bucketed_state
    from aotolith_amd.errors import BucketRangeError

    ostate = random_oracle_state(TINY, 15)
    state = state_to_device(ostate, TINY.group_size)
    runtime = compile_decoder_bucketed_state(runtime_spec(TINY), state, prompt_lengths=[8, 16], max_new_tokens=4)
    assert runtime.prompt_lengths == (8, 16)
    assert runtime.bucket_for(5).prompt_length == 8
    assert runtime.bucket_for(9).prompt_length == 16
    with pytest.raises(BucketRangeError):
        runtime.bucket_for(17)
    ids = np.random.default_rng(16).integers(0, TINY.vocab, 12)
    tokens = runtime.greedy_generate(ids).cpu().numpy()
    oracle = OracleDecoder(TINY, ostate, 16 + 4)
    pad = np.zeros(4, dtype=np.int64)
    logits, compact = oracle.prefill(np.concatenate([pad, ids]), positions=np.concatenate([pad, np.arange(12)]),
                                     mask=oracle_mask(12, 16))
    assert int(tokens[0, 0]) == int(np.argmax(logits))
    # the two buckets share one packed state
    assert runtime.buckets[0].engine.state is runtime.buckets[1].engine.state


def test_selections_name_the_kernels_each_plan_launches():
    """Each plan's selections are one record per kernel it launches, named by the exact symbol,
    and the greedy loop launches exactly the kernels its plans name."""

    from aotolith_amd import ops
    from aotolith_amd.decoder import _prefill_pairs_gate_up

    runtime, _ = _pair(seed=17)
    for plan in (runtime.prefill, runtime.decode, runtime.decode_loop):
        selections = plan.selections
        assert selections, plan.name
        assert all(s.is_native and s.implementation == "hip_kernel" for s in selections)
        assert all(s.device_architecture == "gfx950" and s.artifact_name.startswith("aoto_") for s in selections)
        assert [s.op_index for s in selections] == list(range(len(selections)))
    for plan in (runtime.decode, runtime.decode_loop):
        heads = [s for s in plan.selections if s.kind == "decode_attention" and "." not in s.output_id]
        assert len(heads) == TINY.layers
    paired = _prefill_pairs_gate_up(PROMPT, TINY)
    assert any(name.endswith("_paired") for name in runtime.prefill.kernel_names()) == paired
    ids = np.random.default_rng(19).integers(0, TINY.vocab, PROMPT)
    with ops.recording_launches() as take:
        take()
        runtime.greedy_generate(ids, use_graph=False)
        greedy = take()
        logits, compact = runtime.prefill_ids(ids)
        cache = runtime.pad_cache(compact)
        take()
        runtime.decode_token(torch.tensor([[3]]), cache, PROMPT + 1)
        decode = take()
    assert set(greedy) == set(runtime.prefill.kernel_names()) | set(runtime.decode_loop.kernel_names())
    assert set(decode) == set(runtime.decode.kernel_names())


def test_runtime_rejects_bad_inputs():
    from aotolith_amd.errors import BucketRangeError, PlanInputError

    runtime, _ = _pair(seed=18)
    with pytest.raises(PlanInputError):
        runtime.prefill_ids(np.zeros(PROMPT + 1, dtype=np.int64))
    with pytest.raises(BucketRangeError):
        runtime.prefill_padded(np.zeros(PROMPT + 1, dtype=np.int64))
    cache = torch.zeros((TINY.layers, 2, 1, TINY.kv_heads, PROMPT + NEW, TINY.head_dim), dtype=torch.bfloat16,
                        device="cuda")
    with pytest.raises(PlanInputError):
        runtime.decode_token(torch.tensor([[1]]), cache, PROMPT + NEW)
    with pytest.raises(PlanInputError):
        runtime.greedy_generate(np.zeros(PROMPT, dtype=np.int64), max_new_tokens=NEW + 1)


# hidden 896: the shapes whose q/k/v GEMV takes the argmax finish in its prologue
NARROW = DecoderShape(vocab=4096, hidden=896, intermediate=1024, layers=2, heads=14, kv_heads=2, head_dim=64,
                      eps=1e-6, theta=1e6)


def test_folded_finish_loop_matches_the_unfolded_loop(monkeypatch):
    """The graph loop with each step's finish folded into the next step's q/k/v GEMV gives the
    same tokens and leaves the same loop state as the unfolded loop, graph-replayed or eager,
    synchronized per step or not, for every generation length; and it tracks the oracle."""

    runtime, oracle = _pair(NARROW, seed=21)
    assert runtime.engine.fold_finish
    monkeypatch.setenv("AOTOLITH_FOLD_FINISH", "0")
    plain, _ = _pair(NARROW, seed=21)
    assert not plain.engine.fold_finish
    ids = np.random.default_rng(22).integers(0, NARROW.vocab, PROMPT)
    want = plain.greedy_generate(ids).cpu().numpy()
    state = plain.engine.step_state.cpu().tolist(), int(plain.engine.history_len.item())
    for kwargs in ({}, {"use_graph": False}, {"sync_each_step": True}):
        got = runtime.greedy_generate(ids, **kwargs).cpu().numpy()
        np.testing.assert_array_equal(got, want, err_msg=str(kwargs))
        assert (runtime.engine.step_state.cpu().tolist(), int(runtime.engine.history_len.item())) == state
    for steps in (1, 2, 3, NEW - 1):
        short = runtime.greedy_generate(ids, max_new_tokens=steps).cpu().numpy()
        np.testing.assert_array_equal(short[0], want[0, :steps], err_msg=f"{steps} tokens")
    assert runtime.engine.graph_error is None, runtime.engine.graph_error
    reference, history = oracle.greedy_generate(ids, NEW, record_logits=True)
    divergence = first_divergence(want, reference, history)
    if divergence is not None:
        scale = float(np.abs(history[divergence["step"]]).max())
        assert _margin_ok(divergence, scale), divergence
