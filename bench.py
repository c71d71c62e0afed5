"""Benchmark of the W4 g64 static-cache decode/prefill path on one MI355X.

Workload: Qwen2.5-0.5B-architecture random-init model,
W4 group-64 packed, bf16 activations, batch 1, a 128-token uniform-random
prompt and 64 greedy tokens. One *step* is one greedy generation: prefill of
the prompt (first token) plus 63 device-driven decode steps on a HIP graph.

Printed JSON line (rank 0):
  value            decode tok/s = 63 decode tokens per generation / their device time
  prefill_tok_s    128 / (prefill + cache fill + argmax), device time
  decode_tok_s_sync decode tok/s with a host sync after every token
  roofline         the LM-head W4 GEMV the greedy loop runs (151936 x 896, RMSNorm
                   prologue, fused argmax keys): algorithmic bytes per launch / average
                   launch duration (HIP events on its stream, rotating weight copies
                   > 1 GiB so HBM, not the 256 MB Infinity Cache, feeds it) against 8 TB/s
  kernels          per-kernel table of the decode step and the prefill: each kernel
                   launched once per layer over the model's own 24 layer copies inside
                   a HIP graph, HIP events around the replays; GB/s against 8 TB/s for
                   the decode kernels, TFLOP/s against 2.5 PFLOP/s for the prefill ones
  cpu_baseline     the CPU oracle (restated reference semantics, NumPy) on the host
                   cores: prefill of the same prompt plus 63 decode steps
  parity           greedy tokens of the GPU run vs the CPU oracle over the 64 tokens

``--gpus N`` with N > 1 exits: every GPU box here has one GPU.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
HBM_PEAK_GBS = 8000.0
# Random-init state of the Qwen workload: weights N(0, 0.03) and norms 1 + N(0, 0.1), the
# recipe of the config-4 parity test (a random model at N(0, 0.02) falls onto one
# repeated greedy token within a few steps, which leaves a token comparison no power).
STATE_STD = 0.03
STATE_NORM_STD = 0.1


def qwen_spec():
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family="qwen2", vocab=151936, hidden=896, intermediate=4864, layers=24, heads=14,
                       kv_heads=2, head_dim=64, eps=1e-6, theta=1e6, qkv_bias=True, tied=True,
                       max_position=32768)


def llama8b_spec():
    from aotolith_amd.decoder import DecoderSpec

    return DecoderSpec(family="llama", vocab=128256, hidden=4096, intermediate=14336, layers=32, heads=32,
                       kv_heads=8, head_dim=128, eps=1e-5, theta=5e5, qkv_bias=False, tied=False,
                       max_position=131072)


def gemv_bytes(n: int, k: int, group: int = 64, *, norm: bool = False, bias: bool = False,
               paired: bool = False, bits: int = 4) -> int:
    """Algorithmic bytes of one packed GEMV launch: weights, scales, x, y (+ norm w, bias)."""

    weights = n * k * bits // 8 + n * (k // group) * 2
    total = weights * (2 if paired else 1) + 2 * k + 2 * n
    if norm:
        total += 2 * k
    if bias:
        total += 2 * n
    return total


def step_weight_bytes(spec, group: int = 64, bits: int = 4) -> int:
    """Algorithmic bytes of one decode token's GEMVs (the weight stream)."""

    h, i = spec.hidden, spec.intermediate
    per_layer = (
        gemv_bytes(spec.qkv_width, h, group, norm=True, bias=spec.qkv_bias, bits=bits)
        + gemv_bytes(h, spec.attention_width, group, bias=True, bits=bits)
        + gemv_bytes(i, h, group, norm=True, paired=True, bits=bits)
        + gemv_bytes(h, i, group, bias=True, bits=bits)
    )
    return spec.layers * per_layer + gemv_bytes(spec.vocab, h, group, norm=True, bits=bits)


def measure_lm_head_gemv(spec, torch, ops, *, launches: int = 24, rounds: int = 9, pool_bytes: float = 1.2e9,
                         bits: int = 4) -> dict:
    """Average duration of the LM-head GEMV over a rotating pool of weight copies.

    For four-bit weights this is the greedy loop's own LM-head kernel: the GEMV
    with the RMSNorm prologue that also writes the per-wave argmax keys
    (``ops.w4_gemv_argmax``); the plain GEMV otherwise. Each round queues
    ``launches`` back-to-back launches behind a spin kernel (so they run without
    host gaps) between two HIP events on the launching stream; the result is the
    median round's per-launch time. Long rounds (hundreds of launches) measured
    ~1-2 us per launch slower than short ones on the same box, so rounds are kept
    short.
    """

    n, k, group = spec.vocab, spec.hidden, 64
    per = gemv_bytes(n, k, group, norm=True, bits=bits)
    copies = max(2, int(pool_bytes // per) + 1)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(1)
    words = [torch.randint(-2 ** 31, 2 ** 31 - 1, (n, k * bits // 32), generator=gen, dtype=torch.int32,
                           device="cuda")
             for _ in range(copies)]
    scales = [(torch.rand((n, k // group), generator=gen, device="cuda") * 0.003).to(torch.bfloat16)
              for _ in range(copies)]
    x = torch.randn(k, generator=gen, device="cuda").to(torch.bfloat16)
    norm = torch.ones(k, dtype=torch.bfloat16, device="cuda")
    out = torch.empty(n, dtype=torch.bfloat16, device="cuda")
    key_count = ops.argmax_key_count(k, n, group) if bits == 4 else 0
    keys = torch.empty((max(key_count, 1),), dtype=torch.int64, device="cuda")
    if key_count:
        kernel = ("aoto_w4_gemv_x8x4_n1_argmax / _x32x4_n1_argmax (the greedy loop's LM head: RMSNorm prologue + "
                  "argmax keys)")

        def launch(i):
            ops.w4_gemv_argmax(x, words[i], scales[i], group, keys, norm_weight=norm, eps=spec.eps, out=out)
    else:
        kernel = f"aoto_w{bits}_gemv (RMSNorm prologue)"
        gemv = ops.w4_gemv if bits == 4 else ops.w8_gemv

        def launch(i):
            gemv(x, words[i], scales[i], group, norm_weight=norm, eps=spec.eps, out=out)

    stream = torch.cuda.current_stream()
    for i in range(copies):
        launch(i)
    torch.cuda.synchronize()
    per_round = []
    index = 0
    for _ in range(rounds):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        # A spin kernel holds the stream while Python enqueues the round, so the
        # timed launches run back to back instead of at the host's enqueue rate.
        torch.cuda._sleep(5_000_000)
        start.record(stream)
        for _ in range(launches):
            launch(index % copies)
            index += 1
        end.record(stream)
        torch.cuda.synchronize()
        per_round.append(start.elapsed_time(end) * 1000.0 / launches)
    per_round.sort()
    avg_us = per_round[len(per_round) // 2]
    achieved = per / (avg_us * 1e-6) / 1e9
    del words, scales
    torch.cuda.empty_cache()
    return {
        "kernel": f"{kernel}, LM head {n}x{k}, g64",
        "bytes_per_launch": per,
        "avg_us": avg_us,
        "round_us": [round(v, 3) for v in per_round],
        "achieved": achieved,
        "copies": copies,
        "launches": launches * rounds,
    }


def _graph_us(torch, body, count: int, rounds: int = 5) -> float:
    """Per-launch microseconds of ``body`` (``count`` launches) replayed as one HIP graph."""

    body()  # kernel lookup and any workspace allocation happen outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    graph.replay()
    torch.cuda.synchronize()
    times = []
    for _ in range(rounds):
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        end.record()
        torch.cuda.synchronize()
        times.append(start.elapsed_time(end) * 1000.0 / count)
    del graph
    return sorted(times)[rounds // 2]


def _row(name: str, kernel: str, us: float, *, nbytes: int | None = None, flops: float | None = None) -> dict:
    row = {"name": name, "kernel": kernel, "avg_us": round(us, 3)}
    if nbytes is not None:
        gbs = nbytes / (us * 1e-6) / 1e9
        row.update({"bytes": int(nbytes), "achieved": round(gbs, 1), "unit": "GB/s", "peak": HBM_PEAK_GBS,
                    "frac": round(gbs / HBM_PEAK_GBS, 4)})
    if flops is not None:
        tf = flops / (us * 1e-6) / 1e12
        row.update({"flops": float(flops), "achieved": round(tf, 1), "unit": "TFLOP/s", "peak": MFMA_BF16_PEAK_TFLOPS,
                    "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)})
    return row


def _rotation(weights: list, torch, pool_bytes: float) -> list:
    """The weights to cycle through: the given ones, then copies of them until their
    packed words and scales exceed ``pool_bytes`` (more than the 256 MB Infinity
    Cache and the L2s hold), so no launch finds its weights cached from an earlier one."""

    from dataclasses import replace

    out = list(weights)
    size = sum(w.packed.numel() * 4 + w.scales.numel() * 2 for w in weights)
    while size < pool_bytes:
        w = weights[len(out) % len(weights)]
        out.append(replace(w, packed=w.packed.clone(), scales=w.scales.clone()))
        size += w.packed.numel() * 4 + w.scales.numel() * 2
    return out


def decode_kernel_table(runtime, torch, ops, valid: int | None = None, pool_bytes: float = 0.6e9) -> list[dict]:
    """Per-kernel times of the greedy loop's decode step, one row per kernel kind.

    Each GEMV kind is launched over a rotation of its layers' weights, extended with
    copies to more than ``pool_bytes`` (a small model's 24 layers of one kind fit in
    the Infinity Cache, where the loop, which streams a whole step between two reads
    of one layer, does not find them), inside one HIP graph; the time is the median
    replay / launch count. The attention runs once per layer over the layers' own
    KV windows (as in the loop). Bytes are the algorithmic bytes of one launch
    (weights, scales, x, y, bias or residual, norm weight; the attention's K/V window
    of ``valid`` keys). The loop's state is left as a fresh loop would find it.
    """

    eng = runtime.engine
    spec = runtime.spec
    layers = eng.state.layers
    n = len(layers)
    # per kind: (weight, its layer's norm / bias / up weights), cycled
    qkv_w = _rotation([l.qkv for l in layers], torch, pool_bytes)
    o_w = _rotation([l.o for l in layers], torch, pool_bytes)
    down_w = _rotation([l.down for l in layers], torch, pool_bytes)
    gate_w = _rotation([l.gate for l in layers], torch, pool_bytes / 2)
    up_w = _rotation([l.up for l in layers], torch, pool_bytes / 2)
    bits = eng.state.bits
    h, i = spec.hidden, spec.intermediate
    qd, kd = spec.heads * spec.head_dim, spec.kv_heads * spec.head_dim
    valid = valid or (runtime.prompt_length + runtime.max_new_tokens // 2)
    eng.step_state.copy_(torch.tensor([valid - 1, valid, 1 % eng.capacity, 0], dtype=torch.int32))
    eng.rope_rows[0].copy_(eng.cos[valid - 1])
    eng.rope_rows[1].copy_(eng.sin[valid - 1])
    eng.hidden.copy_(eng.state.embed[1])
    eng.attn.zero_()
    eng.act.zero_()
    rows = []

    def qkv():
        for index, w in enumerate(qkv_w):
            layer = layers[index % n]
            eng._gemv(eng.hidden, w, eng.qkv, norm_weight=layer.input_norm, eps=spec.eps, bias=layer.qkv_bias)

    def attention():
        for index in range(n):
            ops.decode_rope_attention(eng.qkv.view(1, -1), eng.cos, eng.sin, eng.ring[index],
                                      query_heads=spec.heads, query_start=0, key_start=qd, value_start=qd + kd,
                                      step_state=eng.step_state, scale=eng.scale, workspace=eng.workspace,
                                      splits=eng.attention_splits,
                                      rope_rows=eng.rope_rows if eng.keys is not None else None, out=eng.attn)

    def o_proj():
        for w in o_w:
            eng._gemv(eng.attn.view(-1), w, eng.hidden, bias=eng.hidden)

    def gate_up():
        for index, (g, u) in enumerate(zip(gate_w, up_w)):
            eng._gemv(eng.hidden, g, eng.act, norm_weight=layers[index % n].post_norm, eps=spec.eps,
                      up=(u.packed, u.scales))

    def down():
        for w in down_w:
            eng._gemv(eng.act, w, eng.hidden, bias=eng.hidden)

    w = f"w{bits}"
    rows.append(_row("qkv", f"aoto_{w}_gemv (RMSNorm prologue, bias)", _graph_us(torch, qkv, len(qkv_w)),
                     nbytes=gemv_bytes(spec.qkv_width, h, norm=True, bias=spec.qkv_bias, bits=bits)))
    rows.append(_row("attention", f"aoto_decode_rope_attention_d{spec.head_dim} (RoPE, KV write, {valid} keys)",
                     _graph_us(torch, attention, n), nbytes=2 * spec.kv_heads * valid * spec.head_dim * 2))
    rows.append(_row("o", f"aoto_{w}_gemv (residual)", _graph_us(torch, o_proj, len(o_w)),
                     nbytes=gemv_bytes(h, spec.attention_width, bias=True, bits=bits)))
    rows.append(_row("gate_up", f"aoto_{w}_gemv paired (RMSNorm prologue, silu_mul)",
                     _graph_us(torch, gate_up, len(gate_w)),
                     nbytes=gemv_bytes(i, h, norm=True, paired=True, bits=bits)))
    rows.append(_row("down", f"aoto_{w}_gemv (residual)", _graph_us(torch, down, len(down_w)),
                     nbytes=gemv_bytes(h, i, bias=True, bits=bits)))
    for row, weights in zip(rows, (qkv_w, None, o_w, gate_w, down_w)):
        if weights is not None:
            row["rotation"] = len(weights)
    del qkv_w, o_w, down_w, gate_w, up_w
    if eng.keys is not None:
        head = eng.state.lm_head

        def finish():
            for _ in range(n):
                ops.argmax_finish(eng.keys, eng.key_count, out=eng.token, history=None, history_len=None)

        ops.w4_gemv_argmax(eng.hidden, head.packed, head.scales, head.group, eng.keys,
                           norm_weight=eng.state.final_norm, eps=spec.eps, out=eng.logits.view(-1))
        if eng.fold_finish:
            # the loop's per-token form: the finish in layer 0's q/k/v GEMV (the
            # standalone finish runs once per generation, for the last token)
            qkv_f = _rotation([layers[0].qkv], torch, pool_bytes)
            hidden = torch.empty_like(eng.hidden)

            def qkv_finish():
                for w in qkv_f:
                    ops.w4_gemv_finish(eng.keys, eng.key_count, eng.state.embed, w.packed, w.scales, w.group,
                                       norm_weight=layers[0].input_norm, eps=spec.eps, bias=layers[0].qkv_bias,
                                       out=eng.qkv, token_out=eng.token, hidden_out=hidden)

            rows.append(_row("qkv_finish", f"aoto_{w}_gemv_*_finish (the previous token's argmax finish, then "
                             "layer 0's q/k/v GEMV on its embedding row)", _graph_us(torch, qkv_finish, len(qkv_f)),
                             nbytes=gemv_bytes(spec.qkv_width, h, norm=True, bias=spec.qkv_bias, bits=bits)))
            rows[-1]["rotation"] = len(qkv_f)
            del qkv_f
        rows.append(_row("argmax_finish", "aoto_argmax_finish (token from the per-wave keys"
                         + ("; once per generation with the folded loop)" if eng.fold_finish else ")"),
                         _graph_us(torch, finish, n)))
    torch.cuda.synchronize()
    return rows


def prefill_kernel_table(runtime, torch, ops) -> list[dict]:
    """Per-kernel times of the prefill at the bucket length, one row per launch kind.

    Each op is launched once per layer with that layer's weights inside one HIP
    graph (median replay / layer count); a GEMM row includes its split-K reduce (or
    the fused reduce + residual + next RMSNorm) when the plan splits. FLOPs are
    ``2 M N K`` for a projection and ``4 M^2 D Hq / 2`` for the causal attention.
    """

    eng = runtime.engine
    spec = runtime.spec
    layers = eng.state.layers
    n = len(layers)
    m = runtime.prompt_length
    h, i = spec.hidden, spec.intermediate
    dev = eng.device
    bf16 = torch.bfloat16
    gen = torch.Generator(device=dev)
    gen.manual_seed(3)
    x = torch.randn((m, h), generator=gen, device=dev).to(bf16)
    xn = torch.randn((m, h), generator=gen, device=dev).to(bf16)
    qkv = torch.empty((1, m, spec.qkv_width), dtype=bf16, device=dev)
    q = torch.randn((1, spec.heads, m, spec.head_dim), generator=gen, device=dev).to(bf16)
    attn = torch.randn((1, m, spec.attention_width), generator=gen, device=dev).to(bf16)
    act = torch.randn((m, i), generator=gen, device=dev).to(bf16)
    positions = torch.arange(m, dtype=torch.int64, device=dev)[None, :]
    slot0 = eng.capacity - m
    gate_up = ops.w4_matmul_gate_up if eng.state.bits == 4 else ops.w8_matmul_gate_up

    def qkv_rope():
        for index, layer in enumerate(layers):
            ops.matmul_qkv_rope(xn, layer.qkv.packed, layer.qkv.scales, layer.qkv.group, positions.reshape(-1),
                                eng.cos, eng.sin, eng.ring[index], query_heads=spec.heads, kv_heads=spec.kv_heads,
                                head_dim=spec.head_dim, slot0=slot0, bias=layer.qkv_bias, bits=layer.qkv.bits,
                                out=qkv.view(m, -1), q_out=q)

    def attention():
        for index in range(n):
            pair = eng.ring[index]
            ops.prefill_attention(q, pair[0][:, :, slot0:slot0 + m], pair[1][:, :, slot0:slot0 + m], causal=True,
                                  key_start=0, scale=eng.scale, out=attn)

    def o_norm():
        for layer in layers:
            ops.matmul_residual_norm(attn.view(m, -1), layer.o.packed, layer.o.scales, layer.o.group, x,
                                     layer.post_norm, spec.eps, bits=layer.o.bits, out=x, norm_out=xn)

    def mlp():
        for layer in layers:
            gate_up(xn, layer.gate.packed, layer.gate.scales, layer.up.packed, layer.up.scales, layer.gate.group,
                    out=act)

    def down_norm():
        for layer in layers:
            ops.matmul_residual_norm(act, layer.down.packed, layer.down.scales, layer.down.group, x,
                                     layer.input_norm, spec.eps, bits=layer.down.bits, out=x, norm_out=xn)

    bits = eng.state.bits
    plan = ops.wide_plan(m, spec.qkv_width, h)
    gemm = f"aoto_w{bits}_gemm_w* (wide tiles, 32x32x16 MFMA)" if ops.wide_plan(m, h, h) else f"aoto_w{bits}_gemm_n*"
    if ops.lds_plan(m, spec.qkv_width, h, bits=bits, rope=True) is not None:
        qkv_label = ("aoto_w4_gemm_d8w* (packed tiles expanded once per 256-row block into LDS) + bias, then "
                     "aoto_rope_qkv_rows (RoPE and cache fill)")
    elif plan is not None:
        qkv_label = (f"aoto_w{bits}_gemm_w* tile {plan[0]} + bias, then aoto_rope_qkv_rows (RoPE and cache fill)"
                     if plan[1] == 1 else f"aoto_w{bits}_gemm_w* tile {plan[0]}, {plan[1]}-way split, then "
                     "aoto_w4_gemm_reduce_rope (sum, bias, RoPE and cache fill)")
    else:
        qkv_label = (f"aoto_w{bits}_gemm + bias, RoPE and cache fill (split: aoto_w4_gemm_reduce_rope; unsplit: RoPE "
                     "in the GEMM epilogue, or aoto_rope_qkv_rows after it)")
    once = {
        ops.LDS_SHORT_NARROW_TILE: "aoto_w4_gemm_d4c1w1x1_paired (packed tiles expanded once per 128 x (32 + 32) "
                                   "block into LDS, 32x32x16 MFMA)",
        ops.LDS_SHORT_PAIRED_TILE: "aoto_w4_gemm_d4w2x1_paired (packed tiles expanded once per 128 x (64 + 64) "
                                   "block into LDS, 32x32x16 MFMA)",
        ops.LDS_SPLIT_NARROW_TILE: "aoto_w4_gemm_d4c1w1x1_split (packed tiles expanded once per 128 x 32 block "
                                   "into LDS, 32x32x16 MFMA, split-K partials) + reduce",
        ops.LDS_SPLIT_TILE: "aoto_w4_gemm_d4c2w2x1_split (packed tiles expanded once per 128 x 64 block into "
                            "LDS, 32x32x16 MFMA, split-K partials) + reduce",
    }

    def label(n_, k_, paired=False):
        tile = ops.lds_plan(m, n_, k_, paired=paired, bits=bits)
        if tile is None:
            return gemm
        return once.get(tile, "aoto_w4_gemm_d8w* (packed tiles expanded once per 256-row block into LDS, "
                              "32x32x16 MFMA)")

    mlp_label = f"{label(i, h, True)} paired gate/up + silu_mul"
    rows = [
        _row("qkv_rope", qkv_label, _graph_us(torch, qkv_rope, n), flops=2.0 * m * spec.qkv_width * h),
        _row("attention", f"aoto_flash_attention_d{spec.head_dim} (causal)", _graph_us(torch, attention, n),
             flops=4.0 * m * m * spec.head_dim * spec.heads / 2),
        _row("o_norm", f"{label(h, spec.attention_width)} + residual, then the next RMSNorm",
             _graph_us(torch, o_norm, n), flops=2.0 * m * h * spec.attention_width),
        _row("gate_up", mlp_label, _graph_us(torch, mlp, n),
             flops=2.0 * m * 2 * i * h),
        _row("down_norm", f"{label(h, i)} + residual, then the next RMSNorm", _graph_us(torch, down_norm, n),
             flops=2.0 * m * h * i),
    ]
    torch.cuda.synchronize()
    return rows


def counter_traffic() -> int | None:
    """HBM bytes per LM-head GEMV launch from the committed counter summary, or None.

    The figure comes from two rocprofv3 --pmc runs (FETCH_SIZE, WRITE_SIZE) of
    ``bench.py --roofline-only``, calibrated on a copy of known size; the
    summary file records the commands and the raw counts.
    """

    path = os.path.join(ROOT, "profiles", "lm_head_gemv_qwen05b_traffic.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return int(json.loads(block)["traffic_bytes"])
    except (OSError, IndexError, KeyError, ValueError):
        return None


def cpu_baseline(spec, runtime, prompt, gpu_tokens, decode_steps: int) -> dict:
    """Time the CPU oracle on the same state and prompt: prefill + ``decode_steps`` decode steps."""

    import numpy as np
    import torch

    from oracle.decoder import DecoderShape, OracleDecoder

    state = runtime.engine.state

    def bits(t):
        return t.detach().cpu().contiguous().view(torch.int16).numpy().view(np.uint16)

    def f32(t):
        return t.detach().cpu().float().numpy()

    def pair(w):
        return (w.packed.cpu().numpy(), bits(w.scales))

    ostate = {
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
    shape = DecoderShape(vocab=spec.vocab, hidden=spec.hidden, intermediate=spec.intermediate, layers=spec.layers,
                         heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim, eps=spec.eps,
                         theta=spec.theta, bits=runtime.quantize_bits)
    oracle = OracleDecoder(shape, ostate, runtime.cache_capacity)
    ids = np.asarray(prompt, dtype=np.int64).reshape(-1)
    t0 = time.perf_counter()
    oracle.warm()
    t_setup = time.perf_counter() - t0
    t0 = time.perf_counter()
    logits, compact = oracle.prefill(ids)
    first = int(np.argmax(logits))
    t_prefill = time.perf_counter() - t0
    cache = oracle.pad_cache(compact)
    tokens = [first]
    history = [np.asarray(logits, dtype=np.float32).reshape(-1)]  # the oracle's logits of every token
    valid = ids.shape[0]
    t0 = time.perf_counter()
    for _ in range(decode_steps):
        valid += 1
        logits, cache = oracle.decode(tokens[-1], valid, cache)
        history.append(np.asarray(logits, dtype=np.float32).reshape(-1))
        tokens.append(int(np.argmax(logits)))
    t_decode = time.perf_counter() - t0
    margins = []
    for row in history:
        top = np.sort(row.astype(np.float64))[-2:]
        margins.append(float(top[1] - top[0]))
    try:
        from threadpoolctl import threadpool_info

        threads = max((info.get("num_threads", 1) for info in threadpool_info()), default=1)
    except Exception:  # noqa: BLE001 - informational
        threads = 1
    gpu = [int(t) for t in gpu_tokens[: len(tokens)]]
    agree = 0
    for a, b in zip(gpu, tokens):
        if a != b:
            break
        agree += 1
    divergence = None
    if agree < len(tokens):
        divergence = {"step": agree, "gpu": gpu[agree], "oracle": tokens[agree], "oracle_top2_margin": margins[agree],
                      "oracle_logit_max": float(np.abs(history[agree]).max())}
    # Teacher-forced on the oracle's stream (the GPU's own step kernels, fed the oracle's
    # tokens): the GPU logits' deviation at every step and the steps whose argmax differs.
    from tests.helpers import teacher_forced_logits

    forced, picks = teacher_forced_logits(runtime, ids, tokens)
    worst, flips = 0.0, []
    for step, (got, ref) in enumerate(zip(forced, history)):
        got, ref = np.asarray(got, dtype=np.float64), ref.astype(np.float64)
        cos = float(got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref)))
        worst = max(worst, 1.0 - cos)
        if picks[step] != tokens[step]:
            flips.append({"step": step, "oracle_top2_margin": margins[step],
                          "max_abs_logit_diff": float(np.abs(got - ref).max())})
    return {
        "baseline": {
            "value": decode_steps / t_decode,
            "unit": "decode tok/s",
            "cores": int(threads),
            "kind": "port",
            "sample": (f"CPU oracle (NumPy restatement of the reference's mlx-reference semantics, f32/f64 BLAS), "
                       f"same packed state and prompt: prefill of {ids.shape[0]} tokens "
                       f"({ids.shape[0] / t_prefill:.1f} tok/s) then {decode_steps} decode steps; weight "
                       f"unpacking ({t_setup:.1f} s) excluded; host has {len(os.sched_getaffinity(0))} cores"),
            "prefill_tok_s": ids.shape[0] / t_prefill,
        },
        "parity": {
            "steps_compared": len(tokens),
            "identical_prefix": agree,
            "gpu_tokens": gpu,
            "oracle_tokens": tokens,
            "oracle_top2_margins": margins,
            "first_divergence": divergence,
            "teacher_forced_worst_1_minus_cos": worst,
            "teacher_forced_flips": flips,
        },
    }


def run_llama8b(args, torch, ops) -> dict:
    """Config 5: Llama-3-8B shape, buckets {512, 2048}, 256 greedy tokens (one GPU)."""

    from aotolith_amd.decoder import compile_decoder_bucketed_state, random_state

    spec = llama8b_spec()
    print("[bench] building the random-init Llama-3-8B-shape W4 state", file=sys.stderr, flush=True)
    state = random_state(spec, 64, seed=0, norm_std=STATE_NORM_STD)
    new = 256
    runtime = compile_decoder_bucketed_state(spec, state, prompt_lengths=[512, 2048], max_new_tokens=new)
    gen = torch.Generator().manual_seed(0)
    out = {}
    for bucket in (512, 2048):
        prompt = torch.randint(0, spec.vocab, (1, bucket), generator=gen).cuda()
        for _ in range(max(1, args.warmup)):
            runtime.greedy_generate(prompt, max_new_tokens=8)
        torch.cuda.synchronize()
        records = []
        for _ in range(max(1, args.steps // 5)):
            events: dict = {}
            runtime.greedy_generate(prompt, events=events)
            records.append(events)
        torch.cuda.synchronize()
        prefill_ms = sum(e["start"].elapsed_time(e["prefill"]) for e in records) / len(records)
        decode_ms = sum(e["prefill"].elapsed_time(e["end"]) for e in records) / len(records)
        out[f"bucket_{bucket}"] = {
            "prefill_tok_s": round(bucket / (prefill_ms / 1000.0), 1),
            "prefill_gemm_tflops": round(2 * bucket * llama_params(spec) / (prefill_ms / 1000.0) / 1e12, 1),
            "decode_tok_s": round((new - 1) / (decode_ms / 1000.0), 2),
            "decode_ms_per_token": round(decode_ms / (new - 1), 4),
            "decode_weight_stream_gbs": round(step_weight_bytes(spec) * (new - 1) / (decode_ms / 1000.0) / 1e9, 1),
            "generations": len(records),
        }
        print(f"[bench] llama8b bucket {bucket}: {out[f'bucket_{bucket}']}", file=sys.stderr, flush=True)
        if not args.no_kernels:
            b = runtime.bucket_for(bucket)
            out[f"bucket_{bucket}"]["kernels"] = {"decode": decode_kernel_table(b, torch, ops),
                                                  "prefill": prefill_kernel_table(b, torch, ops)}
            for name, table in out[f"bucket_{bucket}"]["kernels"].items():
                for row in table:
                    print(f"[bench] llama8b {bucket} {name} {row['name']}: {row['avg_us']} us {row.get('frac', '')}",
                          file=sys.stderr, flush=True)
    if not args.no_roofline:
        lm = measure_lm_head_gemv(spec, torch, ops, launches=12, rounds=5, pool_bytes=1.5e9)
        out["lm_head_gemv"] = {"avg_us": round(lm["avg_us"], 2), "achieved_gbs": round(lm["achieved"], 1),
                               "frac": round(lm["achieved"] / HBM_PEAK_GBS, 4), "bytes": lm["bytes_per_launch"]}
    return out


def measure_prefill_attention(spec, torch, ops, tokens: int, launches: int = 20, std: float = 1.0) -> dict:
    """The causal prefill attention of one layer at ``tokens`` queries, timed alone.

    q [1, Hq, tokens, D], keys and values [1, Hkv, tokens, D] of N(0, std^2) bf16,
    the model's GQA heads and 1/sqrt(D) scale; the median of 5 replays of a HIP
    graph of ``launches`` launches between HIP events. FLOP = 2 * tokens^2 * D * Hq
    (the causal half of 4 * M * Mk * D * Hq), against the bf16 MFMA peak. The time
    depends on the data (MI355X lowers its clock under MFMA work on busier bit
    patterns: ~10-20% between std 1 and 0.02 at 2048 tokens), hence ``std``.
    """

    gen = torch.Generator(device="cuda")
    gen.manual_seed(0)
    hq, hkv, d = spec.heads, spec.kv_heads, spec.head_dim
    q = (torch.randn(1, hq, tokens, d, generator=gen, device="cuda") * std).to(torch.bfloat16)
    k = (torch.randn(1, hkv, tokens, d, generator=gen, device="cuda") * std).to(torch.bfloat16)
    v = (torch.randn(1, hkv, tokens, d, generator=gen, device="cuda") * std).to(torch.bfloat16)
    out = torch.empty(1, tokens, hq * d, device="cuda", dtype=torch.bfloat16)

    def body():
        for _ in range(launches):
            ops.prefill_attention(q, k, v, causal=True, scale=d ** -0.5, out=out)

    us = _graph_us(torch, body, launches)
    flops = 2.0 * tokens * tokens * d * hq
    return {"kernel": f"aoto_flash_attention_d{d}* (causal)", "avg_us": round(us, 3), "flops": flops,
            "tflops": round(flops / us / 1e6, 1), "frac": round(flops / us / 1e6 / MFMA_BF16_PEAK_TFLOPS, 4)}


def measure_prefill_gemms(spec, torch, ops, tokens: int, launches: int = 10, library: bool = False) -> dict:
    """One decoder layer's prefill projections at ``tokens`` rows, timed alone.

    q/k/v (+bias when the model has it), o (+residual), gate/up (two GEMMs, or the
    paired one where the decoder pairs them) and down (+residual) on random packed
    weights, each the median of 3 replays of a HIP graph of ``launches`` launches
    (no host overhead between them) between HIP events; TFLOP/s = 2 * tokens * N * K
    / duration (for counter runs: MFMA utilization against the bf16 peak).

    ``library``: also time, as a comparison only (never a product path), the vendor
    library's bf16 GEMM (``torch.matmul``, hipBLASLt) on the same weights unpacked to
    bf16 ahead of time, and the unpack (``aoto_w4_dequantize``) of each weight.
    """

    from aotolith_amd.decoder import _prefill_pairs_gate_up

    dev = "cuda"
    gen = torch.Generator(device=dev)
    gen.manual_seed(0)

    def packed(n, k):
        w = (torch.randn(n, k, generator=gen, device=dev) * 0.02).to(torch.bfloat16)
        return ops.w4_quantize(w, 64)

    h, i = spec.hidden, spec.intermediate
    x_h = torch.randn(tokens, h, generator=gen, device=dev).to(torch.bfloat16)
    x_a = torch.randn(tokens, spec.attention_width, generator=gen, device=dev).to(torch.bfloat16)
    x_i = torch.randn(tokens, i, generator=gen, device=dev).to(torch.bfloat16)
    res = torch.randn(tokens, h, generator=gen, device=dev).to(torch.bfloat16)
    qkv_w, o_w, gate_w, up_w, down_w = (packed(spec.qkv_width, h), packed(h, spec.attention_width), packed(i, h),
                                         packed(i, h), packed(h, i))
    bias = torch.randn(spec.qkv_width, generator=gen, device=dev).to(torch.bfloat16) if spec.qkv_bias else None
    out_q = torch.empty(tokens, spec.qkv_width, device=dev, dtype=torch.bfloat16)
    out_h = torch.empty(tokens, h, device=dev, dtype=torch.bfloat16)
    out_i = torch.empty(tokens, i, device=dev, dtype=torch.bfloat16)
    gate = torch.empty_like(out_i)
    paired = _prefill_pairs_gate_up(tokens, spec)
    cases = [
        ("qkv", spec.qkv_width, h, lambda: ops.w4_matmul(x_h, *qkv_w, 64, bias=bias, out=out_q)),
        ("o", h, spec.attention_width, lambda: ops.w4_matmul(x_a, *o_w, 64, residual=res, out=out_h)),
    ]
    if paired:
        cases.append(("gate_up", 2 * i, h, lambda: ops.w4_matmul_gate_up(x_h, *gate_w, *up_w, 64, out=out_i)))
    else:
        cases.append(("gate", i, h, lambda: ops.w4_matmul(x_h, *gate_w, 64, out=gate)))
        cases.append(("up", i, h, lambda: ops.w4_matmul(x_h, *up_w, 64, gate=gate, out=out_i)))
    cases.append(("down", h, i, lambda: ops.w4_matmul(x_i, *down_w, 64, residual=res, out=out_h)))
    if library:
        dense = {}
        for name, w in (("qkv", qkv_w), ("o", o_w), ("gate", gate_w), ("up", up_w), ("down", down_w)):
            dense[name] = ops.w4_dequantize(*w, 64)
        xs = {"qkv": x_h, "o": x_a, "gate": x_h, "up": x_h, "down": x_i}
        for name in dense:
            cases.append((f"library_{name}", dense[name].shape[0], dense[name].shape[1],
                          lambda name=name: torch.matmul(xs[name], dense[name].t())))
            w = {"qkv": qkv_w, "o": o_w, "gate": gate_w, "up": up_w, "down": down_w}[name]
            cases.append((f"unpack_{name}", dense[name].shape[0], dense[name].shape[1],
                          lambda w=w: ops.w4_dequantize(*w, 64)))
        # the epilogues the library GEMM leaves to elementwise kernels: the residual add
        # (o, down) and silu_mul (gate/up); FLOP columns of these rows are not meaningful
        lib_out = torch.empty(tokens, h, device=dev, dtype=torch.bfloat16)
        cases.append(("library_residual_add", h, 1, lambda: torch.add(out_h, res, out=lib_out)))
        lib_g = torch.empty(tokens, i, device=dev, dtype=torch.bfloat16)
        cases.append(("library_silu_mul", i, 1,
                      lambda: torch.mul(torch.nn.functional.silu(out_i), gate, out=lib_g)))
    out = {}
    for name, n, k, run in cases:
        with ops.recording_launches() as take:
            take()
            run()  # allocates any split-K workspace outside the capture
            kernels = take()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            for _ in range(launches):
                run()
        graph.replay()
        torch.cuda.synchronize()
        rounds = []
        for _ in range(3):
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            graph.replay()
            end.record()
            torch.cuda.synchronize()
            rounds.append(start.elapsed_time(end) * 1000.0 / launches)
        us = sorted(rounds)[1]
        tflops = 2.0 * tokens * n * k / (us * 1e-6) / 1e12
        out[name] = {"M": tokens, "N": n, "K": k, "us": round(us, 2), "tflops": round(tflops, 1),
                     "mfma_frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4), "kernels": kernels}
    return out


def llama_params(spec) -> int:
    """Weight elements of the projections (the prefill GEMM work is 2 * tokens * this)."""

    h, i = spec.hidden, spec.intermediate
    per_layer = spec.qkv_width * h + h * spec.attention_width + 2 * i * h + h * i
    return spec.layers * per_layer


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=10, help="timed greedy generations")
    parser.add_argument("--warmup", type=int, default=3)
    parser.add_argument("--prompt", type=int, default=128)
    parser.add_argument("--new", type=int, default=64)
    parser.add_argument("--cpu-decode-steps", type=int, default=63,
                        help="oracle decode steps timed and compared (63: the whole 64-token generation)")
    parser.add_argument("--no-cpu-baseline", action="store_true")
    parser.add_argument("--no-roofline", action="store_true")
    parser.add_argument("--no-kernels", action="store_true", help="skip the per-kernel table")
    parser.add_argument("--workload", choices=("qwen0.5b", "llama8b"), default="qwen0.5b")
    parser.add_argument("--bits", type=int, choices=(4, 8), default=4,
                        help="weight code width of the qwen0.5b workload (8: the quantize_bits=8 variant)")
    parser.add_argument("--roofline-only", action="store_true",
                        help="only the LM-head GEMV loop, after a calibration copy of 256 MiB (for counter runs)")
    parser.add_argument("--prefill-attention-only", type=int, default=0, metavar="TOKENS",
                        help="only the causal prefill attention of one layer at TOKENS queries (timing, counter runs)")
    parser.add_argument("--input-std", type=float, default=1.0,
                        help="standard deviation of the --prefill-attention-only inputs")
    parser.add_argument("--decode-kernels-only", action="store_true",
                        help="only the decode step's per-kernel table (after a 256 MiB calibration copy)")
    parser.add_argument("--library-comparison", action="store_true",
                        help="with --prefill-gemm-only: also time the vendor bf16 GEMM on unpacked weights")
    parser.add_argument("--prefill-gemm-only", type=int, default=0, metavar="TOKENS",
                        help="only one layer's prefill GEMMs at TOKENS rows (for MFMA counter runs)")
    args = parser.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: --gpus {args.gpus} is not supported on this one-GPU path "
              "(no collectives are built; see the sharding design notes)", file=sys.stderr)
        return 2

    import torch

    from aotolith_amd import ops
    from aotolith_amd.decoder import compile_decoder_state, random_state

    torch.cuda.set_device(0)
    if args.roofline_only:
        spec = qwen_spec() if args.workload == "qwen0.5b" else llama8b_spec()
        src = torch.empty(1 << 26, dtype=torch.int32, device="cuda")  # 256 MiB
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        lm = measure_lm_head_gemv(spec, torch, ops, bits=args.bits)
        print(json.dumps({"calibration_copy_bytes": src.numel() * 4, **lm}), flush=True)
        return 0
    if args.prefill_attention_only:
        spec = qwen_spec() if args.workload == "qwen0.5b" else llama8b_spec()
        result = measure_prefill_attention(spec, torch, ops, args.prefill_attention_only, std=args.input_std)
        print(json.dumps({"workload": f"{args.workload} prefill attention", "tokens": args.prefill_attention_only,
                          "input_std": args.input_std, "peak_tflops": MFMA_BF16_PEAK_TFLOPS, **result}), flush=True)
        return 0
    if args.prefill_gemm_only:
        spec = qwen_spec() if args.workload == "qwen0.5b" else llama8b_spec()
        gemms = measure_prefill_gemms(spec, torch, ops, args.prefill_gemm_only, library=args.library_comparison)
        print(json.dumps({"workload": f"{args.workload} prefill GEMMs", "tokens": args.prefill_gemm_only,
                          "peak_tflops": MFMA_BF16_PEAK_TFLOPS, **gemms}), flush=True)
        return 0
    if args.decode_kernels_only:
        # the decode step's per-kernel table alone (after a 256 MiB calibration copy, for
        # counter runs): the workload's full-depth random-init state, bucket = --prompt
        spec = qwen_spec() if args.workload == "qwen0.5b" else llama8b_spec()
        src = torch.empty(1 << 26, dtype=torch.int32, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        prompt = args.prompt if args.workload == "qwen0.5b" else 512
        new = args.new if args.workload == "qwen0.5b" else 256
        std = {"std": STATE_STD} if args.workload == "qwen0.5b" else {}  # as the workload's own bench line
        state = random_state(spec, 64, seed=0, norm_std=STATE_NORM_STD, bits=args.bits, **std)
        runtime = compile_decoder_state(spec, state, prompt_length=prompt, max_new_tokens=new)
        rows = decode_kernel_table(runtime, torch, ops)
        print(json.dumps({"workload": f"{args.workload} decode kernels", "prompt": prompt, "new_tokens": new,
                          "calibration_copy_bytes": src.numel() * 4, "decode": rows}), flush=True)
        return 0
    if args.workload == "llama8b":
        result = run_llama8b(args, torch, ops)
        print(json.dumps({"workload": "llama-3-8b-shape W4g64 buckets {512, 2048}, 256 greedy tokens, bs1",
                          "data": "synthetic random-init", **result}), flush=True)
        return 0
    spec = qwen_spec()
    bits = args.bits
    print(f"[bench] building the random-init W{bits} state on {torch.cuda.get_device_name(0)}", file=sys.stderr,
          flush=True)
    state = random_state(spec, 64, seed=0, std=STATE_STD, norm_std=STATE_NORM_STD, bits=bits)
    runtime = compile_decoder_state(spec, state, prompt_length=args.prompt, max_new_tokens=args.new)
    gen = torch.Generator().manual_seed(0)
    prompt = torch.randint(0, spec.vocab, (1, args.prompt), generator=gen)
    prompt_dev = prompt.cuda()

    for _ in range(args.warmup):
        runtime.greedy_generate(prompt_dev)
    torch.cuda.synchronize()
    print("[bench] warmup done", file=sys.stderr, flush=True)

    records = []
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tokens = None
    for _ in range(args.steps):
        events: dict = {}
        tokens = runtime.greedy_generate(prompt_dev, events=events)
        records.append(events)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    prefill_ms = sum(e["start"].elapsed_time(e["prefill"]) for e in records) / len(records)
    decode_ms = sum(e["prefill"].elapsed_time(e["end"]) for e in records) / len(records)
    decode_steps = args.new - 1
    decode_tok_s = decode_steps / (decode_ms / 1000.0)
    prefill_tok_s = args.prompt / (prefill_ms / 1000.0)
    print(f"[bench] timed {args.steps} generations: prefill {prefill_ms:.3f} ms, decode {decode_ms:.3f} ms",
          file=sys.stderr, flush=True)

    # decode with a host sync after every token (the reference's sync_each_step)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    sync_events: dict = {}
    runtime.greedy_generate(prompt_dev, sync_each_step=True, events=sync_events)
    torch.cuda.synchronize()
    decode_sync_ms = sync_events["prefill"].elapsed_time(sync_events["end"])
    decode_tok_s_sync = decode_steps / (decode_sync_ms / 1000.0)
    _ = time.perf_counter() - t1

    roofline = None
    if not args.no_roofline:
        lm = measure_lm_head_gemv(spec, torch, ops, bits=bits)
        roofline = {
            "bound": "hbm",
            "achieved": round(lm["achieved"], 1),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(lm["achieved"] / HBM_PEAK_GBS, 4),
            "traffic": counter_traffic() if bits == 4 else None,
            "traffic_source": ("recorded: profiles/lm_head_gemv_qwen05b_traffic.md (rocprofv3 --pmc FETCH_SIZE, "
                               "WRITE_SIZE of bench.py --roofline-only, calibrated on a copy)") if bits == 4 else None,
            "kernel": lm["kernel"],
            "avg_us": round(lm["avg_us"], 3),
            "round_us": lm["round_us"],
            "bytes_per_launch": lm["bytes_per_launch"],
        }
        print(f"[bench] LM-head GEMV {lm['avg_us']:.2f} us, {lm['achieved']:.0f} GB/s", file=sys.stderr, flush=True)

    kernels = None
    if not args.no_kernels:
        kernels = {"decode": decode_kernel_table(runtime, torch, ops),
                   "prefill": prefill_kernel_table(runtime, torch, ops)}
        for name, table in kernels.items():
            for row in table:
                print(f"[bench] {name} {row['name']}: {row['avg_us']} us "
                      f"{row.get('frac', '')}", file=sys.stderr, flush=True)

    baseline = None
    parity = None
    if not args.no_cpu_baseline:
        print("[bench] CPU oracle baseline ...", file=sys.stderr, flush=True)
        result = cpu_baseline(spec, runtime, prompt.numpy(), tokens.cpu().numpy().reshape(-1),
                              args.cpu_decode_steps)
        baseline = result["baseline"]
        parity = result["parity"]

    weight_bytes = step_weight_bytes(spec, bits=bits)
    line = {
        "metric": f"decode tok/s + quant-GEMV HBM GB/s, prefill tok/s; Qwen2.5-0.5B-shape W{bits}g64 bs1",
        "value": round(decode_tok_s, 2),
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed * 1000.0 / args.steps, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": f"synthetic (random-init weights N(0,{STATE_STD}) packed W{bits} g64 on the GPU, seeded q/k/v bias, "
                f"norms 1+N(0,{STATE_NORM_STD}), uniform-random prompt ids)",
        "config": {
            "workload": f"qwen2.5-0.5b-shape W{bits}g64 static-cache greedy: prompt 128, 64 new tokens, bs1 "
                        "(one step = one generation: prefill + 63 graph-replayed decode steps)",
            "prompt": args.prompt,
            "new_tokens": args.new,
            "layers": spec.layers,
            "hidden": spec.hidden,
            "vocab": spec.vocab,
        },
        "prefill_tok_s": round(prefill_tok_s, 1),
        "decode_tok_s_sync": round(decode_tok_s_sync, 2),
        "decode_ms_per_token": round(decode_ms / decode_steps, 4),
        "decode_weight_stream_gbs": round(weight_bytes * decode_tok_s / 1e9, 1),
        "decode_graph": runtime.engine.graph_error or "captured",
        "prefill_graph": runtime.engine.prefill_graph_error or "captured",
        "roofline": roofline,
        "kernels": kernels,
        "cpu_baseline": baseline,
        "parity": parity,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
