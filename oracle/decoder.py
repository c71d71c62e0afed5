"""CPU executor of the quantized static-cache decoder graph (the greedy-loop oracle).

Restates the module pair the reference traces - ``DecoderPrefillModule`` and
``DecoderDecodeModule`` with the packed-projection hooks of
``_QuantizedProjections`` (``models/decoder.py:420-745``) - after the rewrites
that decide its rounding points:

* decode: q/k/v ``addmm`` with RMSNorm prologue and bias epilogue, the fused
  ``rope_kv_cache_append`` roll, single-query attention, o/down ``addmm`` with
  the residual as bias, the paired gate/up GEMV with ``silu_mul_paired``, and the
  LM head with the final norm as prologue (``passes/fusion.py:112-549``,
  ``passes/cache.py:193-480``);
* prefill: standalone RMSNorm, dequant + matmul with bias / residual /
  ``silu_mul`` epilogues, RoPE, masked GQA attention, final norm on the last row.

The greedy loop is ``models/decoder.py:934-951, 1054-1087``: the first token is
the argmax of the prefill logits, then ``steps - 1`` decode steps, each at
position ``valid_length - 1`` with the mask "last ``valid_length`` slots".

State layout (a plain dict, filled by the test or bench from a seeded model)::

    embed [V, H], final_norm [H], lm_head (packed, scales_bits),
    layers[i]: qkv, o, gate, up, down as (packed, scales_bits),
               qkv_bias [Hq*D + 2*Hkv*D] or None, input_norm [H], post_norm [H]

Float tensors are f32 arrays of bf16-representable values; scales are bf16 bits.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

from .bf16 import round_bf16
from .ops import argmax_first, attention, rms_norm, rms_scale, rope, rope_tables
from .quant import dequantize_bits_bf16, dequantize_bits_exact


@dataclass(frozen=True)
class DecoderShape:
    vocab: int
    hidden: int
    intermediate: int
    layers: int
    heads: int
    kv_heads: int
    head_dim: int
    eps: float
    theta: float
    group_size: int = 64
    bits: int = 4

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


class OracleDecoder:
    """Prefill/decode/greedy over a packed state, on the CPU."""

    def __init__(self, shape: DecoderShape, state: dict, capacity: int) -> None:
        self.shape = shape
        self.state = state
        self.capacity = capacity
        self.cos, self.sin = rope_tables(capacity, shape.head_dim, shape.theta)
        self._exact: dict[int, np.ndarray] = {}
        self._rounded: dict[int, np.ndarray] = {}

    # weights -----------------------------------------------------------------
    def warm(self) -> None:
        """Unpack every weight once (the f32 exact and bf16-rounded matrices)."""

        self._w_exact(self.state["lm_head"])
        for layer in self.state["layers"]:
            for name in ("qkv", "o", "gate", "up", "down"):
                self._w_exact(layer[name])
                self._w_rounded(layer[name])

    def _w_exact(self, pair) -> np.ndarray:
        key = id(pair[0])
        if key not in self._exact:
            self._exact[key] = dequantize_bits_exact(pair[0], pair[1], self.shape.group_size, self.shape.bits)
        return self._exact[key]

    def _w_rounded(self, pair) -> np.ndarray:
        key = id(pair[0])
        if key not in self._rounded:
            self._rounded[key] = dequantize_bits_bf16(pair[0], pair[1], self.shape.group_size, self.shape.bits)
        return self._rounded[key]

    # decode-side fused GEMV (codegen/matmul.py:542-739) -------------------------
    # The products code * (x * s) are exact in f32; the sums here run in f32
    # BLAS (blocked), whose error (~1e-6 relative at K = 4864) is far below the
    # bf16 rounding every output takes.
    def _gemv(self, x, pair, *, norm=None, bias=None, up=None) -> np.ndarray:
        xv = np.asarray(x, dtype=np.float32).reshape(-1)
        if norm is not None:
            ns = rms_scale(xv, self.shape.eps)[0]
            xv = round_bf16((ns * xv) * norm)
        acc = self._w_exact(pair) @ xv
        if up is not None:
            acc_up = self._w_exact(up) @ xv
            g = round_bf16(acc).astype(np.float64)
            return round_bf16(acc_up.astype(np.float64) * (g / (1.0 + np.exp(-g))))
        if bias is not None:
            return round_bf16(bias.astype(np.float64) + acc.astype(np.float64))
        return round_bf16(acc)

    def _matmul(self, x, pair, *, bias=None, residual=None, gate=None) -> np.ndarray:
        acc = np.asarray(x, dtype=np.float32) @ self._w_rounded(pair).T
        acc = acc.astype(np.float64)
        if bias is not None:
            acc = acc + bias[None, :]
        if residual is not None:
            acc = acc + residual
        if gate is not None:
            g = gate.astype(np.float64)
            acc = acc * (g / (1.0 + np.exp(-g)))
        return round_bf16(acc)

    # prefill (models/decoder.py:524-561) --------------------------------------
    def prefill(self, ids, positions=None, mask=None):
        s = self.shape
        ids = np.asarray(ids, dtype=np.int64).reshape(-1)
        length = ids.shape[0]
        if positions is None:
            positions = np.arange(length)
        positions = np.asarray(positions, dtype=np.int64).reshape(-1)
        if mask is None:
            mask = np.tril(np.ones((length, length), dtype=bool))
        mask = np.asarray(mask, dtype=bool).reshape(length, length)
        cos = self.cos[positions][None, None]
        sin = self.sin[positions][None, None]
        hidden = self.state["embed"][ids]
        cache = np.zeros((s.layers, 2, 1, s.kv_heads, length, s.head_dim), dtype=np.float32)
        qd, kd = s.heads * s.head_dim, s.kv_heads * s.head_dim
        for index, layer in enumerate(self.state["layers"]):
            normalized = rms_norm(hidden, layer["input_norm"], s.eps)
            qkv = self._matmul(normalized, layer["qkv"], bias=layer.get("qkv_bias"))
            q = qkv[:, :qd].reshape(length, s.heads, s.head_dim).transpose(1, 0, 2)[None]
            k = qkv[:, qd : qd + kd].reshape(length, s.kv_heads, s.head_dim).transpose(1, 0, 2)[None]
            v = qkv[:, qd + kd :].reshape(length, s.kv_heads, s.head_dim).transpose(1, 0, 2)[None]
            q = rope(q, cos, sin)
            k = rope(k, cos, sin)
            out = attention(q, k, v, mask[None, None])
            out = out[0].transpose(1, 0, 2).reshape(length, qd)
            hidden = self._matmul(out, layer["o"], residual=hidden)
            normalized = rms_norm(hidden, layer["post_norm"], s.eps)
            gate = self._matmul(normalized, layer["gate"])
            act = self._matmul(normalized, layer["up"], gate=gate)
            hidden = self._matmul(act, layer["down"], residual=hidden)
            cache[index, 0, 0] = k[0]
            cache[index, 1, 0] = v[0]
        last = rms_norm(hidden[-1:], self.state["final_norm"], s.eps)
        logits = self._gemv(last, self.state["lm_head"])
        return logits, cache

    def pad_cache(self, compact) -> np.ndarray:
        """Left-pad a compact cache with zeros to capacity (``models/decoder.py:870-887``)."""

        pad = self.capacity - compact.shape[4]
        zeros = np.zeros(compact.shape[:4] + (pad,) + compact.shape[5:], dtype=np.float32)
        return np.concatenate((zeros, compact), axis=4)

    # decode (models/decoder.py:564-615, 889-932) -------------------------------
    def decode(self, token: int, valid_length: int, cache):
        s = self.shape
        position = valid_length - 1
        cos = self.cos[position]
        sin = self.sin[position]
        keep = np.arange(self.capacity) >= self.capacity - valid_length
        hidden = self.state["embed"][int(token)]
        qd, kd = s.heads * s.head_dim, s.kv_heads * s.head_dim
        next_cache = np.empty_like(cache)
        for index, layer in enumerate(self.state["layers"]):
            qkv = self._gemv(hidden, layer["qkv"], norm=layer["input_norm"], bias=layer.get("qkv_bias"))
            q = rope(qkv[:qd].reshape(1, s.heads, 1, s.head_dim), cos, sin)
            k = rope(qkv[qd : qd + kd].reshape(1, s.kv_heads, 1, s.head_dim), cos, sin)
            v = qkv[qd + kd :].reshape(1, s.kv_heads, 1, s.head_dim)
            pair = cache[index]
            new_pair = np.concatenate((pair[:, :, :, 1:, :], np.stack((k, v), axis=0)), axis=3)
            next_cache[index] = new_pair
            out = attention(q, new_pair[0], new_pair[1], keep[None, None, None, :])
            out = out.reshape(qd)
            hidden = self._gemv(out, layer["o"], bias=hidden)
            act = self._gemv(hidden, layer["gate"], norm=layer["post_norm"], up=layer["up"])
            hidden = self._gemv(act, layer["down"], bias=hidden)
        logits = self._gemv(hidden, self.state["lm_head"], norm=self.state["final_norm"])
        return logits, next_cache

    def greedy_generate(self, prompt_ids, steps: int, *, record_logits: bool = False):
        """Tokens ``[steps]`` (and optionally each step's logits)."""

        ids = np.asarray(prompt_ids, dtype=np.int64).reshape(-1)
        logits, compact = self.prefill(ids)
        cache = self.pad_cache(compact)
        tokens = [int(argmax_first(logits))]
        history = [logits] if record_logits else None
        valid = ids.shape[0]
        for _ in range(steps - 1):
            valid += 1
            logits, cache = self.decode(tokens[-1], valid, cache)
            tokens.append(int(argmax_first(logits)))
            if history is not None:
                history.append(logits)
        if record_logits:
            return np.asarray(tokens, dtype=np.int64), history
        return np.asarray(tokens, dtype=np.int64)
