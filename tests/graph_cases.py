"""Callables and modules the graph-compiler tests capture (shared by the CPU and GPU tests).

Each case is ``(name, fn, inputs_factory, tolerance)``; the inputs are seeded
CPU tensors. Together they cover every node family the gfx950 lowering has:
broadcast elementwise in f32 / bf16 / int64 / bool, reductions and scans over
any dims, mm / bmm / addmm with transposed operands, embedding and advanced
indexing, cat / slice / expand views, fills and aranges, the RMSNorm chain and
scaled-dot-product attention (causal, bool and float masks, grouped heads).
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def _g(seed):
    return torch.Generator().manual_seed(seed)


def _randn(seed, *shape, dtype=torch.float32):
    return torch.randn(*shape, generator=_g(seed)).to(dtype)


def elementwise_broadcast(x, y):
    return (x + y * 2.0).sigmoid() * y.exp() - x.abs().sqrt() / (1.0 + y * y)


def elementwise_math(x):
    return torch.stack([x.tanh(), x.cos(), x.sin(), F.gelu(x), F.gelu(x, approximate="tanh"), F.silu(x),
                        x.relu(), torch.erf(x), x.clamp(-0.5, 0.7), torch.rsqrt(x.abs() + 1)], 0)


def comparisons(x, y):
    lt = x < y
    both = lt & (x > -1.0)
    either = lt | (y >= 0.5)
    return torch.where(both, x, y), either.to(torch.int64).sum(-1), torch.masked_fill(x, ~either, -3.0)


def integer_math(ids):
    pos = torch.arange(ids.shape[-1]) + 3
    prod = ids * pos - 7
    return prod // 4, prod % 5, torch.div(prod, 3, rounding_mode="trunc"), (prod > 10).cumsum(-1)


def reductions(x):
    return (x.sum(-1), x.mean((0, 2), keepdim=True), x.amax(1), x.amin((0, 1)), x.argmax(-1), x.argmin(1),
            (x > 0).any(-1), (x > -3).all(0))


def softmaxes(x):
    return torch.softmax(x, -1), torch.log_softmax(x, 1), torch.softmax(x * 3.0, 0)


def linear(x, w, b):
    return F.linear(x, w, b), F.linear(x, w)


def batched(a, b):
    return torch.bmm(a, b.transpose(1, 2)), a @ b.transpose(1, 2)[:, :, :3]


def indexing(table, ids, x):
    e = F.embedding(ids, table)
    picked = x[:, torch.tensor([2, 0, 1])]
    pair = x[torch.tensor([1, 0]), torch.tensor([3, 2])]
    sel = torch.index_select(x, 1, torch.tensor([3, 3, 0]))
    return e, picked, pair, sel


def views(x, y):
    z = torch.cat([x, y.transpose(0, 1)], dim=1)
    parts = z[:, 1:5:2]
    rep = x.unsqueeze(1).expand(-1, 3, -1).reshape(x.shape[0] * 3, -1)
    return z, parts * 2.0, rep.contiguous() + 1.0, z.permute(1, 0)[::2]


def rms_chain(x, w):
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + 1e-5)
    return w * h.to(x.dtype)


def attention(q, k, v, mask):
    causal = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    masked = F.scaled_dot_product_attention(q, k, v, attn_mask=mask)
    additive = F.scaled_dot_product_attention(q, k, v, attn_mask=torch.where(mask, 0.0, -1e4), scale=0.3)
    return causal, masked, additive


def grouped_attention(q, k, v):
    return F.scaled_dot_product_attention(q, k, v, is_causal=True, enable_gqa=True)


def bf16_block(x, w, norm_w):
    h = rms_chain(x, norm_w)
    y = F.linear(h, w)
    return F.silu(y) * y, (y.float().softmax(-1)).to(torch.bfloat16)


CASES = [
    ("elementwise_broadcast", elementwise_broadcast, lambda: (_randn(1, 3, 1, 5), _randn(2, 4, 5)), 1e-5),
    ("elementwise_math", elementwise_math, lambda: (_randn(3, 6, 7),), 2e-5),
    ("comparisons", comparisons, lambda: (_randn(4, 5, 6), _randn(5, 6)), 1e-6),
    ("integer_math", integer_math, lambda: (torch.randint(-20, 20, (3, 9), generator=_g(6)),), 0.0),
    ("reductions", reductions, lambda: (_randn(7, 5, 6, 33),), 1e-5),
    ("softmaxes", softmaxes, lambda: (_randn(8, 4, 5, 40),), 1e-5),
    ("linear", linear, lambda: (_randn(9, 2, 5, 48), _randn(10, 40, 48), _randn(11, 40)), 2e-5),
    ("batched", batched, lambda: (_randn(12, 3, 70, 33), _randn(13, 3, 65, 33)), 2e-5),
    ("indexing", indexing, lambda: (_randn(14, 50, 16), torch.randint(0, 50, (2, 7), generator=_g(15)),
                                    _randn(16, 4, 5, 3)), 0.0),
    ("views", views, lambda: (_randn(17, 6, 4), _randn(18, 5, 6)), 1e-6),
    ("rms_chain", rms_chain, lambda: (_randn(19, 3, 64), 1.0 + 0.1 * _randn(20, 64)), 1e-5),
    ("attention", attention, lambda: (_randn(21, 2, 3, 9, 16), _randn(22, 2, 3, 11, 16), _randn(23, 2, 3, 11, 8),
                                      torch.rand(9, 11, generator=_g(24)) > 0.3), 2e-5),
    ("grouped_attention", grouped_attention, lambda: (_randn(25, 1, 4, 6, 8), _randn(26, 1, 2, 6, 8),
                                                      _randn(27, 1, 2, 6, 8)), 2e-5),
    ("bf16_block", bf16_block, lambda: (_randn(28, 5, 32, dtype=torch.bfloat16),
                                        _randn(29, 24, 32, dtype=torch.bfloat16) * 0.2,
                                        (1.0 + 0.1 * _randn(30, 32)).to(torch.bfloat16)), 1.6e-2),
]


def tiny_llama(seed: int = 0):
    """Config 1: the reference's tiny Llama (vocab 128, hidden 32, 2 layers, 4/2 heads, max_pos 16), fp32."""

    from transformers import LlamaConfig, LlamaForCausalLM

    torch.manual_seed(seed)
    config = LlamaConfig(vocab_size=128, hidden_size=32, intermediate_size=64, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=16)
    return LlamaForCausalLM(config).eval()


def tiny_qwen2(seed: int = 0):
    from transformers import Qwen2Config, Qwen2ForCausalLM

    torch.manual_seed(seed)
    config = Qwen2Config(vocab_size=96, hidden_size=32, intermediate_size=48, num_hidden_layers=2,
                         num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=32,
                         tie_word_embeddings=True)
    model = Qwen2ForCausalLM(config).eval()
    with torch.no_grad():
        for layer in model.model.layers:
            for proj in (layer.self_attn.q_proj, layer.self_attn.k_proj, layer.self_attn.v_proj):
                proj.bias.copy_(torch.randn(proj.bias.shape, generator=_g(seed + 5)) * 0.1)
    return model


def config1_ids(seed: int = 0):
    """input_ids int64 [1, 4] ~ U[0, 128) (config 1)."""

    return torch.randint(0, 128, (1, 4), generator=_g(seed))


def module_case(model):
    """A wrapper whose forward is the HF call the reference's compile_module captures."""

    class Logits(torch.nn.Module):
        def __init__(self, inner):
            super().__init__()
            self.inner = inner

        def forward(self, input_ids):
            return self.inner(input_ids=input_ids, use_cache=False).logits

    return Logits(model).eval()
