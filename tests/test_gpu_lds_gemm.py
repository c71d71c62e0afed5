"""GPU parity of the dequant-once prefill GEMM (csrc/w4_gemm_lds.h, tile codes 811 / 812 /
813 / 814 / 821 / 822 / 823).

Each 64-k step of a block's packed words is expanded once into an LDS bf16 tile that the
block's waves (8 on 256-row blocks, 4 on the short prompts' 128-row blocks) read as
MFMA operands. Every form is compared with the CPU oracle within one bf16 ulp (two for the
silu_mul products) and with the wide-tile kernel under an explicit plan: ragged M and N
tails, step counts that leave every remainder of the six-step unrolled loop, groups of 32 /
64 / 128, the bias and residual epilogues (in place too), the paired gate/up; the automatic
plan's choice at 2048 rows and at short prompts; graph replays against eager; the refusals.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import ops as oracle
from oracle.bf16 import round_bf16
from oracle.quant import pack_weight_bits_bf16
from tests.helpers import assert_bf16_parity, bf16_normal, from_gpu_bf16, to_gpu_bf16, to_gpu_bits

pytestmark = pytest.mark.gpu


def _ops():
    from aotolith_amd import ops

    return ops


def _weights(rng, n, k, group=64):
    packed, scales = pack_weight_bits_bf16(bf16_normal(rng, (n, k), 0.02), group, 4)
    return packed, scales, torch.from_numpy(packed).cuda(), to_gpu_bits(scales)


def _atol(expected):
    return 2e-2 * max(1.0, float(np.abs(expected).max()) / 4)


def _traced(fn):
    ops = _ops()
    with ops.recording_launches() as take:
        take()
        out = fn()
        names = take()
    return out, names


def _lds(names):
    return [name for name in names if name.startswith(("aoto_w4_gemm_d8w", "aoto_w4_gemm_d4"))]


SHORT_PAIRED = {811: "aoto_w4_gemm_d4c1w1x1_paired", 812: "aoto_w4_gemm_d4w2x1_paired"}
SHORT_SPLIT = {813: "aoto_w4_gemm_d4c1w1x1_split", 814: "aoto_w4_gemm_d4c2w2x1_split"}


@pytest.mark.parametrize("group,k", [(32, 448), (32, 896), (32, 576), (64, 640), (32, 704), (128, 768),
                                     (64, 1152)])
@pytest.mark.parametrize("epilogue", ["none", "bias", "residual"])
def test_lds_gemm_explicit(epilogue, group, k):
    """Tile 822 on 300 rows (one full and one ragged 256-row block) and N = 720 (five full
    128-column blocks and a ragged one); K = 448 ... 1152 gives 7, 14, 9, 10, 11, 12 and 18
    steps of 64: every remainder 0-5 of the six-step unrolled loop."""

    ops = _ops()
    m, n = 300, 720
    rng = np.random.default_rng(700 + group + k + len(epilogue))
    packed, scales, gp, gs = _weights(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    gkw = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: ops.w4_matmul(gx, gp, gs, group, tile=822, **gkw))
    assert names == [f"aoto_w4_gemm_d8w2x2_b{int(epilogue == 'bias')}_r{int(epilogue == 'residual')}"], names
    expected = oracle.w4_matmul(x, packed, scales, group, **kwargs)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))
    if k % 128 == 0 and (k // group) % 2 == 0:
        wide = ops.w4_matmul(gx, gp, gs, group, tile=441, splits=1, **gkw)
        assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(wide), max_ulp=1.0, atol=_atol(expected))


@pytest.mark.parametrize("group,k", [(32, 448), (64, 640), (128, 768), (32, 1216)])
@pytest.mark.parametrize("epilogue", ["none", "bias", "residual"])
def test_lds_gemm_192_columns_explicit(epilogue, group, k):
    """Tile 823 (256 x 192 blocks, X in two staging buffers) on 300 rows and N = 720 (three
    full 192-column blocks and a ragged one); K = 448 / 640 / 768 / 1216: 7 / 10 / 12 / 19
    steps of 64."""

    ops = _ops()
    m, n = 300, 720
    rng = np.random.default_rng(710 + group + k + len(epilogue))
    packed, scales, gp, gs = _weights(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    gkw = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    y, names = _traced(lambda: ops.w4_matmul(to_gpu_bf16(x), gp, gs, group, tile=823, **gkw))
    assert names == [f"aoto_w4_gemm_d8w2x3_b{int(epilogue == 'bias')}_r{int(epilogue == 'residual')}"], names
    expected = oracle.w4_matmul(x, packed, scales, group, **kwargs)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))


@pytest.mark.parametrize("group,k", [(64, 640), (32, 1088)])
def test_lds_gate_up_explicit(group, k):
    """Tile 821: bf16(up * silu(bf16(gate))), N = 608 (nine full 64-column blocks and a
    half one), within the bars of the oracle's two-step result."""

    ops = _ops()
    m, n = 300, 608
    rng = np.random.default_rng(720 + group + k)
    gpk, gsc, g_packed, g_scales = _weights(rng, n, k, group)
    upk, usc, u_packed, u_scales = _weights(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    y, names = _traced(lambda: ops.w4_matmul_gate_up(to_gpu_bf16(x), g_packed, g_scales, u_packed, u_scales, group,
                                                     tile=821))
    assert names == ["aoto_w4_gemm_d8w2x1_paired"], names
    want_gate = round_bf16(oracle.w4_matmul(x, gpk, gsc, group))
    expected = oracle.w4_matmul(x, upk, usc, group, gate=want_gate)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0)


@pytest.mark.parametrize("tile", [811, 812])
@pytest.mark.parametrize("m,group,k", [(1, 64, 640), (16, 32, 448), (96, 64, 896), (128, 128, 768),
                                       (200, 32, 704), (128, 64, 1152)])
def test_lds_gate_up_short_prompt_tiles(tile, m, group, k):
    """Tiles 811 / 812 (128-row blocks of 4 waves, 32 + 32 / 64 + 64 columns): ragged and
    partial row blocks (1-200 rows), N = 608 (19 / 9.5 column blocks), K of 7 / 14 / 12 /
    11 / 18 steps (every remainder of the six-step loop but 3, which 9 steps of the next
    test cover), groups 32-128, within the bars of the oracle's two-step result; both
    tiles give the same bits (one summation order)."""

    ops = _ops()
    n = 608
    rng = np.random.default_rng(725 + m + group + k)
    gpk, gsc, g_packed, g_scales = _weights(rng, n, k, group)
    upk, usc, u_packed, u_scales = _weights(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: ops.w4_matmul_gate_up(gx, g_packed, g_scales, u_packed, u_scales, group, tile=tile))
    assert names == [SHORT_PAIRED[tile]], names
    want_gate = round_bf16(oracle.w4_matmul(x, gpk, gsc, group))
    expected = oracle.w4_matmul(x, upk, usc, group, gate=want_gate)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0)
    other = ops.w4_matmul_gate_up(gx, g_packed, g_scales, u_packed, u_scales, group, tile=1623 - tile)
    assert torch.equal(y, other)


def test_lds_gate_up_is_the_automatic_plan_at_short_prompts():
    """The paired gate/up of a 0.5B-class MLP (896 -> 2 x 4864) at 128 rows takes tile 811
    (152 blocks) by itself, an 8B-class one (4096 -> 2 x 14336) tile 812 (224 blocks), and
    16 rows stay on the 16x16 kernel; K = 576 in groups of 32 (9 steps) covers the loop's
    remainder 3."""

    ops = _ops()
    assert ops.lds_plan(128, 4864, 896, paired=True) == ops.LDS_SHORT_NARROW_TILE
    assert ops.lds_plan(128, 14336, 4096, paired=True) == ops.LDS_SHORT_PAIRED_TILE
    assert ops.lds_plan(16, 4864, 896, paired=True) is None
    rng = np.random.default_rng(745)
    for m, n, k, group, want in [(128, 4864, 576, 32, 811), (128, 14336, 4096, 64, 812)]:
        gpk, gsc, g_packed, g_scales = _weights(rng, n, k, group)
        upk, usc, u_packed, u_scales = _weights(rng, n, k, group)
        x = bf16_normal(rng, (m, k))
        y, names = _traced(lambda: ops.w4_matmul_gate_up(to_gpu_bf16(x), g_packed, g_scales, u_packed, u_scales,
                                                         group))
        assert names == [SHORT_PAIRED[want]], names
        want_gate = round_bf16(oracle.w4_matmul(x, gpk, gsc, group))
        expected = oracle.w4_matmul(x, upk, usc, group, gate=want_gate)
        assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=2.0, atol=_atol(expected))
    x = to_gpu_bf16(bf16_normal(rng, (16, 576)))
    gpk, gsc, g_packed, g_scales = _weights(rng, 4864, 576)
    _, names = _traced(lambda: ops.w4_matmul_gate_up(x, g_packed, g_scales, g_packed, g_scales, 64))
    assert not _lds(names), names


@pytest.mark.parametrize("tile", [813, 814])
@pytest.mark.parametrize("m,group,k,splits,epilogue", [
    (1, 64, 640, 3, "bias"),         # 10 steps in slices of 4, 4, 2
    (50, 32, 2240, 0, "residual"),   # automatic split count, 35 steps
    (128, 64, 4864, 0, "norm"),      # the 0.5B down shape's K, residual + next RMSNorm
    (200, 128, 1536, 1, "none"),     # one slice: partials + reduce all the same
    (128, 64, 1152, 7, "residual"),  # 18 steps in slices of 3
])
def test_lds_split_short_prompt_tiles(tile, m, group, k, splits, epilogue):
    """Tiles 813 / 814 (the single form's split-K partials on 128 x 32 / 128 x 64 blocks
    of 4 waves) summed and finished by the reduce launches: ragged rows (1-200), N = 608
    (19 / 9.5 column blocks), slices that leave every kind of last slice, groups 32-128,
    the bias, residual and residual + RMSNorm epilogues, within one bf16 ulp of the
    oracle."""

    ops = _ops()
    n = 608
    rng = np.random.default_rng(770 + m + k + splits + len(epilogue))
    packed, scales, gp, gs = _weights(rng, n, k, group)
    x = bf16_normal(rng, (m, k))
    gx = to_gpu_bf16(x)
    ws = torch.empty(max(ops.gemm_workspace_bytes(m, n, k, tile, splits), 16), dtype=torch.uint8, device="cuda")
    if epilogue == "norm":
        residual = bf16_normal(rng, (m, n), 2.0)
        weight = bf16_normal(rng, (n,), 0.1) + 1.0
        (y, normed), names = _traced(lambda: ops.matmul_residual_norm(
            gx, gp, gs, group, to_gpu_bf16(residual), to_gpu_bf16(weight), 1e-6, tile=tile, splits=splits,
            workspace=ws))
        assert names == [SHORT_SPLIT[tile], "aoto_w4_gemm_reduce_norm"], names
        expected = oracle.w4_matmul(x, packed, scales, group, residual=residual)
        assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))
        want_norm = oracle.rms_norm(from_gpu_bf16(y), round_bf16(weight), 1e-6)
        assert_bf16_parity(from_gpu_bf16(normed), want_norm, max_ulp=1.0)
        return
    kwargs = {}
    if epilogue == "bias":
        kwargs["bias"] = bf16_normal(rng, (n,), 0.5)
    elif epilogue == "residual":
        kwargs["residual"] = bf16_normal(rng, (m, n), 2.0)
    gkw = {key: to_gpu_bf16(value) for key, value in kwargs.items()}
    y, names = _traced(lambda: ops.w4_matmul(gx, gp, gs, group, tile=tile, splits=splits, workspace=ws, **gkw))
    assert names == [SHORT_SPLIT[tile], "aoto_w4_gemm_reduce"], names
    expected = oracle.w4_matmul(x, packed, scales, group, **kwargs)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))


def test_lds_split_is_the_automatic_plan_for_short_long_k_projections():
    """At 128 rows a 0.5B down projection (4864 -> 896) takes tile 813 split eight ways by
    itself and an 8B o projection (4096 -> 4096) tile 814; K = 896 stays on the 16x16
    kernel; each within one ulp of the oracle."""

    ops = _ops()
    rng = np.random.default_rng(780)
    for n, k, want in [(896, 4864, 813), (4096, 4096, 814), (896, 896, None)]:
        m = 128
        assert ops.lds_plan(m, n, k) == want
        packed, scales, gp, gs = _weights(rng, n, k)
        x = bf16_normal(rng, (m, k))
        residual = bf16_normal(rng, (m, n), 2.0)
        y, names = _traced(lambda: ops.w4_matmul(to_gpu_bf16(x), gp, gs, 64, residual=to_gpu_bf16(residual)))
        if want is None:
            assert not _lds(names) and not any(name.endswith("_split") for name in names), names
        else:
            assert names == [SHORT_SPLIT[want], "aoto_w4_gemm_reduce"], names
        expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual)
        assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))


def test_lds_gemm_in_place_residual():
    ops = _ops()
    m, n, k = 512, 512, 1024
    rng = np.random.default_rng(730)
    packed, scales, gp, gs = _weights(rng, n, k)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    buf = to_gpu_bf16(residual)
    ops.w4_matmul(to_gpu_bf16(x), gp, gs, 64, residual=buf, out=buf, tile=822)
    expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual)
    assert_bf16_parity(from_gpu_bf16(buf), expected, max_ulp=1.0, atol=_atol(expected))


@pytest.mark.timeout(300)
def test_lds_gemm_is_the_automatic_plan_at_2048_rows():
    """At 2048 rows an o-shaped projection (N = 4096: 32 x 8 = 256 blocks, one full round)
    and a paired gate/up of N = 4096 (512 blocks) take the dequant-once kernel by
    themselves; the results match the oracle and the wide kernel."""

    ops = _ops()
    m, n, k = 2048, 4096, 1024
    assert ops.lds_plan(m, n, k) == ops.LDS_TILE and ops.lds_plan(m, n, k, paired=True) == ops.LDS_PAIRED_TILE
    rng = np.random.default_rng(740)
    packed, scales, gp, gs = _weights(rng, n, k)
    x = bf16_normal(rng, (m, k))
    residual = bf16_normal(rng, (m, n), 2.0)
    gx = to_gpu_bf16(x)
    y, names = _traced(lambda: ops.w4_matmul(gx, gp, gs, 64, residual=to_gpu_bf16(residual)))
    assert names == ["aoto_w4_gemm_d8w2x2_b0_r1"], names
    expected = oracle.w4_matmul(x, packed, scales, 64, residual=residual)
    assert_bf16_parity(from_gpu_bf16(y), expected, max_ulp=1.0, atol=_atol(expected))
    wide = ops.w4_matmul(gx, gp, gs, 64, residual=to_gpu_bf16(residual), tile=441, splits=1)
    assert_bf16_parity(from_gpu_bf16(y), from_gpu_bf16(wide), max_ulp=1.0, atol=_atol(expected))

    upk, usc, u_packed, u_scales = _weights(rng, n, k)
    p, names = _traced(lambda: ops.w4_matmul_gate_up(gx, gp, gs, u_packed, u_scales, 64))
    assert names == ["aoto_w4_gemm_d8w2x1_paired"], names
    want_gate = round_bf16(oracle.w4_matmul(x, packed, scales, 64))
    expected = oracle.w4_matmul(x, upk, usc, 64, gate=want_gate)
    # Over 8.4M outputs the silu_mul product's tail reaches 3 ulp on either kernel: where
    # the f32 gate sum rounds to the neighbouring bf16 (another summation order), silu's
    # slope carries that ulp into the product, which adds its own rounding.
    wide = ops.w4_matmul_gate_up(gx, gp, gs, u_packed, u_scales, 64, tile=241, splits=1)
    wide_stats = assert_bf16_parity(from_gpu_bf16(wide), expected, max_ulp=3.0)
    stats = assert_bf16_parity(from_gpu_bf16(p), expected, max_ulp=3.0)
    print(f"paired 2048 x {n} x {k}: dequant-once {stats}, wide {wide_stats}")


def test_lds_gemms_replay_in_a_graph_like_eager():
    """A captured bias, residual (in place), paired and split sequence on tiles 822 / 821 /
    811 / 813 replays three times, with eager work and synchronizations between,
    bit-identical to its eager pass each time."""

    ops = _ops()
    m, n, k = 512, 640, 768
    rng = np.random.default_rng(750)
    weights = [_weights(rng, n, k)[2:] for _ in range(3)]
    x = to_gpu_bf16(bf16_normal(rng, (m, k)))
    bias = to_gpu_bf16(bf16_normal(rng, (n,), 0.5))
    residual0 = to_gpu_bf16(bf16_normal(rng, (m, n), 2.0))
    outs = {name: torch.empty((m, n), dtype=torch.bfloat16, device="cuda") for name in ("bias", "paired")}
    residual = residual0.clone()

    outs["short"] = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    outs["split"] = torch.empty((m, n), dtype=torch.bfloat16, device="cuda")
    ws = torch.empty(ops.gemm_workspace_bytes(m, n, k, 813, 3), dtype=torch.uint8, device="cuda")

    def body():
        ops.w4_matmul(x, *weights[0], 64, bias=bias, out=outs["bias"], tile=822)
        ops.w4_matmul_gate_up(x, *weights[1], *weights[2], 64, out=outs["paired"], tile=821)
        ops.w4_matmul_gate_up(x, *weights[1], *weights[2], 64, out=outs["short"], tile=811)
        ops.w4_matmul(x, *weights[2], 64, bias=bias, out=outs["split"], tile=813, splits=3, workspace=ws)
        ops.w4_matmul(x, *weights[0], 64, residual=residual, out=residual, tile=822)

    _, names = _traced(body)
    assert len(_lds(names)) == 5, names
    torch.cuda.synchronize()
    eager = {name: t.clone() for name, t in outs.items()}
    eager["residual"] = residual.clone()
    residual.copy_(residual0)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        body()
    torch.cuda.synchronize()
    for replay in range(3):
        for t in outs.values():
            t.fill_(float("nan"))
        residual.copy_(residual0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        for name, t in outs.items():
            assert torch.equal(t, eager[name]), (replay, name)
        assert torch.equal(residual, eager["residual"]), replay
        ops.w4_matmul(x, *weights[2], 64, out=outs["bias"], tile=822)  # eager work between replays
        torch.cuda.synchronize()


def test_lds_tiles_refuse_what_they_cannot_run():
    from aotolith_amd._lib import HipKernelError, UnsupportedShape

    ops = _ops()
    rng = np.random.default_rng(760)
    _, _, gp, gs = _weights(rng, 256, 576)  # 9 groups of 64 per row: odd
    x = to_gpu_bf16(bf16_normal(rng, (64, 576)))
    with pytest.raises(UnsupportedShape):
        ops.w4_matmul(x, gp, gs, 64, tile=822)
    _, _, gp, gs = _weights(rng, 256, 512)
    x = to_gpu_bf16(bf16_normal(rng, (64, 512)))
    with pytest.raises(HipKernelError, match="tile 822"):
        ops.w4_matmul(x, gp, gs, 64, tile=822, gate=to_gpu_bf16(bf16_normal(rng, (64, 256))))
    with pytest.raises(HipKernelError, match="tile 821"):
        ops.w4_matmul(x, gp, gs, 64, tile=821)
    with pytest.raises(HipKernelError, match="tile 811"):
        ops.w4_matmul(x, gp, gs, 64, tile=811)
    with pytest.raises(HipKernelError, match="tile 812"):
        ops.w4_matmul_gate_up(x, gp, gs, gp, gs, 64, tile=812, splits=2)
    with pytest.raises(HipKernelError, match="tile 822"):
        ops.w4_matmul_gate_up(x, gp, gs, gp, gs, 64, tile=822)
    with pytest.raises(HipKernelError, match="tile 813"):
        ops.w4_matmul_gate_up(x, gp, gs, gp, gs, 64, tile=813)
    with pytest.raises(HipKernelError, match="tile 822"):
        ops.w4_matmul(x, gp, gs, 64, tile=822, splits=2)
    packed8, scales8 = pack_weight_bits_bf16(bf16_normal(rng, (256, 512), 0.02), 64, 8)
    with pytest.raises(HipKernelError, match="tile 822"):
        ops.w8_matmul(x, torch.from_numpy(packed8).cuda(), to_gpu_bits(scales8), 64, tile=822)
