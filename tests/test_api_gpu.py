"""GPU tests of the operator and provider API: the reference's GPU contract tests (tests/test_kernels_gpu.py:30-105)
restated for this build, plus the provider seam, the ternary modules and the exact deferred split-K slices.

Bars: the P-part dot against FP64 sum_c acc_c * s_c * alpha from exact integer accumulators, rtol 2e-6 / atol 1e-6;
linear against dense FP64 relative Frobenius error < 2e-2 / 1e-4 / 1e-6 for P = 1 / 2 / 3; PackedLinear < 1e-5;
exact split-K slices + finish bitwise equal to the unsplit GEMM; provider calls bitwise equal to the layer's own.
Integer accumulators come from the pinned CPU oracle (exact int32 sums, the reference test's int64 formula).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from kea_kernels import formats, lowbit
from kea_kernels.binary import bits, configs, hybrid_exact, layer as L, layer_parts, provider
from kea_kernels.binary.kernels import GemmConfig
from kea_kernels.ternary import encoder4, fused_kernels, runtime
from oracle import oracle as O

pytestmark = pytest.mark.gpu

SHAPES = [(1024, 1024), (4096, 1024), (1024, 4096), (3072, 1024)]


def _weights(n, k, seed):
    g = torch.Generator().manual_seed(seed)
    signs = torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8)
    scale = torch.rand(n, generator=g) * 0.02 + 0.001
    return bits.pack_signs(signs), scale.float(), signs


def _exact_epilogue(q, qs, codes, k, scale, parts):
    """FP64 sum_c acc_c * s_c * alpha, acc from the oracle's exact int32 GEMM."""
    acc = O.b1_gemm(q[:parts, :, :].cpu().numpy(), codes.numpy(), k).astype(np.float64)
    s = qs[:parts].cpu().double().numpy()
    y = sum(acc[c] * s[c][:, None] for c in range(parts))
    return torch.from_numpy(y * scale.double().numpy()[None, :])


@pytest.mark.parametrize("parts", [1, 2, 3])
@pytest.mark.parametrize("n,k", SHAPES)
@pytest.mark.parametrize("m", [38, 126, 300])
@torch.inference_mode()
def test_b1_dot_equals_exact_integer_reference(parts, n, k, m):
    codes, scale, _ = _weights(n, k, seed=n + k + m)
    layer = layer_parts.LAYERS[parts].prepare(codes, scale, None, k, "cuda")
    assert layer.fast
    x = torch.randn(m, k, device="cuda")
    q, qs, ldq = L.quantize(x, (0, x.stride(0), x.stride(1), m), m, k)
    y = torch.empty(m, n, device="cuda")
    layer.dot(q[:parts], qs[:parts], ldq, m, y, parts=parts)
    torch.cuda.synchronize()
    ref = _exact_epilogue(q, qs, codes, k, scale, parts)
    torch.testing.assert_close(y.cpu().double(), ref, rtol=2e-6, atol=1e-6)


@pytest.mark.parametrize("parts,tol", [(1, 2e-2), (2, 1e-4), (3, 1e-6)])
@torch.inference_mode()
def test_linear_matches_dense_fp64_within_activation_precision(parts, tol):
    n, k, m = 1024, 4096, 126
    codes, scale, _ = _weights(n, k, seed=7)
    layer = layer_parts.LAYERS[parts].prepare(codes, scale, None, k, "cuda")
    x = torch.randn(2, m // 2, k, device="cuda")
    y = layer.linear(x).cpu().double()
    ref = x.cpu().double() @ bits.dense_weight(codes, scale, k).t()
    err = (y - ref).norm() / ref.norm()
    assert err < tol


@torch.inference_mode()
def test_conv_is_the_transposed_linear():
    n, k, b, t = 256, 512, 2, 37
    codes, scale, _ = _weights(n, k, seed=11)
    bias = torch.randn(n)
    layer = L.Int8MmaLayer.prepare(codes, scale, bias, k, "cuda")
    x = torch.randn(b, k, t, device="cuda")
    yc = layer.conv(x)
    assert yc.shape == (b, n, t)
    yl = layer.linear(x.transpose(1, 2).contiguous())
    assert torch.equal(yc, yl.transpose(1, 2))
    ref = x.transpose(1, 2).cpu().double() @ bits.dense_weight(codes, scale, k).t() + bias.double()
    assert (yc.transpose(1, 2).cpu().double() - ref).norm() / ref.norm() < 1e-6


@pytest.mark.parametrize("parts", [2, 3])
@pytest.mark.parametrize("m,n,k", [(38, 1024, 1024), (38, 1024, 4096), (126, 1024, 4096)])
@torch.inference_mode()
def test_exact_split_k_finish_equals_in_kernel_finish(parts, m, n, k):
    """Deferred integer slices finished by finish_slices are bitwise the unsplit in-kernel epilogue."""
    codes, scale, _ = _weights(n, k, seed=m * n + k)
    bias = torch.randn(n) * 0.1
    layer = layer_parts.LAYERS[parts].prepare(codes, scale, bias, k, "cuda")
    xx = torch.randn(1, m, k, device="cuda")
    q, qs = layer_parts.m1_quantize_parts(xx, parts)
    y = torch.empty(1, m, n, device="cuda")
    layer.dot(q, qs, k, m, y.view(m, n), config=GemmConfig(configs.choose(m, n, k, parts).tile, 1), parts=parts)
    auto = hybrid_exact.choose_exact_deferred(m, n, k, parts)
    quads = -(-(-(-k // 128)) // 4)  # groups of four native words along K: the most slices a call can have
    for cfg in [c for c in (auto, GemmConfig(4, 2), GemmConfig(1, 4), GemmConfig(4, 8)) if c and c.split <= quads]:
        slices = torch.empty(cfg.split, parts, m, n, device="cuda", dtype=torch.int32)
        hybrid_exact.dot_slices(layer, q, qs, k, m, slices, cfg)
        value = hybrid_exact.ExactDeferredProjection(slices, layer.scale, layer.bias, cfg.split, (1, m, n), qs)
        exact = value.finish()
        acc = torch.empty(parts, m, n, device="cuda", dtype=torch.int32)
        hybrid_exact.finish_slices(value, None, acc)
        torch.cuda.synchronize()
        assert torch.equal(exact, y), cfg
        ref_acc = O.b1_gemm(q.cpu().numpy(), codes.numpy(), k)
        assert np.array_equal(acc.cpu().numpy(), ref_acc), cfg
    with pytest.raises(RuntimeError, match="integer slices"):
        value.partial


@torch.inference_mode()
def test_project_deferred_matches_project():
    n, k, m = 1024, 4096, 38
    codes, scale, _ = _weights(n, k, seed=5)
    layer = L.Int8MmaLayer.prepare(codes, scale, None, k, "cuda")
    x = torch.randn(1, m, k, device="cuda")
    value = hybrid_exact.project_deferred(layer, x, config=GemmConfig(4, 4))
    assert isinstance(value, hybrid_exact.ExactDeferredProjection)
    assert torch.equal(value.finish(), layer.project(x))


@torch.inference_mode()
def test_slices_entry_points_reject_bad_arguments():
    codes, scale, _ = _weights(64, 256, seed=1)
    layer = L.Int8MmaLayer.prepare(codes, scale, None, 256, "cuda")
    q = torch.zeros(3, 8, 256, device="cuda", dtype=torch.int8)
    qs = torch.ones(3, 8, device="cuda")
    with pytest.raises(ValueError, match="slices"):
        hybrid_exact.dot_slices(layer, q, qs, 256, 8, torch.empty(2, 3, 8, 32, device="cuda", dtype=torch.int32))
    with pytest.raises(ValueError, match="split"):  # 256 = one group of four words: no second slice exists
        hybrid_exact.dot_slices(layer, q, qs, 256, 8, torch.empty(2, 3, 8, 64, device="cuda", dtype=torch.int32))


@pytest.mark.parametrize("mode,parts", [("bf16x3", 3), ("x2", 2), ("x1", 1)])
@torch.inference_mode()
def test_ternary_packed_linear_matches_dense_fp64(mode, parts):
    n, k, m = 1024, 1024, 64
    g = torch.Generator().manual_seed(3)
    codes = torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8)
    scale = torch.rand(n, generator=g) * 0.02 + 0.001
    module = runtime.PackedLinear(formats.pack_ternary(codes), scale.float(), k, mode=mode).cuda()
    x = torch.randn(m, k, device="cuda")
    y = module(x).cpu().double()
    ref = x.cpu().double() @ (codes.double() * scale.double()[:, None]).t()
    tol = {3: 1e-5, 2: 1e-4, 1: 2e-2}[parts]
    assert (y - ref).norm() / ref.norm() < tol


@torch.inference_mode()
def test_ternary_provider_fused_norm_silu_and_conv():
    n, k, b, t = 512, 1024, 2, 40
    g = torch.Generator().manual_seed(9)
    codes = torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8)
    scale = torch.rand(n, generator=g) * 0.02 + 0.001
    bias = torch.randn(n, generator=g)
    mod = runtime.PackedPointwiseConv1d(formats.pack_ternary(codes), scale, k, bias).cuda()
    norm = torch.nn.LayerNorm(k)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(k, generator=g) + 0.5)
        norm.bias.copy_(torch.randn(k, generator=g) * 0.1)
    dnorm = torch.nn.LayerNorm(k).cuda()
    dnorm.load_state_dict(norm.state_dict())
    proj = encoder4.ExpandedProjection()
    assert proj.bytes == 0
    x = torch.randn(b, k, t, device="cuda")
    y = proj(x, mod, conv=True, components=3, activation="silu", norm=dnorm, input_activation="silu")
    assert y.shape == (b, n, t)
    z = torch.nn.functional.silu(norm(x.cpu().transpose(1, 2)).double())
    ref = torch.nn.functional.silu(z @ (codes.double() * scale.double()[:, None]).t() + bias.double())
    assert (y.transpose(1, 2).cpu().double() - ref).norm() / ref.norm() < 1e-5
    same = fused_kernels.int8_matmul(x, mod, True, 3, "silu", dnorm, None, "silu")
    assert torch.equal(y, same)


@torch.inference_mode()
def test_binary_provider_table_and_part_count_on_gpu():
    n, k = 256, 1024
    layers = {}
    for i, name in enumerate(["b.0.self_attn.linear_q", "b.0.self_attn.linear_k", "b.0.self_attn.linear_v",
                              "b.0.feed_forward1.linear1"]):
        codes, scale, _ = _weights(n * (1 + 3 * ("linear1" in name)), k, seed=20 + i)
        layers[name] = (codes, scale, torch.randn(codes.shape[0]) if "linear1" in name else None, "linear", k)
    table, modules = provider.prepare_table(layers, layer_parts.Int8MmaPartsLayer, "cuda")
    proj = provider.BinaryProjection(table)
    x = torch.randn(2, 19, k, device="cuda")
    q, kk, v = (modules[f"b.0.self_attn.{s}"] for s in provider.QKV)
    fused = torch.cat([q.packed_t, kk.packed_t, v.packed_t], 1)
    handle = type("H", (), {"packed_t": fused})()
    y = proj(x, handle)
    assert y.shape == (2, 19, 3 * n)
    assert torch.equal(proj(x, kk), y[..., n:2 * n])
    qkv_layer = table.segments[0].layer
    assert torch.equal(y, qkv_layer.project(x))
    ff = modules["b.0.feed_forward1.linear1"]
    ff_codes, ff_scale, ff_bias = layers["b.0.feed_forward1.linear1"][:3]
    ref = x.cpu().double() @ bits.dense_weight(ff_codes, ff_scale, k).t() + ff_bias.double()
    for parts, tol in [(1, 2e-2), (2, 1e-4), (3, 1e-6)]:
        yp = provider.PartCount(proj, parts)(x, ff, components=3)
        assert (yp.cpu().double() - ref).norm() / ref.norm() < tol
    assert table.weight_bytes() == sum(s.layer.weight_bytes() for s in table.segments)


def test_layer_errors_match_the_reference_contract():
    codes, scale, _ = _weights(64, 128, seed=2)
    with pytest.raises(ValueError, match="GPU"):
        L.Int8MmaLayer.prepare(codes, scale, None, 128, "cpu")
    layer = L.Int8MmaLayer.prepare(codes, scale, None, 128, "cuda")
    with pytest.raises(ValueError, match="input"):
        layer.linear(torch.randn(4, 100, device="cuda"))
    with pytest.raises(ValueError, match="FP32"):
        layer.linear(torch.randn(4, 128, device="cuda", dtype=torch.float64))
    q = torch.zeros(3, 4, 136, device="cuda", dtype=torch.int8)[:, :, 8:]
    with pytest.raises(ValueError, match="aligned"):
        layer.dot(q, torch.ones(3, 4, device="cuda"), 128, 4, torch.empty(4, 64, device="cuda"))
    with pytest.raises(RuntimeError, match="inference only"):
        layer.linear(torch.randn(4, 128, device="cuda", requires_grad=True))
    layer.linear(torch.randn(4, 128, device="cuda"))  # a layout the layer now launches without its checks
    with pytest.raises(RuntimeError, match="inference only"):
        layer.linear(torch.randn(4, 128, device="cuda", requires_grad=True))
    with pytest.raises(ValueError, match="input on"):
        layer.linear(torch.randn(4, 128))


@torch.inference_mode()
def test_output_dtypes_through_the_layer():
    n, k, m = 512, 1024, 64
    codes, scale, _ = _weights(n, k, seed=4)
    layer = L.Int8MmaLayer.prepare(codes, scale, None, k, "cuda")
    x = torch.randn(m, k, device="cuda")
    y32 = layer.linear(x)
    for dt in (torch.float16, torch.bfloat16):
        y = layer.linear(x, out_dtype=dt)
        assert y.dtype == dt and torch.equal(y, y32.to(dt))


@torch.inference_mode()
def test_quantize_zero_rows_and_lowbit_zero_m():
    x = torch.empty(0, 64, device="cuda")
    q, qs, ldq = lowbit.quantize(x, (0, 64, 1, 1), 0, 64, 3)
    assert q.shape == (3, 0, 64) and qs.shape == (3, 0)


# --- launches resolved once per call layout (lowbit.Launches) ----------------------------------------------------------

def _uncached(layer, x, rows, m, parts, y, *, silu=False, norm=None, input_activation=""):
    """The checked, uncached path: quantize() then gemm() on the layer's weights."""
    q, qs, _ = lowbit.quantize(x, rows, m, layer.in_features, parts, norm=norm, input_activation=input_activation)
    lowbit.gemm(layer.WBITS, q, qs, layer.words, layer.out_features, layer.in_features, layer.scale, layer.bias, y,
                None, m=m, silu=silu)


@pytest.mark.parametrize("parts", [1, 3])
@torch.inference_mode()
def test_cached_launches_are_bitwise_the_checked_path(parts):
    """linear (2-D, 3-D, strided, f16 input), conv and project (LayerNorm, input SiLU, SiLU epilogue) through the
    layer's cached launches: every call, including repeated calls of one layout on new buffers, gives the checked
    path's bits; a layout is resolved once."""
    n, k = 300, 1024
    codes, scale, _ = _weights(n, k, seed=parts + 40)
    bias = torch.randn(n, generator=torch.Generator().manual_seed(41))
    layer = layer_parts.LAYERS[parts].prepare(codes, scale, bias, k, "cuda")
    g = torch.Generator().manual_seed(parts)
    for step in range(3):  # the same layouts again, on new inputs
        xs = [torch.randn(37, k, generator=g).cuda(),
              torch.randn(2, 19, k, generator=g).cuda(),
              torch.randn(70, 2 * k, generator=g).cuda()[:, ::2],
              torch.randn(16, k, generator=g).cuda().half(),
              torch.randn(2, 3, 19, k, generator=g).cuda().transpose(0, 1)]  # its 3-D view is a copy
        for x in xs:
            got = layer.linear(x)
            assert got.shape == (*x.shape[:-1], n)
            x3 = x.reshape(-1, x.shape[-2], x.shape[-1]) if x.dim() >= 3 else x
            m = got.numel() // n
            rows = (x3.stride(0), x3.stride(1), x3.stride(2), x3.shape[1]) if x.dim() >= 3 else \
                (0, x.stride(0), x.stride(1), m)
            want = torch.empty(m, n, device="cuda")
            _uncached(layer, x3, rows, m, parts, want)
            torch.cuda.synchronize()
            assert torch.equal(got.reshape(m, n).view(torch.int32), want.view(torch.int32)), (step, tuple(x.shape))
        xc = torch.randn(3, k, 25, generator=g).cuda()
        got = layer.conv(xc)
        want = torch.empty(3 * 25, n, device="cuda")
        _uncached(layer, xc, (xc.stride(0), xc.stride(2), xc.stride(1), 25), 75, parts, want)
        assert torch.equal(got.transpose(1, 2).reshape(75, n).view(torch.int32), want.view(torch.int32))
        norm = torch.nn.LayerNorm(k).cuda()
        with torch.no_grad():
            norm.weight.copy_(torch.rand(k, generator=g) + 0.5)
            norm.bias.copy_(torch.randn(k, generator=g) * 0.1)
        xp = torch.randn(2, 33, k, generator=g).cuda()
        got = layer.project(xp, components=parts, activation="silu", norm=norm, input_activation="silu")
        want = torch.empty(66, n, device="cuda")
        _uncached(layer, xp, (xp.stride(0), xp.stride(1), xp.stride(2), 33), 66, parts, want, silu=True, norm=norm,
                  input_activation="silu")
        torch.cuda.synchronize()
        assert torch.equal(got.reshape(66, n).view(torch.int32), want.view(torch.int32))
    # one entry per layout, not per call: 5 linear layouts, conv, and project once per LayerNorm (a new one per step)
    assert 1 <= len(layer.launches) <= 9
    # repeated linear / conv calls skip the checks (a kept entry per input layout), except where x's 3-D view copies
    assert layer.launches.recall(("linear", xs[0].shape, xs[0].stride(), xs[0].dtype, xs[0].device, torch.float32))
    assert layer.launches.recall(("conv", xc.shape, xc.stride(), xc.dtype, xc.device, torch.float32))
    assert not layer.launches.recall(("linear", xs[4].shape, xs[4].stride(), xs[4].dtype, xs[4].device,
                                      torch.float32))


@pytest.mark.parametrize("seed", [21, 22, 23])
@torch.inference_mode()
def test_seeded_random_operator_calls_equal_the_checked_path(seed):
    """Int8MmaPartsLayer.linear / .conv on random shapes (1-, 2-, 3- and 4-D inputs, column-sliced rows, f32 / f16
    input, f32 / f16 / bf16 output, 1 to 3 parts, with and without bias), each layout called twice (the second call
    takes the kept launch): every output bitwise the checked quantize() + gemm() on the same rows."""
    rng = np.random.default_rng(seed)
    dtypes = [torch.float32, torch.float16, torch.bfloat16]
    for i in range(8):
        parts, n, k = int(rng.integers(1, 4)), int(rng.integers(1, 700)), int(rng.integers(1, 2100))
        codes, scale, _ = _weights(n, k, seed=seed * 100 + i)
        bias = torch.randn(n, generator=torch.Generator().manual_seed(i)) if rng.integers(0, 2) else None
        layer = layer_parts.LAYERS[parts].prepare(codes, scale, bias, k, "cuda")
        out_dtype = dtypes[int(rng.integers(0, 3))]
        x_dtype = [torch.float32, torch.float16][int(rng.integers(0, 2))]
        dims, conv = int(rng.integers(1, 5)), bool(rng.integers(0, 4) == 0)
        lead = [int(rng.integers(1, 40)) for _ in range(dims - 1)]
        for _ in range(2):
            g = torch.Generator().manual_seed(int(rng.integers(0, 1 << 30)))
            if conv:
                b, t = int(rng.integers(1, 4)), int(rng.integers(1, 60))
                x = torch.randn(b, k, t, generator=g).to("cuda", x_dtype)
                got = layer.conv(x, out_dtype=out_dtype).transpose(1, 2).reshape(b * t, n)
                xr, rows, m = x, (x.stride(0), x.stride(2), x.stride(1), t), b * t
            else:
                wide = bool(rng.integers(0, 2))  # rows that are a column slice of a wider tensor
                full = torch.randn(*lead, k + (7 if wide else 0), generator=g).to("cuda", x_dtype)
                x = full[..., 3:3 + k] if wide else full
                got = layer.linear(x, out_dtype=out_dtype)
                assert got.shape == (*lead, n)
                m = got.numel() // n
                got = got.reshape(m, n)
                xr = x.reshape(-1, x.shape[-2], x.shape[-1]) if x.dim() >= 3 else x
                rows = ((xr.stride(0), xr.stride(1), xr.stride(2), xr.shape[1]) if x.dim() >= 3 else
                        (0, x.stride(0), x.stride(1), m) if x.dim() == 2 else (0, 0, x.stride(0), 1))
            want = torch.empty(m, n, device="cuda", dtype=out_dtype)
            q, qs, _ = lowbit.quantize(xr, rows, m, k, parts)
            lowbit.gemm(1, q, qs, layer.words, n, k, layer.scale, layer.bias, want, None, m=m)
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16 if out_dtype != torch.float32 else torch.int32),
                               want.view(torch.int16 if out_dtype != torch.float32 else torch.int32)), (seed, i)


@torch.inference_mode()
def test_cached_dot_split_k_workspace_and_acc_out():
    """dot through the cached plan: a split-K configuration (its workspace allocated per call) and raw
    accumulators, bitwise the checked gemm() on the same parts; a layer whose weights are replaced gets new plans."""
    n, k, m = 256, 4096, 64
    codes, scale, _ = _weights(n, k, seed=77)
    layer = layer_parts.LAYERS[2].prepare(codes, scale, None, k, "cuda")
    x = torch.randn(m, k, device="cuda")
    q, qs, ldq = L.quantize(x, (0, x.stride(0), x.stride(1), m), m, k, parts=2)
    cfg = GemmConfig(tile=1, split=4)
    for _ in range(2):
        y = torch.empty(m, n, device="cuda")
        acc = torch.empty(2, m, n, dtype=torch.int32, device="cuda")
        layer.dot(q, qs, ldq, m, y, config=cfg, acc_out=acc)
        y_ref = torch.empty_like(y)
        acc_ref = torch.empty_like(acc)
        lowbit.gemm(1, q, qs, layer.words, n, k, layer.scale, None, y_ref, acc_ref, m=m, config=cfg)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int32), y_ref.view(torch.int32)) and torch.equal(acc, acc_ref)
    assert np.array_equal(acc.cpu().numpy(), O.b1_gemm(q.cpu().numpy(), codes.numpy(), k))
    old = layer.launches
    layer.scale = layer.scale * 2
    assert layer.launches is not old


@pytest.mark.parametrize("parts,tile,split", [(1, 1, 4), (3, 1, 4), (2, 13, 2), (3, 23, 4)])
@torch.inference_mode()
def test_projection_plan_with_split_k_slices_in_its_workspace(parts, tile, split):
    """A projection plan whose GEMM splits K (LDS-ring tile 16x64 and wave-split tiles 16x128 k/4, 16x16 k/4): the
    int32 slices sit in the one workspace after the int8 parts and their scales; repeated calls on new inputs give
    the bits of the checked quantize() + gemm() with the same configuration, f16 output."""
    n, k, m = 256, 4096, 50
    codes, scale, _ = _weights(n, k, seed=90 + parts)
    layer = layer_parts.LAYERS[parts].prepare(codes, scale, None, k, "cuda")
    cfg = GemmConfig(tile=tile, split=split)
    g = torch.Generator().manual_seed(parts)
    for _ in range(3):
        x = torch.randn(m, k, generator=g).cuda()
        rows = (0, x.stride(0), x.stride(1), m)
        y = torch.empty(m, n, device="cuda", dtype=torch.float16)
        e = layer.launches.project(x, rows, m, parts, y, config=cfg)
        assert e and e.need >= parts * m * k + split * parts * m * n * 4
        q, qs, _ = lowbit.quantize(x, rows, m, k, parts)
        want = torch.empty_like(y)
        lowbit.gemm(1, q, qs, layer.words, n, k, layer.scale, None, want, None, m=m, config=cfg)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), want.view(torch.int16))
    assert len(layer.launches) == 1


@torch.inference_mode()
def test_ternary_int8_matmul_cached_equals_checked_path():
    n, k = 200, 640
    g = torch.Generator().manual_seed(5)
    vals = torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8)
    packed = formats.pack_ternary(vals)
    mod = runtime.PackedLinear(packed, torch.rand(n, generator=g) * 0.05 + 0.01, k, torch.randn(n, generator=g),
                               mode="fp16").cuda()
    for _ in range(2):
        x = torch.randn(3, 21, k, generator=g).cuda()
        got = fused_kernels.int8_matmul(x, mod, components=2, activation="silu")
        q, qs, _ = lowbit.quantize(x, (x.stride(0), x.stride(1), x.stride(2), 21), 63, k, 2)
        want = torch.empty(63, n, device="cuda")
        lowbit.gemm(2, q, qs, runtime.native_words(mod), n, k, mod.scale, mod.bias, want, None, silu=True)
        torch.cuda.synchronize()
        assert torch.equal(got.reshape(63, n).view(torch.int32), want.view(torch.int32))
