"""The synthetic FastConformer encoder: host-side pieces on the CPU, the quantized encoder
against its FP32 dense twin on the GPU (relative Frobenius error bars per part count), and graph replay = eager."""
from __future__ import annotations

import copy
import ctypes
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from kea_kernels import _hip, encoder as E
from oracle import oracle as O


def test_rel_shift_matches_the_relative_index():
    """rel_shift(bd)[i, j] must be the score of query i against relative position i - j, i.e. column (T-1) - (i-j)
    of the [2T-1] relative axis (positions T-1 .. -(T-1))."""
    t = 7
    x = torch.arange(t * (2 * t - 1), dtype=torch.float32).view(1, 1, t, 2 * t - 1)
    y = E.rel_shift(x)
    for i in range(t):
        for j in range(t):
            assert y[0, 0, i, j] == x[0, 0, i, (t - 1) - (i - j)]


def test_relative_positions_closed_form():
    cfg = E.EncoderConfig(d_model=8)
    pe = E.relative_positions(cfg, 3, "cpu")
    assert pe.shape == (5, 8)
    for row, pos in enumerate([2, 1, 0, -1, -2]):
        for i in range(4):
            w = math.exp(-(2 * i) * math.log(10000.0) / 8)
            assert abs(float(pe[row, 2 * i]) - math.sin(pos * w)) < 1e-6
            assert abs(float(pe[row, 2 * i + 1]) - math.cos(pos * w)) < 1e-6


def test_mel_filterbank_is_triangular_and_area_normalised():
    cfg = E.EncoderConfig()
    fb = E.mel_filterbank(cfg)
    assert fb.shape == (128, 257) and (fb >= 0).all()
    peaks = fb.argmax(axis=1)
    assert (np.diff(peaks) >= 0).all()
    # Slaney normalisation: height 2 / bandwidth gives every triangle unit area in Hz (sampled at FFT bins)
    hz = np.linspace(0, cfg.sample_rate / 2, 257)
    area = (fb * (hz[1] - hz[0])).sum(axis=1)
    assert ((area[48:] > 0.9) & (area[48:] < 1.12)).all()  # wide filters: sampled area close to 1


def test_lengths_and_batchnorm_fold():
    cfg = E.EncoderConfig(layers=1)
    assert E.frames_for(cfg, 160000) == 1000 and E.encoded_length(1000) == 125
    w = E.synthetic_weights(cfg, seed=3)
    enc = E.FastConformerEncoder(w, cfg, "cpu", dense=True)
    pre = "encoder.layers.0.conv."
    x = torch.randn(2, cfg.d_model, 20)
    bn = torch.nn.BatchNorm1d(cfg.d_model, eps=cfg.eps).eval()
    bn.weight.data, bn.bias.data = w[pre + "batch_norm.weight"], w[pre + "batch_norm.bias"]
    bn.running_mean, bn.running_var = w[pre + "batch_norm.running_mean"], w[pre + "batch_norm.running_var"]
    ref = bn(F.conv1d(x, w[pre + "depthwise_conv.weight"], padding=4, groups=cfg.d_model))
    got = F.conv1d(x, enc.layers[0]["dw_w"], enc.layers[0]["dw_b"], padding=4, groups=cfg.d_model)
    torch.testing.assert_close(got, ref, rtol=1e-5, atol=1e-5)


def test_dense_encoder_runs_on_cpu():
    cfg = E.EncoderConfig(layers=2)
    enc = E.FastConformerEncoder(E.synthetic_weights(cfg, seed=1), cfg, "cpu", dense=True)
    out = enc(torch.randn(2, 160000, generator=torch.Generator().manual_seed(0)))
    assert out.shape == (2, 125, 1024) and torch.isfinite(out).all()
    assert 0.5 < float(out.std()) < 2.0  # LayerNorm output


@pytest.mark.gpu
@pytest.mark.parametrize("parts,tol", [(1, 5e-2), (2, 5e-4), (3, 5e-6)])
@torch.inference_mode()
def test_quantized_encoder_matches_dense_fp32(parts, tol):
    """4 layers, batch 2: the int8-activation encoder against the same weights as FP32 dense matmuls. The bars are
    the per-layer precision of P int8 parts (the reference's P-dependent linear bars 2e-2 / 1e-4 / 1e-6,
    tests/test_kernels_gpu.py:47-57) widened for four layers of error propagation."""
    cfg = E.EncoderConfig(layers=4)
    w = E.synthetic_weights(cfg, seed=11)
    audio = torch.randn(2, 160000, generator=torch.Generator().manual_seed(12)).cuda()
    quant = E.FastConformerEncoder(w, cfg, "cuda", parts=parts)(audio)
    dense = E.FastConformerEncoder(w, cfg, "cuda", dense=True)(audio)
    rel = float((quant.double() - dense.double()).norm() / dense.double().norm())
    assert rel < tol, rel


@pytest.fixture(scope="module")
def config5_weights():
    """The 24-layer synthetic model of BASELINE.json config 5 (random init, seed 5 as bench.py uses)."""
    cfg = E.EncoderConfig()
    return cfg, E.synthetic_weights(cfg, seed=5)


@pytest.mark.gpu
@pytest.mark.parametrize("parts,tol", [(1, 5e-2), (3, 5e-6)])
@torch.inference_mode()
def test_config5_full_encoder_matches_dense_fp32(config5_weights, parts, tol):
    """Config 5 at its workload: 10 s of 16 kHz noise -> log-mel (1000 frames) -> 8x subsampling (125 frames) -> 24
    FastConformer layers, batch 1 and batch 8, every linear 1-bit with P int8 activation parts, run as the HIP graph
    the benchmark times. Bar: relative Frobenius error against the same model with FP32 dense linears. One int8
    part carries ~2^-8 relative error per linear (the reference's one-part linear bar is 2e-2,
    tests/test_kernels_gpu.py:47-57); through 24 residual layers the measured error is 3.0-3.2e-2, so the bar is
    5e-2. Three parts carry ~2^-24 per linear, at the FP32 rounding of the dense twin itself (measured 7-10e-7): the
    bar is 5e-6."""
    cfg, w = config5_weights
    assert cfg.layers == 24 and cfg.d_model == 1024
    dense = E.FastConformerEncoder(w, cfg, "cuda", dense=True)
    quant = E.FastConformerEncoder(w, cfg, "cuda", parts=parts)
    for batch in (1, 8):
        audio = torch.randn(batch, 160000, generator=torch.Generator().manual_seed(5 + batch)).cuda()
        graph = E.EncoderGraph(quant, batch, 160000)
        got = graph(audio).clone()
        ref = dense(audio)
        torch.cuda.synchronize()
        assert got.shape == ref.shape == (batch, 125, 1024)
        assert torch.isfinite(got).all()
        rel = float((got.double() - ref.double()).norm() / ref.double().norm())
        print(f"config5 parts={parts} batch={batch}: rel_err_vs_dense_fp32 = {rel:.3e}", flush=True)
        assert rel < tol, (batch, rel)
        del graph


@pytest.mark.gpu
@torch.inference_mode()
def test_encoder_graph_replays_equal_eager():
    cfg = E.EncoderConfig(layers=3)
    enc = E.FastConformerEncoder(E.synthetic_weights(cfg, seed=4), cfg, "cuda", parts=1)
    audio = torch.randn(1, 48000, generator=torch.Generator().manual_seed(5)).cuda()
    eager = enc(audio)
    graph = E.EncoderGraph(enc, 1, 48000)
    for _ in range(3):
        got = graph(audio)
        torch.cuda.synchronize()
        torch.testing.assert_close(got, eager, rtol=0, atol=0)
        _ = enc(audio)  # eager work between replays


def _attention_inputs(b, t, h=8, dk=128):
    g = torch.Generator().manual_seed(b * 1000 + t)
    qkv = torch.randn(b, t, 3 * h * dk, generator=g)
    pos = torch.randn(2 * t - 1, h * dk, generator=g)
    u, v = torch.randn(h, dk, generator=g) * 0.1, torch.randn(h, dk, generator=g) * 0.1
    return qkv, pos, u, v


def _attention_fp64(qkv, pos, u, v, h=8, dk=128):
    b, t, _ = qkv.shape
    q, k, vv = qkv.double().view(b, t, 3, h, dk).unbind(2)
    qu = (q + u.double()).transpose(1, 2)
    qv = (q + v.double()).transpose(1, 2)
    ac = qu @ k.permute(0, 2, 3, 1)
    bd = E.rel_shift(qv @ pos.double().view(2 * t - 1, h, dk).permute(1, 2, 0))
    a = torch.softmax((ac + bd) / math.sqrt(dk), dim=-1)
    return (a @ vv.transpose(1, 2)).transpose(1, 2).reshape(b, t, h * dk)


@pytest.mark.gpu
@pytest.mark.parametrize("b,t", [(1, 125), (1, 32), (2, 96), (1, 64), (2, 128), (1, 17)])
@torch.inference_mode()
def test_key_split_attention_matches_fp64(b, t):
    """The key-split form (two workgroups per (clip, query tile, head), halves merged by a second launch): the same
    FP64 bar as the unsplit kernel, the same result on repeated calls over one workspace, and within FP32 rounding of
    the unsplit kernel."""
    h = 8
    qkv, pos, u, v = _attention_inputs(b, t)
    ws = E.attention_workspace(b, t, h, "cuda")
    assert ws is not None and ws.numel() > 0
    dq, dp, du, dv = qkv.cuda(), pos.cuda(), u.cuda(), v.cuda()
    ref = _attention_fp64(qkv, pos, u, v)
    outs = [E.relpos_attention(dq, dp, du, dv, h, workspace=ws) for _ in range(2)]
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1])
    got = outs[0].cpu().double()
    assert float((got - ref).abs().max() / ref.abs().max()) < 2e-6
    unsplit = E.relpos_attention(dq, dp, du, dv, h).cpu().double()
    assert float((got - unsplit).abs().max() / ref.abs().max()) < 2e-6


@pytest.mark.gpu
@pytest.mark.parametrize("b,t,parts", [(1, 125, 1), (1, 125, 3), (2, 64, 2), (1, 17, 1)])
@torch.inference_mode()
def test_attention_merge_quantize_is_the_quantizer_of_the_merged_output(b, t, parts):
    """Quantizing the two halves directly (the merged rows are never written) gives bitwise what the library's
    quantizer and the oracle give on the merged output."""
    h = 8
    qkv, pos, u, v = _attention_inputs(b, t)
    ws = E.attention_workspace(b, t, h, "cuda")
    dq, dp, du, dv = qkv.cuda(), pos.cuda(), u.cuda(), v.cuda()
    assert E.relpos_attention(dq, dp, du, dv, h, workspace=ws, merged=False) is None
    q, qs = E.attention_merge_quantize(ws, b, t, h, parts)
    merged = E.relpos_attention(dq, dp, du, dv, h, workspace=ws)  # same halves, merged by the merge kernel
    lq, lqs, _ = E.lowbit.quantize(merged, (merged.stride(0), merged.stride(1), 1, t), b * t, h * 128, parts)
    torch.cuda.synchronize()
    assert torch.equal(q, lq) and torch.equal(qs, lqs)
    rq, rqs = O.quantize(merged.cpu().numpy().reshape(b * t, h * 128), parts, ldq=q.shape[2])
    assert np.array_equal(q.cpu().numpy(), rq) and np.array_equal(qs.cpu().numpy(), rqs)


def test_key_split_applies_only_to_small_even_grids():
    """Host-side rule and contract checks of the key-split attention (nothing is launched)."""
    L = E._hip.lib()
    rows = 125
    assert L.kea_relpos_attention_workspace(1, 125, 8) == 4 * (2 * rows * 8 * 128 + 2 * rows * 8 * 2)
    assert L.kea_relpos_attention_workspace(2, 128, 8) > 0       # 2 x 8 x 8 x 2 = 256 workgroups
    assert L.kea_relpos_attention_workspace(8, 125, 8) == 0      # 512 workgroups already fill the GPU
    assert L.kea_relpos_attention_workspace(1, 40, 8) == 0       # three 16-key tiles
    assert L.kea_relpos_attention_workspace(1, 200, 8) == 0      # the long-sequence kernel
    assert E.attention_workspace(8, 125, 8, "cuda") is None
    need = L.kea_relpos_attention_workspace(1, 125, 8)
    q = ctypes.c_void_p(16)
    assert L.kea_attention_merge_quantize(q, need, 1, 125, 8, 4, q, 1024, q, None) == -1            # parts
    assert L.kea_attention_merge_quantize(q, need, 8, 125, 8, 1, q, 1024, q, None) == -1            # no split
    assert L.kea_attention_merge_quantize(q, need - 4, 1, 125, 8, 1, q, 1024, q, None) == -4        # workspace
    assert L.kea_attention_merge_quantize(q, need, 1, 125, 8, 1, q, 1000, q, None) == -1            # ldq < k
    assert L.kea_attention_merge_quantize(ctypes.c_void_p(8), need, 1, 125, 8, 1, q, 1024, q, None) == -2
    assert L.kea_relpos_attention_ws(q, 3072, q, 1024, q, q, q, 1024, 1, 125, 8, 128, 1.0, q, need - 4, None) == -4
    assert L.kea_relpos_attention_ws(q, 3072, q, 1024, q, q, None, 1024, 8, 125, 8, 128, 1.0, None, 0, None) == -1


@pytest.mark.gpu
@pytest.mark.parametrize("b,t", [(1, 125), (2, 37), (1, 256), (3, 1), (8, 100), (5, 128), (4, 200)])
@torch.inference_mode()
def test_fused_relpos_attention_matches_fp64(b, t):
    """The fused kernel against the same formula in FP64 (rel_shift form); FP32 accumulation over 128-dim dot
    products and T-term sums bounds the error near 1e-6 relative."""
    h, dk = 8, 128
    g = torch.Generator().manual_seed(b * 1000 + t)
    qkv = torch.randn(b, t, 3 * h * dk, generator=g)
    pos = torch.randn(2 * t - 1, h * dk, generator=g)
    u, v = torch.randn(h, dk, generator=g) * 0.1, torch.randn(h, dk, generator=g) * 0.1
    got = E.relpos_attention(qkv.cuda(), pos.cuda(), u.cuda(), v.cuda(), h).cpu().double()
    q, k, vv = qkv.double().view(b, t, 3, h, dk).unbind(2)
    qu = (q + u.double()).transpose(1, 2)
    qv = (q + v.double()).transpose(1, 2)
    ac = qu @ k.permute(0, 2, 3, 1)
    bd = E.rel_shift(qv @ pos.double().view(2 * t - 1, h, dk).permute(1, 2, 0))
    a = torch.softmax((ac + bd) / math.sqrt(dk), dim=-1)
    ref = (a @ vv.transpose(1, 2)).transpose(1, 2).reshape(b, t, h * dk)
    assert float((got - ref).abs().max() / ref.abs().max()) < 2e-6


@pytest.mark.gpu
@torch.inference_mode()
def test_fused_glu_dwconv_matches_torch():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(2, 50, 2 * 96, generator=g)
    w = torch.randn(96, 1, 9, generator=g) / 3
    bias = torch.randn(96, generator=g)
    got = E.glu_dwconv(x.cuda(), w.cuda(), bias.cuda()).cpu().double()
    ref = F.conv1d(F.glu(x.double(), dim=-1).transpose(1, 2), w.double(), bias.double(), padding=4,
                   groups=96).transpose(1, 2)
    assert float((got - ref).abs().max()) < 1e-5


@pytest.mark.gpu
@torch.inference_mode()
def test_fused_encoder_matches_unfused():
    cfg = E.EncoderConfig(layers=3)
    w = E.synthetic_weights(cfg, seed=21)
    audio = torch.randn(2, 64000, generator=torch.Generator().manual_seed(22)).cuda()
    fused = E.FastConformerEncoder(w, cfg, "cuda", parts=3)(audio)
    plain = E.FastConformerEncoder(w, cfg, "cuda", parts=3, fused=False)(audio)
    rel = float((fused.double() - plain.double()).norm() / plain.double().norm())
    assert rel < 5e-6, rel


@pytest.mark.gpu
@torch.inference_mode()
def test_graph_cache_bounds_shapes_and_returns_owned_outputs():
    """At most max_graphs graphs (one per shape and stream), bitwise the eager forward on every replay; a shape past
    the limit runs eagerly; a returned tensor is the caller's (changing it changes no later result); every graph
    has its own key-split attention workspace, not the encoder's shared one."""
    cfg = E.EncoderConfig(layers=2)
    enc = E.FastConformerEncoder(E.synthetic_weights(cfg, seed=41), cfg, "cuda", parts=1)
    g = torch.Generator().manual_seed(42)
    clips = {n: torch.randn(1, n, generator=g).cuda() for n in (32000, 48000, 64000)}
    eager = {n: enc(a).clone() for n, a in clips.items()}
    cache = E.EncoderGraphCache(enc, max_graphs=2)
    for _ in range(2):
        for n, a in clips.items():
            got = cache(a)
            torch.cuda.synchronize()
            assert torch.equal(got, eager[n]), n
    assert len(cache.entries) == 2
    cache(clips[32000]).zero_()
    assert torch.equal(cache(clips[32000]), eager[32000])
    shared = {w.data_ptr() for w in enc._att_ws.values() if w is not None}
    own = [w for graph in cache.entries.values() for w in graph.workspaces.values() if w is not None]
    assert own and all(w.data_ptr() not in shared for w in own)
    cache.clear()
    assert not cache.entries


def _layer_norm(k: int, g: torch.Generator) -> torch.nn.LayerNorm:
    n = torch.nn.LayerNorm(k)
    with torch.no_grad():
        n.weight.copy_(torch.rand(k, generator=g) + 0.5)
        n.bias.copy_(torch.randn(k, generator=g) * 0.1)
    return n


@pytest.mark.gpu
@pytest.mark.parametrize("k,rows", [(1024, 74), (300, 9), (64, 1), (516, 130)])
@torch.inference_mode()
def test_norm_quantize_matches_layer_norm_and_oracle(k, rows):
    """kea_norm_quantize: x_out = LayerNorm0(x) within FP32 rounding of an FP64 LayerNorm; q / qs bitwise the oracle's
    normalised quantization (LayerNorm1) of that x_out, zero padding to ldq included."""
    from oracle import oracle as O
    g = torch.Generator().manual_seed(k + rows)
    x = torch.randn(1, rows, k, generator=g) * 3 + 0.5
    n0, n1 = _layer_norm(k, g), _layer_norm(k, g)
    d0, d1 = copy.deepcopy(n0).cuda(), copy.deepcopy(n1).cuda()
    out, q, qs = E.norm_quantize(x.cuda(), d0, d1, 3)
    xi = x.cuda()
    _, qi, qsi = E.norm_quantize(xi, d0, d1, 3, out=xi)  # in place
    torch.cuda.synchronize()
    assert torch.equal(xi, out) and torch.equal(qi, q) and torch.equal(qsi, qs)
    ref = F.layer_norm(x.double(), (k,), n0.weight.double(), n0.bias.double(), n0.eps)
    assert float((out.cpu().double() - ref).abs().max()) < 2e-5
    ldq = q.shape[2]
    rq, rqs = O.quantize(out.cpu().reshape(rows, k).numpy(), 3, ldq=ldq,
                         norm=(n1.weight.detach().numpy(), n1.bias.detach().numpy()), eps=n1.eps)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(qs.cpu().numpy(), rqs)


@pytest.mark.gpu
@pytest.mark.parametrize("b,t,c", [(2, 50, 96), (1, 125, 1024), (3, 17, 1536), (1, 1, 1024)])
@torch.inference_mode()
def test_glu_dwconv_quantize_equals_the_two_kernel_path(b, t, c):
    """kea_glu_dwconv_quantize: bitwise kea_glu_dwconv followed by kea_quantize with the input SiLU; and the parts sum
    to silu(conv(GLU(x))) (FP64) within half the last part's step."""
    from kea_kernels import lowbit
    g = torch.Generator().manual_seed(b * 1000 + t + c)
    x = torch.randn(b, t, 2 * c, generator=g)
    w = torch.randn(c, 1, 9, generator=g) / 3
    bias = torch.randn(c, generator=g)
    xd, wd, bd = x.cuda(), w.cuda(), bias.cuda()
    q, qs = E.glu_dwconv_quantize(xd, wd, bd, 3)
    z = E.glu_dwconv(xd, wd, bd)
    rq, rqs, _ = lowbit.quantize(z, (z.stride(0), z.stride(1), 1, t), b * t, c, 3, input_activation="silu")
    torch.cuda.synchronize()
    assert torch.equal(q, rq) and torch.equal(qs, rqs)
    conv = F.conv1d(F.glu(x.double(), dim=-1).transpose(1, 2), w.double(), bias.double(), padding=4,
                    groups=c).transpose(1, 2).reshape(b * t, c)
    ref = conv * torch.sigmoid(conv)
    deq = sum(q[i, :, :c].cpu().double() * qs[i].cpu().double()[:, None] for i in range(3))
    assert bool(((deq - ref).abs() <= 0.5 * qs[2].cpu().double()[:, None] + 2e-6 * ref.abs().amax(1, keepdim=True)).all())


@pytest.mark.gpu
@pytest.mark.parametrize("split,out_dtype", [(1, torch.float32), (2, torch.float32), (1, torch.float16)])
@torch.inference_mode()
def test_gemm_glu_pairs_feed_the_convolution_bitwise(split, out_dtype):
    """The GEMM's GLU epilogue on interleaved (value, gate) weight rows + kea_dwconv_quantize equals the plain GEMM +
    kea_glu_dwconv_quantize bit for bit; the GLU values match value * sigmoid(gate) of the plain output."""
    from oracle import oracle as O
    from kea_kernels import lowbit
    from kea_kernels.binary import kernels
    b, t, c, k = 2, 40, 256, 512
    m = b * t
    g = torch.Generator().manual_seed(split + 7)
    signs = torch.where(torch.rand(2 * c, k, generator=g) < 0.5, -1, 1).to(torch.int8)
    codes = torch.from_numpy(O.pack_signs(signs.numpy()))
    scale = torch.rand(2 * c, generator=g) * 0.09 + 0.01
    bias = torch.randn(2 * c, generator=g) * 0.1
    x = torch.randn(1, m, k, generator=g).cuda()
    q, qs, _ = lowbit.quantize(x, (0, k, 1, m), m, k, 3)
    w_plain = kernels.relayout_codes(codes, k, 1).cuda()
    w_il = kernels.relayout_codes(E.glu_interleave(codes), k, 1).cuda()
    y = torch.empty(m, 2 * c, device="cuda", dtype=out_dtype)
    lowbit.gemm(1, q, qs, w_plain, 2 * c, k, scale.cuda(), bias.cuda(), y, None)
    u = torch.empty(m, c, device="cuda", dtype=out_dtype)
    lowbit.gemm(1, q, qs, w_il, 2 * c, k, E.glu_interleave(scale).cuda(), E.glu_interleave(bias).cuda(), u, None,
                glu=True, config=kernels.GemmConfig(4, split))
    torch.cuda.synchronize()
    y64 = y.double()
    ref = y64[:, :c] * torch.sigmoid(y64[:, c:])
    tol = 1e-6 if out_dtype == torch.float32 else 2e-3
    assert float(((u.double() - ref).abs() / (ref.abs() + 1e-3)).max()) < tol
    if out_dtype == torch.float32:
        dw = torch.randn(c, 1, 9, generator=g).cuda() / 3
        db = torch.randn(c, generator=g).cuda()
        qa, qsa = E.glu_dwconv_quantize(y.view(b, t, 2 * c), dw, db, 3)
        qb, qsb = E.dwconv_quantize(u.view(b, t, c), dw, db, 3)
        torch.cuda.synchronize()
        assert torch.equal(qa, qb) and torch.equal(qsa, qsb)


@pytest.mark.gpu
@torch.inference_mode()
def test_gemm_glu_contract_errors():
    from kea_kernels import lowbit
    from kea_kernels.binary import kernels
    k = 128
    codes = torch.zeros(6, k // 8, dtype=torch.uint8)
    w = kernels.relayout_codes(codes, k, 1).cuda()
    q = torch.zeros(1, 4, k, dtype=torch.int8, device="cuda")
    qs = torch.ones(1, 4, device="cuda")
    scale = torch.ones(6, device="cuda")
    with pytest.raises(ValueError):  # SiLU and GLU together
        lowbit.gemm(1, q, qs, w, 6, k, scale, None, torch.empty(4, 3, device="cuda"), None, glu=True, silu=True)
    with pytest.raises(ValueError):  # odd n
        lowbit.gemm(1, q, qs, w, 5, k, scale[:5], None, torch.empty(4, 3, device="cuda"), None, glu=True)


@pytest.mark.gpu
@pytest.mark.parametrize("b,frames", [(1, 1000), (2, 999), (3, 37)])
@torch.inference_mode()
def test_fused_subsampling_matches_pytorch(b, frames):
    """kea_subsample_front + pointwise products + kea_dwconv2d_s2 + kea_bias_relu_flatten + output linear (x sqrt(d)
    folded in) against PyTorch's convolution stack in FP64."""
    cfg = E.EncoderConfig(layers=1)
    w = E.synthetic_weights(cfg, seed=4)
    enc = E.FastConformerEncoder(w, cfg, "cuda", parts=1)
    feats = torch.randn(b, cfg.feat_in, frames, generator=torch.Generator().manual_seed(frames)).cuda()
    got = enc._subsample_fused(feats).double()
    s = {k: v.double() for k, v in enc.sub.items()}
    c = cfg.sub_channels
    x = feats.double().transpose(1, 2).unsqueeze(1)
    x = F.relu(F.conv2d(x, s["conv.0.weight"], s["conv.0.bias"], stride=2, padding=1))
    for i in (2, 5):
        x = F.conv2d(x, s[f"conv.{i}.weight"], s[f"conv.{i}.bias"], stride=2, padding=1, groups=c)
        x = F.relu(F.conv2d(x, s[f"conv.{i + 1}.weight"], s[f"conv.{i + 1}.bias"]))
    bb, _, t, f = x.shape
    ref = F.linear(x.transpose(1, 2).reshape(bb, t, c * f), s["out.weight"], s["out.bias"]) * math.sqrt(cfg.d_model)
    assert got.shape == ref.shape
    assert float((got - ref).abs().max() / ref.abs().max()) < 1e-5


@pytest.mark.gpu
@pytest.mark.parametrize("b,samples", [(1, 160000), (3, 48000), (2, 16000)])
@torch.inference_mode()
def test_fused_logmel_matches_pytorch(b, samples):
    """kea_logmel_normalize (each mel filter's nonzero bins, log, per-feature normalisation) against the PyTorch
    preprocessor computed in FP64 after the same STFT."""
    cfg = E.EncoderConfig()
    audio = torch.randn(b, samples, generator=torch.Generator().manual_seed(samples)).cuda()
    got = E.Preprocessor(cfg, "cuda", fused=True)(audio).double()
    pre = E.Preprocessor(cfg, "cuda")
    x = torch.cat([audio[:, :1], audio[:, 1:] - cfg.preemph * audio[:, :-1]], dim=1)
    spec = torch.stft(x, n_fft=cfg.n_fft, hop_length=cfg.hop_length, win_length=cfg.win_length, window=pre.window,
                      center=True, pad_mode="constant", return_complex=True)
    frames = E.frames_for(cfg, samples)
    power = torch.view_as_real(spec[:, :, :frames]).double().pow(2).sum(-1)
    logmel = torch.log(torch.matmul(pre.fb.double(), power) + 2.0 ** -24)
    ref = (logmel - logmel.mean(2, keepdim=True)) / (logmel.std(2, keepdim=True) + 1e-5)
    assert got.shape == ref.shape
    assert float((got - ref).abs().max()) < 1e-4


@pytest.mark.gpu
@pytest.mark.parametrize("b,samples", [(1, 160000), (3, 48000), (2, 16001), (1, 300), (2, 1), (1, 159)])
@torch.inference_mode()
def test_stft_frames_give_torch_stft_spectrum_bitwise(b, samples):
    """kea_stft_frames' frames, through torch's real FFT, are the spectrum torch.stft returns for the pre-emphasised
    audio (centred, constant padding, Hann 400 in n_fft 512), bit for bit and frame-major; the frame-major log-mel
    kernel then gives the bin-major one's output bit for bit."""
    cfg = E.EncoderConfig()
    audio = torch.randn(b, samples, generator=torch.Generator().manual_seed(samples + b)).cuda()
    pre = E.Preprocessor(cfg, "cuda", fused=True)
    frames = pre.stft_frames(audio)
    assert frames.shape == (b, 1 + samples // cfg.hop_length, cfg.n_fft)
    x = torch.cat([audio[:, :1], audio[:, 1:] - cfg.preemph * audio[:, :-1]], dim=1)
    ref = torch.stft(x, n_fft=cfg.n_fft, hop_length=cfg.hop_length, win_length=cfg.win_length, window=pre.window,
                     center=True, pad_mode="constant", return_complex=True)
    got = torch.fft.rfft(frames, dim=-1)
    assert torch.equal(torch.view_as_real(got), torch.view_as_real(ref.transpose(1, 2)))
    n = E.frames_for(cfg, samples)
    if n == 0:
        return
    lib, stream = _hip.lib(), _hip.stream_handle(audio.device)
    spec = ref.contiguous()
    y_bins = torch.empty(b, cfg.feat_in, n, device="cuda")
    y_frames = torch.full_like(y_bins, float("nan"))
    _hip.check(lib.kea_logmel_normalize(torch.view_as_real(spec).data_ptr(), b, spec.shape[1], n, spec.shape[2],
                                        pre.fb.data_ptr(), pre.lo.data_ptr(), pre.hi.data_ptr(), cfg.feat_in,
                                        2.0 ** -24, 1e-5, y_bins.data_ptr(), stream), "kea_logmel_normalize")
    _hip.check(lib.kea_logmel_normalize_frames(torch.view_as_real(got).data_ptr(), b, got.shape[2], n, got.shape[1],
                                               pre.fb.data_ptr(), pre.lo.data_ptr(), pre.hi.data_ptr(), cfg.feat_in,
                                               2.0 ** -24, 1e-5, y_frames.data_ptr(), stream),
               "kea_logmel_normalize_frames")
    assert torch.equal(y_frames, y_bins)
    assert torch.equal(pre(audio), y_bins)


@pytest.mark.gpu
@pytest.mark.parametrize("frames,ld,seed", [(700, 703, 1), (1, 1, 2), (513, 520, 3)])
@torch.inference_mode()
def test_frame_major_logmel_equals_bin_major_on_wide_bands(frames, ld, seed):
    """kea_logmel_normalize_frames (bands staged through LDS 16 bins at a time, 512 frames at a time) against
    kea_logmel_normalize on the transposed spectrum, bit for bit, with filter bands of 0 to 40 bins."""
    g = torch.Generator().manual_seed(seed)
    b, bins, mels = 2, 257, 9
    spec_f = torch.randn(b, ld, bins, 2, generator=g)
    lo = torch.randint(0, bins, (mels,), generator=g, dtype=torch.int32)
    width = torch.tensor([0, 1, 5, 12, 16, 17, 31, 40, 3], dtype=torch.int32)
    hi = torch.minimum(lo + width, torch.tensor(bins, dtype=torch.int32))
    fb = torch.zeros(mels, bins)
    for m in range(mels):
        fb[m, lo[m]:hi[m]] = torch.rand(int(hi[m] - lo[m]), generator=g) + 0.01
    spec_b = spec_f.transpose(1, 2).contiguous()   # [b][bins][ld][2]
    dev = "cuda"
    spec_f, spec_b, fb, lo, hi = (t.to(dev) for t in (spec_f, spec_b, fb, lo, hi))
    lib, stream = _hip.lib(), _hip.stream_handle(torch.device(dev))
    y_b = torch.full((b, mels, frames), float("nan"), device=dev)
    y_f = torch.full_like(y_b, float("nan"))
    _hip.check(lib.kea_logmel_normalize(spec_b.data_ptr(), b, bins, frames, ld, fb.data_ptr(), lo.data_ptr(),
                                        hi.data_ptr(), mels, 2.0 ** -24, 1e-5, y_b.data_ptr(), stream), "bin-major")
    _hip.check(lib.kea_logmel_normalize_frames(spec_f.data_ptr(), b, bins, frames, ld, fb.data_ptr(), lo.data_ptr(),
                                               hi.data_ptr(), mels, 2.0 ** -24, 1e-5, y_f.data_ptr(), stream),
               "frame-major")
    torch.cuda.synchronize()
    assert torch.equal(y_f, y_b)
    assert not torch.isnan(y_f).any()


def test_stft_and_logmel_entry_points_check_sizes_before_any_launch():
    """The framing and frame-major log-mel entry points refuse sizes they cannot run before touching the GPU."""
    L = _hip.lib()
    vp = ctypes.c_void_p
    assert L.kea_stft_frames(vp(16), 1, 1000, 0.97, vp(16), 511, 160, vp(16), None) == -1     # odd n_fft
    assert b"n_fft" in L.kea_last_error()
    assert L.kea_stft_frames(vp(16), 1, 0, 0.97, vp(16), 512, 160, vp(16), None) == -1        # no samples
    assert L.kea_stft_frames(vp(16), 1, 1000, 0.97, vp(16), 512, 0, vp(16), None) == -1       # hop
    assert L.kea_stft_frames(vp(16), 70000, 1000, 0.97, vp(16), 512, 160, vp(16), None) == -1  # batch
    assert L.kea_stft_frames(None, 1, 1000, 0.97, vp(16), 512, 160, vp(16), None) == -1       # null audio
    assert L.kea_stft_frames(None, 0, 1000, 0.97, None, 512, 160, None, None) == 0             # empty batch
    args = (vp(16), 1, 257, 10, 9, vp(16), vp(16), vp(16), 80, 2.0 ** -24, 1e-5, vp(16), None)
    assert L.kea_logmel_normalize_frames(*args) == -1                                           # ld_f < frames
    assert L.kea_logmel_normalize_frames(vp(12), *args[1:4], 10, *args[5:]) == -2               # alignment


def test_fused_launchers_check_parameters_before_any_call():
    """The encoder's fused-kernel launchers refuse, before any C call, parameters the kernels would read past: a
    depthwise weight or bias not of C x KW / C elements, positions shorter than 2T - 1 rows, head biases not of d
    elements, LayerNorm parameters not of K elements, and non-FP32 inputs."""
    from kea_kernels import encoder as E
    c, kw, t = 4, 9, 4
    x = torch.zeros(1, t, 2 * c)
    u = torch.zeros(1, t, c)
    w, b = torch.zeros(c, 1, kw), torch.zeros(c)
    for fn, inp in ((E.glu_dwconv, x), (lambda *a: E.glu_dwconv_quantize(*a, 1), x),
                    (lambda *a: E.dwconv_quantize(*a, 1), u)):
        with pytest.raises(ValueError, match="weight"):
            fn(inp, torch.zeros(c - 1, 1, kw), b)
        with pytest.raises(ValueError, match="bias"):
            fn(inp, w, torch.zeros(c + 1))
        with pytest.raises(ValueError, match="FP32"):
            fn(inp.half(), w, b)
    heads, d = 2, 256
    qkv, pos = torch.zeros(1, t, 3 * d), torch.zeros(2 * t - 1, d)
    bu = bv = torch.zeros(heads, d // heads)
    with pytest.raises(ValueError, match="pos"):
        E.relpos_attention(qkv, pos[:-1], bu, bv, heads)
    with pytest.raises(ValueError, match="bias_u"):
        E.relpos_attention(qkv, pos, bu[:1], bv, heads)
    with pytest.raises(ValueError, match="heads"):
        E.relpos_attention(qkv, pos, bu, bv, 3)
    with pytest.raises(ValueError, match="qkv"):
        E.relpos_attention(qkv.half(), pos, bu, bv, heads)
    ln_k, ln_short = torch.nn.LayerNorm(d), torch.nn.LayerNorm(d - 1)
    with pytest.raises(ValueError, match="norm1.weight"):
        E.norm_quantize(torch.zeros(1, t, d), ln_k, ln_short, 1)


def test_fused_preprocessor_refuses_host_and_mismatched_audio_before_any_call():
    """The framing kernel's launcher refuses audio that is not contiguous FP32 [B, S], on another device than its
    window, or on the host (no GPU pointer to launch on), before any C call."""
    cfg = E.EncoderConfig()
    pre = E.Preprocessor(cfg, "cpu", fused=True)
    with pytest.raises(ValueError, match="FP32"):
        pre.stft_frames(torch.zeros(1, 1600, dtype=torch.float64))
    with pytest.raises(ValueError, match="contiguous"):
        pre.stft_frames(torch.zeros(1600, 2).t())
    with pytest.raises(ValueError, match="GPU"):
        pre.stft_frames(torch.zeros(1, 1600))
    pre.window_nfft = pre.window_nfft.to("meta")
    with pytest.raises(ValueError, match="preprocessor on meta"):
        pre.stft_frames(torch.zeros(1, 1600))


def test_graph_cache_limits_and_eager_paths_on_cpu():
    with pytest.raises(ValueError, match="max_graphs"):
        E.EncoderGraphCache(None, max_graphs=0)
    cfg = E.EncoderConfig(layers=1)
    enc = E.FastConformerEncoder(E.synthetic_weights(cfg, seed=43), cfg, "cpu", dense=True)
    audio = torch.randn(1, 16000, generator=torch.Generator().manual_seed(44))
    cache = E.EncoderGraphCache(enc)
    assert torch.equal(cache(audio), enc(audio))  # CPU audio: eager, nothing captured
    assert not cache.entries
