"""GPU parity of the low-bit GEMM (called through the C ABI) against the pinned CPU oracle.

The bar: int32 accumulators bit-exact; dequantized outputs bitwise equal to the oracle's FP32 epilogue rounded to the
output type (the epilogue is a fixed sequence of IEEE operations on both sides), except SiLU, whose exp differs by
ulps between the GPU's and the C library's implementation (checked within a stated tolerance instead). Shapes cover
BASELINE.json's configs 1-4 at full size, plus ragged K, N tails, P = 1..3, every tile and every split.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from kea_kernels import lowbit
from kea_kernels.binary import kernels
from oracle import oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"


class Case:
    """Seeded inputs on the CPU (torch.Generator, as the reference's tests), uploaded once."""

    def __init__(self, wbits, p, m, n, k, seed, *, scale_dtype=torch.float16, bias=False, pad_garbage=True):
        g = torch.Generator().manual_seed(seed)
        self.wbits, self.p, self.m, self.n, self.k = wbits, p, m, n, k
        self.ldq = -(-k // 16) * 16 + (16 if pad_garbage else 0)
        q = torch.randint(-127, 128, (p, m, self.ldq), generator=g, dtype=torch.int8)
        if not pad_garbage:
            q[:, :, k:] = 0
        self.q = q
        if wbits == 1:
            w = torch.where(torch.rand(n, k, generator=g) < 0.5, -1, 1).to(torch.int8)
            self.codes = O.pack_signs(w.numpy())
        else:
            w = torch.randint(-1, 2, (n, k), generator=g, dtype=torch.int8)
            self.codes = O.pack_ternary(w.numpy())
        qs = torch.rand(p, m, generator=g) * 0.02 + 1e-3
        qs = qs / torch.tensor([1.0, 254.0, 254.0 ** 2][:p])[:, None]
        self.qs = qs.to(scale_dtype)
        self.alpha = (torch.rand(n, generator=g) * 0.09 + 0.01).to(scale_dtype)
        self.bias = torch.randn(n, generator=g).to(scale_dtype) if bias else None
        self.words = kernels.relayout_codes(torch.from_numpy(self.codes), k, wbits).to(DEV)
        self.dq, self.dqs, self.dalpha = self.q.to(DEV), self.qs.to(DEV), self.alpha.to(DEV)
        self.dbias = None if self.bias is None else self.bias.to(DEV)

    def oracle_acc(self):
        fn = O.b1_gemm if self.wbits == 1 else O.t2_gemm
        return fn(self.q.numpy(), self.codes, self.k)

    def oracle_y(self, acc, *, silu=False, order=0):
        bias = None if self.bias is None else self.bias.float().numpy()
        return O.epilogue(acc, self.qs.float().numpy(), self.alpha.float().numpy(), bias, silu=silu, order=order)

    def run(self, *, out_dtype=torch.float16, acc=True, silu=False, order=0, config=None, ldy=None):
        ldy = ldy or self.n
        y = torch.full((self.m, ldy), float("nan"), device=DEV, dtype=out_dtype) if out_dtype else None
        a = torch.full((self.p, self.m, self.n), -7, device=DEV, dtype=torch.int32) if acc else None
        lowbit.gemm(self.wbits, self.dq, self.dqs, self.words, self.n, self.k, self.dalpha, self.dbias,
                    None if y is None else y, a, silu=silu, order=order, config=config)
        torch.cuda.synchronize()
        return (None if y is None else y[:, :self.n].cpu()), (None if a is None else a.cpu().numpy())


def _bits(y32, dtype):
    if dtype == torch.float16:
        return O.to_f16_bits(y32)
    if dtype == torch.bfloat16:
        return O.to_bf16_bits(y32)
    return y32.view(np.uint32)


def _gpu_bits(y, dtype):
    if dtype == torch.float32:
        return y.numpy().view(np.uint32)
    return y.view(torch.int16).numpy().view(np.uint16)


def assert_parity(case, y, acc, *, out_dtype=torch.float16, silu=False, order=0):
    ref_acc = case.oracle_acc()
    if acc is not None:
        assert np.array_equal(acc, ref_acc), f"int32 mismatch at {np.argwhere(acc != ref_acc)[:5].tolist()}"
    if y is not None:
        ref = case.oracle_y(ref_acc, silu=silu, order=order)
        if silu:
            got = y.float().numpy()
            tol = {torch.float32: 2e-6, torch.float16: 1e-3, torch.bfloat16: 8e-3}[out_dtype]
            np.testing.assert_allclose(got, ref, rtol=tol, atol=tol)
        else:
            want = _bits(ref, out_dtype)
            got = _gpu_bits(y, out_dtype)
            bad = np.argwhere(got != want)
            assert bad.size == 0, f"{bad.shape[0]} output mismatches, first {bad[:5].tolist()}"


# --- BASELINE configs ------------------------------------------------------------------------------------------------

@torch.inference_mode()
def test_config1_b1_m128_k1024_n4096_fp16():
    case = Case(1, 1, 128, 4096, 1024, seed=128 + 4096 + 1024)
    y, acc = case.run()
    assert_parity(case, y, acc)


@torch.inference_mode()
def test_config2_ternary_m128_k4096_n1024_fp16():
    case = Case(2, 1, 128, 1024, 4096, seed=2)
    y, acc = case.run()
    assert_parity(case, y, acc)


@pytest.mark.parametrize("n,k", [(3072, 1024), (1024, 1024), (4096, 1024), (1024, 4096), (2048, 1024)])
@torch.inference_mode()
def test_config3_encoder_linears_m1000(n, k):
    case = Case(1, 1, 1000, n, k, seed=n + k + 1000)
    y, acc = case.run()
    assert_parity(case, y, acc)


@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("n,k", [(2560, 640), (1030, 640), (1024, 4096)])
@torch.inference_mode()
def test_config4_small_m_every_split(wbits, m, n, k):
    if (n, k) == (1024, 4096) and m != 16:
        pytest.skip("BASELINE config 4 runs 4096->1024 at M = 16")
    case = Case(wbits, 1, m, n, k, seed=wbits * 100 + m + n + k)
    ref = None
    for split in (1, 2, 4, 0):
        y, acc = case.run(config=kernels.GemmConfig(tile=1, split=split) if split else None)
        assert_parity(case, y, acc)
        if ref is None:
            ref = (y, acc)
        assert torch.equal(y.view(torch.int16), ref[0].view(torch.int16)) and np.array_equal(acc, ref[1])


# --- parts, flags, dtypes, tails ---------------------------------------------------------------------------------

@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("p", [1, 2, 3])
@pytest.mark.parametrize("order", [0, 1])
@torch.inference_mode()
def test_parts_and_order(wbits, p, order):
    case = Case(wbits, p, 77, 1030, 640, seed=p * 10 + order + wbits, bias=True)
    y, acc = case.run(out_dtype=torch.float32, order=order)
    assert_parity(case, y, acc, out_dtype=torch.float32, order=order)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("scale_dtype", [torch.float32, torch.float16])
@torch.inference_mode()
def test_output_and_scale_dtypes(out_dtype, scale_dtype):
    case = Case(1, 2, 50, 300, 1024, seed=5, scale_dtype=scale_dtype, bias=True)
    y, acc = case.run(out_dtype=out_dtype)
    assert_parity(case, y, acc, out_dtype=out_dtype)


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("wbits,p", [(1, 1), (2, 3)])
@torch.inference_mode()
def test_split_k_finish_with_bias_and_output_dtypes(out_dtype, wbits, p):
    """Split K = 4: the int32 slices are summed and finished by the separate epilogue kernel, which applies the bias
    and writes f32 / bf16 (order 1 at three parts) bit for bit as the oracle."""
    case = Case(wbits, p, 45, 300, 2048, seed=60 + p, scale_dtype=torch.float32, bias=True)
    order = 1 if p == 3 else 0
    y, acc = case.run(out_dtype=out_dtype, order=order, config=kernels.GemmConfig(0, 4))
    assert_parity(case, y, acc, out_dtype=out_dtype, order=order)


@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("k", [1, 15, 17, 300, 1100])
@torch.inference_mode()
def test_ragged_k_with_garbage_padding(wbits, k):
    case = Case(wbits, 2, 33, 45, k, seed=k + wbits, bias=True, pad_garbage=True)
    y, acc = case.run(out_dtype=torch.float32)
    assert_parity(case, y, acc, out_dtype=torch.float32)


@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("m,n,k,parts", [(1, 1030, 1100, 1), (5, 37, 17, 3), (16, 2560, 640, 2), (40, 300, 4100, 1)])
@torch.inference_mode()
def test_every_wave_split_tile_on_ragged_small_m_shapes(wbits, m, n, k, parts):
    """Each wave-split tile (its K range cut over 4 or 8 waves, N tails of one 16-column block or less) against the
    oracle at the small-M shapes the narrow tiles serve: one row, ragged K with garbage padding, N not a multiple of
    16, several activation parts."""
    case = Case(wbits, parts, m, n, k, seed=m + n + k + wbits, bias=True, pad_garbage=True)
    ran = 0
    for tile in range(1, kernels.tile_count() + 1):
        if " k/" not in kernels.config_name(tile):
            continue
        try:
            y, acc = case.run(out_dtype=torch.float32, config=kernels.GemmConfig(tile=tile, split=0))
        except ValueError as e:
            # tiles whose registers cannot hold this many parts, and K % 16 != 0 ranges too long for one workgroup
            if "does not fit" in str(e) or "unsplit K range" in str(e):
                continue
            raise
        assert_parity(case, y, acc, out_dtype=torch.float32)
        ran += 1
    assert ran >= 3  # at least three tiles take every one of these shapes


def _random_cases(count, seed):
    """Seeded shapes, part counts, tiles, splits, output and scale types, biases and SiLU flags drawn at random:
    combinations no hand-written case covers."""
    rng = np.random.default_rng(seed)
    out_dtypes = [torch.float32, torch.float16, torch.bfloat16]
    for i in range(count):
        yield dict(wbits=int(rng.integers(1, 3)), p=int(rng.integers(1, 4)), m=int(rng.integers(1, 260)),
                   n=int(rng.integers(1, 600)), k=int(rng.integers(1, 2200)), tile=int(rng.integers(0, 24)),
                   split=int(rng.choice([0, 1, 2, 4])), out_dtype=out_dtypes[int(rng.integers(0, 3))],
                   scale_dtype=[torch.float32, torch.float16][int(rng.integers(0, 2))], bias=bool(rng.integers(0, 2)),
                   order=int(rng.integers(0, 2)), seed=seed * 1000 + i)


@pytest.mark.parametrize("seed", [11, 12, 13])
@torch.inference_mode()
def test_seeded_random_cases_bitwise(seed):
    """Random shapes (ragged M, N and K with garbage padding), 1 to 3 parts, any tile (0: the library's choice) and
    split, f32 / f16 / bf16 output, f32 / f16 scales, with and without bias, both epilogue orders: int32 accumulators
    and outputs bitwise the oracle's. Configurations the library refuses (a tile that cannot hold the parts, a split
    without a second slice, an unsplit ragged K range too long for one workgroup) are skipped, not counted."""
    ran = 0
    for c in _random_cases(12, seed):
        case = Case(c["wbits"], c["p"], c["m"], c["n"], c["k"], seed=c["seed"], scale_dtype=c["scale_dtype"],
                    bias=c["bias"], pad_garbage=True)
        config = kernels.GemmConfig(tile=c["tile"], split=c["split"]) if c["tile"] else None
        try:
            y, acc = case.run(out_dtype=c["out_dtype"], order=c["order"], config=config)
        except ValueError as e:
            if any(s in str(e) for s in ("does not fit", "unsplit K range", "split", "slices")):
                continue
            raise
        assert_parity(case, y, acc, out_dtype=c["out_dtype"], order=c["order"])
        ran += 1
    assert ran >= 6, ran


@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16])
@torch.inference_mode()
def test_silu_epilogue_within_tolerance(out_dtype):
    case = Case(1, 1, 64, 512, 1024, seed=8, bias=True)
    y, acc = case.run(out_dtype=out_dtype, silu=True)
    assert_parity(case, y, acc, out_dtype=out_dtype, silu=True)


@pytest.mark.parametrize("wbits,parts", [(1, 2), (2, 2), (1, 1), (2, 1)])
@torch.inference_mode()
def test_every_tile_gives_identical_results(wbits, parts):
    case = Case(wbits, parts, 70, 200, 1152, seed=31 + parts, bias=True)
    ref = None
    for tile in range(1, kernels.tile_count() + 1):
        try:
            y, acc = case.run(config=kernels.GemmConfig(tile=tile, split=1))
        except ValueError as e:
            # a tile whose registers hold one part's operands and accumulators only (the 16-wave producer tile, the
            # widest eight-wave tiles) refuses more parts; at one part every tile must run
            if parts > 1 and "does not fit" in str(e):
                continue
            raise
        if ref is None:
            assert_parity(case, y, acc)
            ref = (y, acc)
        assert torch.equal(y.view(torch.int16), ref[0].view(torch.int16)), f"tile {tile}"
        assert np.array_equal(acc, ref[1]), f"tile {tile}"


@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("m,n,k", [(70, 200, 1152), (1000, 512, 256), (257, 4096, 4096), (130, 384, 2048)])
@torch.inference_mode()
def test_producer_wave_tiles_equal_their_compute_tiles(wbits, m, n, k):
    """Tiles 6 and 7 are tiles 11 and 8 with waves that only issue the ring's copies: same bits, unsplit and split
    (split-K slices and the masked last stage pass through the producer hand-over too)."""
    assert kernels.config_name(6).endswith(" p8") and kernels.config_name(7).endswith(" p4")
    case = Case(wbits, 1, m, n, k, seed=m + n + k, bias=True)
    for producer, compute in ((6, 11), (7, 8)):
        want_y, want_acc = case.run(config=kernels.GemmConfig(tile=compute, split=1))
        for split in (1, 2, 3):
            y, acc = case.run(config=kernels.GemmConfig(tile=producer, split=split))
            assert torch.equal(y.view(torch.int16), want_y.view(torch.int16)), (producer, split)
            assert np.array_equal(acc, want_acc), (producer, split)
    assert_parity(case, want_y, want_acc)


@pytest.mark.parametrize("wbits,parts", [(1, 1), (2, 2)])
@pytest.mark.parametrize("out_dtype", [torch.float32, torch.float16, torch.bfloat16])
@torch.inference_mode()
def test_glu_fast_epilogue_equals_the_general_one_on_every_tile(wbits, parts, out_dtype):
    """GLU outputs of whole blocks take a compile-time epilogue when y rows are vector-aligned; an odd row stride
    sends every block through the general epilogue. Both must give the same bits, on every tile (partial row and
    column blocks included: M = 70, 200 output pairs)."""
    case = Case(wbits, parts, 70, 400, 1152, seed=90 + parts, bias=True)
    want = None
    for tile in range(1, kernels.tile_count() + 1):
        outs = []
        for ldy in (200, 201):
            y = torch.full((70, ldy), float("nan"), device=DEV, dtype=out_dtype)
            try:
                lowbit.gemm(wbits, case.dq, case.dqs, case.words, 400, 1152, case.dalpha, case.dbias, y, None,
                            glu=True, config=kernels.GemmConfig(tile=tile, split=1))
            except ValueError as e:
                if parts > 1 and "does not fit" in str(e):  # one-part tiles, as in the every-tile test
                    break
                raise
            torch.cuda.synchronize()
            outs.append(y[:, :200].contiguous().view(torch.int16 if out_dtype != torch.float32 else torch.int32))
        if not outs:
            continue
        assert torch.equal(outs[0], outs[1]), f"tile {tile}: fast and general GLU epilogues differ"
        if want is None:
            want = outs[0]
        assert torch.equal(outs[0], want), f"tile {tile}"


def _at_odd_offset(t: torch.Tensor) -> torch.Tensor:
    """A copy of contiguous t whose storage starts one element past an aligned address (2-byte aligned f16)."""
    buf = torch.zeros(t.numel() + 1, dtype=t.dtype, device=DEV)
    view = buf[1:].view(t.shape)
    view.copy_(t)
    assert view.data_ptr() % 4 == 2
    return view


@pytest.mark.parametrize("tile", [13, 14, 15, 18, 20])
@pytest.mark.parametrize("parts", [1, 3])
@torch.inference_mode()
def test_f16_scales_at_odd_element_offsets_on_wave_split_tiles(tile, parts):
    """The wave-split kernel loads f16 per-token scales, weight scales and bias as the aligned 32-bit word holding
    each element and picks the half by address: vectors that start 2 bytes into a word give the oracle's bits."""
    case = Case(1, parts, 37, 96, 1024, seed=tile + parts, bias=True)
    qs, alpha, bias = _at_odd_offset(case.dqs), _at_odd_offset(case.dalpha), _at_odd_offset(case.dbias)
    y = torch.full((case.m, case.n), float("nan"), device=DEV, dtype=torch.float16)
    lowbit.gemm(1, case.dq, qs, case.words, case.n, case.k, alpha, bias, y, None,
                config=kernels.GemmConfig(tile=tile, split=1))
    torch.cuda.synchronize()
    assert_parity(case, y.cpu(), None)


@torch.inference_mode()
def test_strided_output_rows_and_acc_only():
    case = Case(1, 1, 20, 100, 256, seed=44)
    y, _ = case.run(out_dtype=torch.float32, acc=False, ldy=131)  # odd row stride: no vector stores
    assert_parity(case, y, None, out_dtype=torch.float32)
    _, acc = case.run(out_dtype=None, acc=True)
    assert_parity(case, None, acc)


@pytest.mark.parametrize("wbits,k,split", [(1, 384, 1), (2, 384, 1), (1, 2048, 4), (2, 2048, 4)])
@torch.inference_mode()
def test_leading_rows_of_a_taller_q(wbits, k, split):
    """m below q's row count, three parts: the part planes sit rows * ldq apart (a gap after each part's m rows) and
    the scale rows `rows` apart. The m output rows match the oracle on the first m activation rows, bit for bit,
    unsplit and split, and the output rows past m stay untouched."""
    case = Case(wbits, 3, 40, 96, k, seed=45)
    m, n = 25, 96
    y = torch.full((40, n), float("nan"), device=DEV, dtype=torch.float16)
    acc = torch.full((3, m, n), -7, device=DEV, dtype=torch.int32)
    lowbit.gemm(wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, None, y, acc, m=m,
                config=kernels.GemmConfig(0, split))
    torch.cuda.synchronize()
    ref_acc = case.oracle_acc()[:, :m]
    assert np.array_equal(acc.cpu().numpy(), ref_acc)
    ref = O.epilogue(ref_acc, case.qs.float().numpy()[:, :m], case.alpha.float().numpy(), None)
    assert np.array_equal(_gpu_bits(y[:m].cpu(), torch.float16), _bits(ref, torch.float16))
    assert torch.isnan(y[m:]).all()


@pytest.mark.parametrize("wbits,m,n,k,config", [(1, 128, 4096, 1024, None), (2, 40, 300, 4096, (4, 4)),
                                                 (1, 70, 200, 1152, (kernels.tile_count(), 0))])
@torch.inference_mode()
def test_plan_launches_equal_direct_calls(wbits, m, n, k, config):
    """lowbit.GemmPlan (kea_lowbit_gemm_plan + _launch): validated once, launched twice, the same bits as gemm()
    and the oracle, including a split-K plan (its own workspace) and a residual epilogue."""
    case = Case(wbits, 1, m, n, k, seed=46 + m, bias=True)
    cfg = None if config is None else kernels.GemmConfig(*config)
    y_ref, acc_ref = case.run(config=cfg)
    assert_parity(case, y_ref, acc_ref)
    y = torch.full((m, n), float("nan"), device=DEV, dtype=torch.float16)
    acc = torch.full((1, m, n), -7, device=DEV, dtype=torch.int32)
    plan = lowbit.GemmPlan(wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, case.dbias, y, acc, config=cfg)
    for _ in range(2):
        y.fill_(float("nan"))
        plan()
        torch.cuda.synchronize()
        assert torch.equal(y.cpu().view(torch.int16), y_ref.view(torch.int16))
        assert np.array_equal(acc.cpu().numpy(), acc_ref)
    # residual epilogue through a plan: y = r + value * 0.5, against gemm(residual=...)
    r = torch.randn(m, n, generator=torch.Generator().manual_seed(3)).to(DEV)
    y1, y2 = torch.empty(m, n, device=DEV), torch.empty(m, n, device=DEV)
    lowbit.gemm(wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, case.dbias, y1, None, config=cfg,
                residual=r, residual_factor=0.5)
    lowbit.GemmPlan(wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, case.dbias, y2, None, config=cfg,
                    residual=r, residual_factor=0.5)()
    torch.cuda.synchronize()
    assert torch.equal(y1.view(torch.int32), y2.view(torch.int32))


@torch.inference_mode()
def test_zero_rows_is_a_no_op():
    case = Case(1, 1, 4, 64, 128, seed=1)
    y = torch.zeros(0, 64, device=DEV)
    lowbit.gemm(1, case.dq[:, :0], case.dqs[:, :0], case.words, 64, 128, case.dalpha, None, y, None)
    torch.cuda.synchronize()


# --- the quantizer ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("k", [17, 256, 300, 1024, 1500, 2050, 4096, 8192])
@pytest.mark.parametrize("with_norm", [False, True])
@torch.inference_mode()
def test_quantizer_bitwise_against_oracle(k, with_norm):
    g = torch.Generator().manual_seed(k + with_norm)
    x = torch.randn(57, k, generator=g) * 2 + 0.25
    norm = None
    if with_norm:
        norm = torch.nn.LayerNorm(k)
        with torch.no_grad():
            norm.weight.copy_(torch.rand(k, generator=g) + 0.5)
            norm.bias.copy_(torch.randn(k, generator=g) * 0.1)
    xd = x.to(DEV)
    dnorm = None
    if norm is not None:
        dnorm = torch.nn.LayerNorm(k).to(DEV)
        dnorm.load_state_dict(norm.state_dict())
    q, qs, ldq = lowbit.quantize(xd, (0, xd.stride(0), 1, 57), 57, k, 3, norm=dnorm)
    torch.cuda.synchronize()
    rq, rqs = O.quantize(x.numpy(), 3, ldq=ldq,
                         norm=None if norm is None else (norm.weight.detach().numpy(), norm.bias.detach().numpy()),
                         eps=1e-5)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(qs.cpu().numpy(), rqs)


@pytest.mark.parametrize("k", [64, 1024, 2048])
@torch.inference_mode()
def test_quantizer_strided_rows_bitwise(k):
    """x [B, K, T] read as rows (b, t) with element stride T (the pointwise-convolution layout)."""
    g = torch.Generator().manual_seed(k)
    x = torch.randn(3, k, 41, generator=g)
    norm = torch.nn.LayerNorm(k)
    with torch.no_grad():
        norm.weight.copy_(torch.rand(k, generator=g) + 0.5)
        norm.bias.copy_(torch.randn(k, generator=g) * 0.1)
    dnorm = torch.nn.LayerNorm(k).to(DEV)
    dnorm.load_state_dict(norm.state_dict())
    xd = x.to(DEV)
    q, qs, ldq = lowbit.quantize(xd, (xd.stride(0), xd.stride(2), xd.stride(1), 41), 3 * 41, k, 2, norm=dnorm)
    torch.cuda.synchronize()
    rows = x.transpose(1, 2).reshape(3 * 41, k).contiguous().numpy()
    rq, rqs = O.quantize(rows, 2, ldq=ldq, norm=(norm.weight.detach().numpy(), norm.bias.detach().numpy()), eps=1e-5)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(qs.cpu().numpy(), rqs)


@torch.inference_mode()
def test_quantizer_fp16_input_and_scales():
    g = torch.Generator().manual_seed(77)
    x = (torch.randn(40, 1024, generator=g)).to(torch.float16)
    xd = x.to(DEV)
    q, qs, ldq = lowbit.quantize(xd, (0, 1024, 1, 40), 40, 1024, 1, qs_dtype=torch.float16)
    torch.cuda.synchronize()
    rq, rqs = O.quantize(x.numpy(), 1, ldq=ldq, qs_f16=True)
    assert np.array_equal(q.cpu().numpy(), rq)
    assert np.array_equal(qs.cpu().float().numpy(), rqs)


@pytest.mark.parametrize("parts", [1, 2, 3])
@pytest.mark.parametrize("qs_dtype", [torch.float32, torch.float16])
@pytest.mark.parametrize("k,x_dtype", [(256, np.float32), (1024, np.float32), (1024, np.float16), (300, np.float32)])
@torch.inference_mode()
def test_quantizer_rounds_exact_ties_half_to_even(parts, qs_dtype, k, x_dtype):
    """Rows whose first-part quotients are exact half-integers (tests/tie_rows.py): the GPU quantizer rounds them half
    to even (0.5 -> 0, 1.5 -> 2, -2.5 -> -2; expected codes from integer arithmetic), on the one-wave (K <= 256) and
    four-wave row paths, f32 and f16 inputs and scales; every part bitwise the oracle's."""
    from tie_rows import NAMED, tie_rows
    x, want = tie_rows(23, k, seed=k + parts, dtype=x_dtype)
    xt = torch.from_numpy(x)
    xd = xt.to(DEV)
    q, qs, ldq = lowbit.quantize(xd, (0, k, 1, 23), 23, k, parts, qs_dtype=qs_dtype)
    torch.cuda.synchronize()
    got = q.cpu().numpy()
    assert np.array_equal(got[0, :, :k], want)
    s0 = qs.cpu().float().numpy()[0]
    for h, c in NAMED.items():
        cols = np.nonzero(x[0].astype(np.float64) == h * float(s0[0]))[0]
        assert cols.size and (got[0, 0, cols] == c).all(), h
    rq, rqs = O.quantize(x, parts, ldq=ldq, qs_f16=qs_dtype == torch.float16)
    assert np.array_equal(got, rq)
    assert np.array_equal(qs.cpu().float().numpy(), rqs)


@torch.inference_mode()
def test_graph_replays_match_eager():
    """Captured launches replayed several times, with eager work between replays, equal the eager result."""
    case = Case(1, 1, 128, 1024, 1024, seed=12)
    y_eager, acc_eager = case.run()
    y = torch.zeros(case.m, case.n, device=DEV, dtype=torch.float16)
    stream = torch.cuda.Stream()
    with torch.cuda.stream(stream):
        lowbit.gemm(1, case.dq, case.dqs, case.words, case.n, case.k, case.dalpha, None, y, None)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=stream):
        for _ in range(3):
            lowbit.gemm(1, case.dq, case.dqs, case.words, case.n, case.k, case.dalpha, None, y, None)
    for i in range(4):
        y.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y.cpu().view(torch.int16), y_eager.view(torch.int16)), f"replay {i}"
        case.run()  # eager work between replays


# --- per-group weight scales ---------------------------------------------------------------------------------------

def _group_run(case, ws_group, alpha_g, *, out_dtype, silu=False, order=0, config=None):
    """Runs the GEMM with alpha_g [N, G] group scales (dtype of case.qs)."""
    y = torch.full((case.m, case.n), float("nan"), device=DEV, dtype=out_dtype)
    a = torch.full((case.p, case.m, case.n), -7, device=DEV, dtype=torch.int32)
    lowbit.gemm(case.wbits, case.dq, case.dqs, case.words, case.n, case.k, alpha_g.to(DEV), case.dbias, y, a,
                silu=silu, order=order, config=config, ws_group=ws_group)
    torch.cuda.synchronize()
    return y.cpu(), a.cpu().numpy()


def _group_ref(case, ws_group, alpha_g, *, silu=False, order=0):
    fn = O.b1_gemm if case.wbits == 1 else O.t2_gemm
    acc_g = fn(case.q.numpy(), case.codes, case.k, group=ws_group)
    bias = None if case.bias is None else case.bias.float().numpy()
    y = O.epilogue(acc_g, case.qs.float().numpy(), alpha_g.float().numpy(), bias, silu=silu, order=order)
    return y, acc_g.sum(axis=0, dtype=np.int64).astype(np.int32)


@pytest.mark.parametrize("wbits", [1, 2])
@pytest.mark.parametrize("ws_group", [64, 128, 256])
@pytest.mark.parametrize("p", [1, 3])
@torch.inference_mode()
def test_group_scales_bitwise(wbits, ws_group, p):
    case = Case(wbits, p, 70, 300, 1000, seed=ws_group + p + wbits, bias=True)
    groups = -(-case.k // ws_group)
    g = torch.Generator().manual_seed(ws_group * 7 + p)
    alpha_g = (torch.rand(case.n, groups, generator=g) * 0.09 + 0.01).to(case.qs.dtype)
    y, acc = _group_run(case, ws_group, alpha_g, out_dtype=torch.float32, order=p % 2)
    ref_y, ref_acc = _group_ref(case, ws_group, alpha_g, order=p % 2)
    assert np.array_equal(acc, ref_acc)
    bad = np.argwhere(y.numpy().view(np.uint32) != ref_y.view(np.uint32))
    assert bad.size == 0, f"{bad.shape[0]} mismatches, first {bad[:5].tolist()}"


@torch.inference_mode()
def test_config2_ternary_group128_fp16():
    """BASELINE config 2 with group-128 fp16 scales [1024, 32], fp16 output."""
    case = Case(2, 1, 128, 1024, 4096, seed=22)
    g = torch.Generator().manual_seed(23)
    alpha_g = (torch.rand(case.n, 32, generator=g) * 0.09 + 0.01).to(torch.float16)
    y, acc = _group_run(case, 128, alpha_g, out_dtype=torch.float16)
    ref_y, ref_acc = _group_ref(case, 128, alpha_g)
    assert np.array_equal(acc, ref_acc)
    assert np.array_equal(_gpu_bits(y, torch.float16), O.to_f16_bits(ref_y))
    # tile 1 and tile 4 give the same bits
    y1, _ = _group_run(case, 128, alpha_g, out_dtype=torch.float16, config=kernels.GemmConfig(tile=1, split=1))
    assert torch.equal(y1.view(torch.int16), y.view(torch.int16))


@pytest.mark.parametrize("wbits,p,m,n,k", [(2, 1, 128, 1024, 4096), (1, 1, 70, 300, 1024), (2, 2, 37, 200, 2048),
                                           (1, 3, 16, 64, 1024), (2, 1, 1, 72, 4096)])
@pytest.mark.parametrize("ws_group", [64, 128, 256])
@torch.inference_mode()
def test_group_scales_on_every_wave_split_tile(wbits, p, m, n, k, ws_group):
    """Per-group scales on the wave-split tiles (each wave's int32 group sums through LDS, the fold in group order by
    one wave per block): every tile that takes groups at this K, bitwise the oracle's per-group rule, with bias, f16
    scales and f16 output; acc_out is the full-K sum."""
    case = Case(wbits, p, m, n, k, seed=k + n + ws_group + p, bias=True)
    groups = -(-k // ws_group)
    g = torch.Generator().manual_seed(ws_group + m)
    alpha_g = (torch.rand(n, groups, generator=g) * 0.09 + 0.01).to(case.qs.dtype)
    ref_y, ref_acc = _group_ref(case, ws_group, alpha_g, order=p % 2)
    ran = 0
    for tile in range(1, kernels.tile_count() + 1):
        if " k/" not in kernels.config_name(tile):
            continue
        try:
            y, acc = _group_run(case, ws_group, alpha_g, out_dtype=torch.float16, order=p % 2,
                                config=kernels.GemmConfig(tile=tile, split=1))
        except ValueError as e:
            # tiles that cannot take groups at this K, or whose registers cannot hold this many parts
            assert "per-group weight scales on wave-split tile" in str(e) or "does not fit" in str(e)
            continue
        assert np.array_equal(acc, ref_acc), kernels.config_name(tile)
        assert np.array_equal(_gpu_bits(y, torch.float16), O.to_f16_bits(ref_y)), kernels.config_name(tile)
        ran += 1
    assert ran >= 1


@pytest.mark.parametrize("seed", [31, 32])
@torch.inference_mode()
def test_seeded_random_group_scale_cases_bitwise(seed):
    """Per-group scales on random shapes: groups of 64, 128 or 256, ragged K, 1 to 3 parts, f32 / f16 scales, f32 / f16
    output, with and without bias, both epilogue orders, the library's tile choice (wave-split group tiles where K
    fits one workgroup, else the ring's group tiles) and, where K is a whole number of k-steps of 64 for 4 or 8
    waves, every wave-split tile that takes groups: y and acc_out bitwise the oracle's per-group rule."""
    rng = np.random.default_rng(seed)
    ran = 0
    for i in range(10):
        wbits, parts, ws_group = int(rng.integers(1, 3)), int(rng.integers(1, 4)), int(rng.choice([64, 128, 256]))
        m, n = int(rng.integers(1, 130)), int(rng.integers(1, 500))
        k = int(rng.choice([64 * 4 * int(rng.integers(1, 9)), 64 * 8 * int(rng.integers(1, 5)),
                            int(rng.integers(1, 2500))]))
        out_dtype = [torch.float32, torch.float16][int(rng.integers(0, 2))]
        case = Case(wbits, parts, m, n, k, seed=seed * 100 + i, bias=bool(rng.integers(0, 2)),
                    scale_dtype=[torch.float32, torch.float16][int(rng.integers(0, 2))])
        g = torch.Generator().manual_seed(seed * 100 + i)
        alpha_g = (torch.rand(n, -(-k // ws_group), generator=g) * 0.09 + 0.01).to(case.qs.dtype)
        order = int(rng.integers(0, 2))
        ref_y, ref_acc = _group_ref(case, ws_group, alpha_g, order=order)
        tiles = [None] + [t for t in range(1, kernels.tile_count() + 1) if " k/" in kernels.config_name(t)]
        for tile in tiles:
            config = None if tile is None else kernels.GemmConfig(tile=tile, split=1)
            try:
                y, acc = _group_run(case, ws_group, alpha_g, out_dtype=out_dtype, order=order, config=config)
            except ValueError as e:
                assert tile is not None and ("per-group weight scales on wave-split tile" in str(e)
                                             or "does not fit" in str(e)), str(e)
                continue
            assert np.array_equal(acc, ref_acc), (seed, i, tile)
            assert np.array_equal(_gpu_bits(y, out_dtype), _bits(ref_y, out_dtype)), (seed, i, tile)
            ran += 1
    assert ran >= 10


@pytest.mark.parametrize("k", [17, 300, 4096 + 64])
@torch.inference_mode()
def test_group_scales_ragged_k_and_silu(k):
    case = Case(1, 2, 33, 45, k, seed=k, bias=True, pad_garbage=True)
    groups = -(-k // 64)
    g = torch.Generator().manual_seed(k)
    alpha_g = (torch.rand(case.n, groups, generator=g) * 0.09 + 0.01).to(case.qs.dtype)
    y, acc = _group_run(case, 64, alpha_g, out_dtype=torch.float32)
    ref_y, ref_acc = _group_ref(case, 64, alpha_g)
    assert np.array_equal(acc, ref_acc)
    assert np.array_equal(y.numpy().view(np.uint32), ref_y.view(np.uint32))
    ys, _ = _group_run(case, 64, alpha_g, out_dtype=torch.float32, silu=True)
    ref_s, _ = _group_ref(case, 64, alpha_g, silu=True)
    np.testing.assert_allclose(ys.numpy(), ref_s, rtol=2e-6, atol=2e-6)


@torch.inference_mode()
def test_group_scales_reject_unsupported_arguments():
    case = Case(1, 1, 8, 64, 256, seed=3)
    alpha_g = torch.ones(64, 4, dtype=case.qs.dtype)
    with pytest.raises(ValueError, match="ws_group"):
        _group_run(case, 96, alpha_g, out_dtype=torch.float32)
    with pytest.raises(ValueError, match="tile configs"):
        _group_run(case, 64, alpha_g, out_dtype=torch.float32, config=kernels.GemmConfig(tile=2, split=1))
    with pytest.raises(ValueError, match="unsplit"):
        _group_run(case, 64, alpha_g, out_dtype=torch.float32, config=kernels.GemmConfig(tile=4, split=2))


# --- residual epilogue ------------------------------------------------------------------------------------------------

@pytest.mark.parametrize("wbits,p,m,n,k,split", [(1, 1, 125, 1024, 4096, 1), (1, 3, 38, 1024, 4096, 4),
                                                 (2, 2, 300, 512, 640, 1), (1, 1, 1000, 1024, 1024, 1)])
@pytest.mark.parametrize("in_place", [False, True])
@torch.inference_mode()
def test_residual_epilogue_bitwise(wbits, p, m, n, k, split, in_place):
    """y = residual + value * factor (IEEE multiply, then add) on the unsplit and the split-K (finish) paths."""
    case = Case(wbits, p, m, n, k, seed=m + n + p, bias=True, scale_dtype=torch.float32)
    g = torch.Generator().manual_seed(m * 3 + split)
    res = torch.randn(m, n, generator=g)
    factor = 0.5
    dres = res.to(DEV)
    y = dres if in_place else torch.empty(m, n, device=DEV)
    lowbit.gemm(case.wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, case.dbias, y, None,
                config=kernels.GemmConfig(tile=1 if p > 1 else 4, split=split), residual=dres, residual_factor=factor)
    torch.cuda.synchronize()
    value = case.oracle_y(case.oracle_acc())
    want = (res.numpy() + value * np.float32(factor)).astype(np.float32)
    got = y.cpu().numpy()
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("wbits,p,m,n,k,split", [(1, 1, 37, 300, 1024, 0), (2, 2, 37, 300, 640, 0),
                                                 (1, 1, 37, 300, 4096, 2), (1, 3, 19, 72, 1100, 0)])
@pytest.mark.parametrize("in_place", [False, True])
@torch.inference_mode()
def test_residual_epilogue_bitwise_on_every_wave_split_tile(wbits, p, m, n, k, split, in_place):
    """The wave-split kernel loads its residual values with the epilogue's scales, before the MFMAs, from clamped rows
    and columns (partial M and N blocks, an unused clamped block when a wave finishes more blocks than exist): on
    every wave-split tile, unsplit and split, in place and not, y = residual + value * factor bitwise."""
    case = Case(wbits, p, m, n, k, seed=m + n + p + k, bias=True, scale_dtype=torch.float32)
    g = torch.Generator().manual_seed(m * 5 + k)
    res = torch.randn(m, n, generator=g)
    factor = 0.5
    want = (res.numpy() + case.oracle_y(case.oracle_acc()) * np.float32(factor)).astype(np.float32)
    ran = 0
    for tile in range(1, kernels.tile_count() + 1):
        if " k/" not in kernels.config_name(tile):
            continue
        dres = res.to(DEV)
        y = dres if in_place else torch.full((m, n), float("nan"), device=DEV)
        try:
            lowbit.gemm(case.wbits, case.dq, case.dqs, case.words, n, k, case.dalpha, case.dbias, y, None,
                        config=kernels.GemmConfig(tile=tile, split=split), residual=dres, residual_factor=factor)
        except ValueError as e:
            if "does not fit" in str(e) or "unsplit K range" in str(e):
                continue  # registers that cannot hold this many parts, or a ragged K range too long for one workgroup
            raise
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), kernels.config_name(tile)
        ran += 1
    assert ran >= 5


@torch.inference_mode()
def test_residual_epilogue_with_group_scales():
    case = Case(2, 1, 70, 300, 1000, seed=5, bias=True, scale_dtype=torch.float32)
    g = torch.Generator().manual_seed(6)
    alpha_g = (torch.rand(case.n, 8, generator=g) * 0.09 + 0.01)
    res = torch.randn(case.m, case.n, generator=g)
    y = torch.empty(case.m, case.n, device=DEV)
    lowbit.gemm(2, case.dq, case.dqs, case.words, case.n, case.k, alpha_g.to(DEV), case.dbias, y, None,
                ws_group=128, residual=res.to(DEV), residual_factor=0.25)
    torch.cuda.synchronize()
    ref_y, _ = _group_ref(case, 128, alpha_g)
    want = (res.numpy() + ref_y * np.float32(0.25)).astype(np.float32)
    assert np.array_equal(y.cpu().numpy().view(np.uint32), want.view(np.uint32))
