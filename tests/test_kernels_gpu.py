"""Kernel-level parity on the GPU, through the C ABI (laya_op_*), against NumPy oracles.

Mirrors the reference's kernel tests (tests/test_gpu.py, tests/test_attention.py): bit-exact
gathers and residual adds, bias-before-rounding, LayerNorm and GEMM tolerances, packed ragged
attention with padding rows returning exact zeros.  Device memory comes from torch (plumbing
only); every computation runs in liblaya_hip.
"""
import ctypes as ct
import math

import numpy as np
import pytest

import oracle.encoder as E
from laya_cuda import _lib

pytestmark = pytest.mark.gpu

DTYPES = {"f16": (_lib.F16, np.float16), "bf16": (_lib.BF16, None)}


def torch():
    import torch as t
    return t


def dev(array, device):
    t = torch()
    return t.from_numpy(np.ascontiguousarray(array)).to(device)


def p(tensor):
    return ct.c_void_p(tensor.data_ptr()) if tensor is not None else None


def stream():
    return ct.c_void_p(torch().cuda.current_stream().cuda_stream)


def sync():
    torch().cuda.synchronize()


def half_round(a, kind):
    """Round float32 values to the 16-bit operand type, as float32."""
    from laya_cuda.synthetic import bf16_round
    a = np.asarray(a, np.float32)
    return a.astype(np.float16).astype(np.float32) if kind == "f16" else bf16_round(a)


def to16(a, kind, device):
    t = torch()
    x = dev(half_round(a, kind), device)
    return x.to(t.float16 if kind == "f16" else t.bfloat16)


def from16(x):
    return x.float().cpu().numpy()


def check(code):
    _lib.check(code)


# ---------------- embedding gather + LayerNorm ----------------

def test_embed_gather_is_bit_exact(gpu):
    t = torch()
    lib = _lib.load()
    rng = np.random.default_rng(1)
    table = rng.normal(0, 1, (1000, 768)).astype(np.float32)
    pos = rng.normal(0, 1, (64, 768)).astype(np.float32)
    typ = rng.normal(0, 1, (2, 768)).astype(np.float32)
    ids = np.array([0, 999, 3, 3, 17, 500, 3, 999], np.int32)
    positions = np.array([0, 1, 2, 3, 63, 5, 6, 0], np.int32)
    d_ids, d_pos, d_table, d_ptab, d_type = (dev(a, gpu) for a in (ids, positions, table, pos, typ))
    out = t.full((len(ids), 768), float("nan"), device=gpu)
    check(lib.laya_op_embed(p(d_ids), p(d_pos), p(d_table), None, None, None, None, 0.0, p(out), None, _lib.F16,
                            len(ids), 768, 1000, 64, stream()))
    sync()
    np.testing.assert_array_equal(out.cpu().numpy(), table[ids])
    check(lib.laya_op_embed(p(d_ids), p(d_pos), p(d_table), p(d_ptab), p(d_type), None, None, 0.0, p(out), None,
                            _lib.F16, len(ids), 768, 1000, 64, stream()))
    sync()
    np.testing.assert_array_equal(out.cpu().numpy(), (table[ids] + pos[positions]) + typ[0])


@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("width", [128, 768, 1024])
def test_embed_norm_matches_oracle(gpu, kind, width):
    t = torch()
    lib = _lib.load()
    rng = np.random.default_rng(width)
    table = rng.normal(0, .5, (300, width)).astype(np.float32)
    pos = rng.normal(0, .5, (128, width)).astype(np.float32)
    typ = rng.normal(0, .5, (2, width)).astype(np.float32)
    gamma, beta = rng.normal(1, .1, width).astype(np.float32), rng.normal(0, .1, width).astype(np.float32)
    ids = rng.integers(0, 300, 77).astype(np.int32)
    positions = np.arange(77, dtype=np.int32)
    out32 = t.full((77, width), float("nan"), device=gpu)
    out16 = t.empty((77, width), dtype=t.float16 if kind == "f16" else t.bfloat16, device=gpu)
    args = [dev(a, gpu) for a in (ids, positions, table, pos, typ, gamma, beta)]
    check(lib.laya_op_embed(*[p(a) for a in args], 1e-12, p(out32), p(out16), DTYPES[kind][0], 77, width, 300, 128,
                            stream()))
    sync()
    expected = E.layer_norm((table[ids] + pos[positions]) + typ[0], gamma, beta, 1e-12)
    np.testing.assert_allclose(out32.cpu().numpy(), expected, atol=2e-5, rtol=1e-5)
    np.testing.assert_array_equal(from16(out16), half_round(out32.cpu().numpy(), kind))


# ---------------- residual add + LayerNorm ----------------

@pytest.mark.parametrize("width", [64, 768, 1024, 1088])
@pytest.mark.parametrize("normalize,out32", [(False, False), (False, True), (True, False), (True, True)])
def test_norm_residual_and_aliases(gpu, width, normalize, out32):
    """tests/test_gpu.py:79-103 of the reference: residual add bit-exact, LN within tolerance,
    fp32 output aliasing the residual (in-place post-LN)."""
    t = torch()
    lib = _lib.load()
    rng = np.random.default_rng(31)
    source = rng.normal(2, .3, (3, width)).astype(np.float32)
    branch = rng.normal(0, .1, (3, width)).astype(np.float32)
    gamma, beta = rng.normal(1, .1, width).astype(np.float32), rng.normal(0, .1, width).astype(np.float32)
    residual, d_branch, d_g, d_b = (dev(a, gpu) for a in (source, branch, gamma, beta))
    added = source + branch
    if out32:
        out, out16, sum_out = residual, None, None
    else:
        out, out16, sum_out = None, t.empty((3, width), dtype=t.float16, device=gpu), residual
    check(lib.laya_op_norm(p(residual), p(d_branch), 1, 0, None, p(d_g) if normalize else None,
                           p(d_b) if normalize else None, 1e-5, p(sum_out), p(out), p(out16), _lib.F16, 3, width,
                           stream()))
    sync()
    got = residual.cpu().numpy() if out32 else from16(out16)
    if normalize:
        a64 = added.astype(np.float64)
        expected = (a64 - a64.mean(-1, keepdims=True)) / np.sqrt(a64.var(-1, keepdims=True) + 1e-5) * gamma + beta
        np.testing.assert_allclose(got, expected, atol=2e-5 if out32 else 4e-3, rtol=1e-5 if out32 else 2e-3)
    else:
        np.testing.assert_array_equal(got, added if out32 else added.astype(np.float16).astype(np.float32))
    if not out32:
        np.testing.assert_array_equal(residual.cpu().numpy(), added)


def test_norm_sums_split_partials_and_bias_in_order(gpu):
    lib = _lib.load()
    rng = np.random.default_rng(2)
    rows, width, splits = 5, 768, 3
    res = rng.normal(0, 1, (rows, width)).astype(np.float32)
    parts = rng.normal(0, 1, (splits, rows, width)).astype(np.float32)
    bias = rng.normal(0, 1, width).astype(np.float32)
    d_res, d_parts, d_bias = (dev(a, gpu) for a in (res, parts, bias))
    check(lib.laya_op_norm(p(d_res), p(d_parts), splits, rows * width, p(d_bias), None, None, 1e-5, None, p(d_res),
                           None, _lib.F16, rows, width, stream()))
    sync()
    np.testing.assert_array_equal(d_res.cpu().numpy(), res + (((parts[0] + parts[1]) + parts[2]) + bias))


# ---------------- option-row gathers (decision head) ----------------

@pytest.mark.parametrize("kind", ["f16", "bf16"])
@pytest.mark.parametrize("width", [64, 768, 1024])
def test_option_row_gather_is_bit_exact(gpu, kind, width):
    """tests/test_gpu.py:106-112 of the reference: gathered rows keep the order of the indices,
    duplicates included, bit for bit; here in fp32 and 16-bit at once, with rows past the live
    count written as zeros."""
    t = torch()
    lib = _lib.load()
    rng = np.random.default_rng(width)
    values = rng.normal(0, 3, (40, width)).astype(np.float32)
    values[5, :7] = [0.0, -0.0, np.inf, -np.inf, 1e-40, -3e38, 65504.0]  # signed zero, inf, subnormal
    indices = np.array([0, 39, 3, 3, 1, 5, 39, 0, 22, 7, 7], np.int32)
    live, rows = 9, len(indices)
    half = t.float16 if kind == "f16" else t.bfloat16
    src32 = dev(values, gpu)
    src16 = dev(values, gpu).to(half)
    dst32 = t.full((rows, width), float("nan"), device=gpu)
    dst16 = t.full((rows, width), float("nan"), device=gpu).to(half)
    d_idx, d_live = dev(indices, gpu), dev(np.array([live], np.int32), gpu)
    check(lib.laya_op_gather_rows(p(src32), p(dst32), p(src16), p(dst16), DTYPES[kind][0], p(d_idx), p(d_live), rows,
                                  width, stream()))
    sync()
    got32 = dst32.cpu().numpy()
    np.testing.assert_array_equal(got32[:live].view(np.uint32), values[indices[:live]].view(np.uint32))
    assert not got32[live:].view(np.uint32).any()
    bits16 = src16.view(t.int16).cpu().numpy()
    got16 = dst16.view(t.int16).cpu().numpy()
    np.testing.assert_array_equal(got16[:live], bits16[indices[:live]])
    assert not got16[live:].any()
    # The 16-bit copy alone (the fp32 pair skipped): fp32 rows stay as they were.
    dst32.fill_(7.0)
    dst16.zero_()
    check(lib.laya_op_gather_rows(None, None, p(src16), p(dst16), DTYPES[kind][0], p(d_idx), p(d_live), rows, width,
                                  stream()))
    sync()
    np.testing.assert_array_equal(dst16.view(t.int16).cpu().numpy()[:live], bits16[indices[:live]])
    assert (dst32.cpu().numpy() == 7.0).all()


@pytest.mark.parametrize("width", [768, 1024])
def test_head_gather_adds_type_rows_bit_exactly(gpu, width):
    """type_add + gather (kernels.cu:155-162; laya.py:236-238): each scorer row is its packed
    source row plus its question's type row, one fp32 add (bit-exact), then scorer.0's LayerNorm
    (eps 1e-5).  Rows past the live count are not written."""
    t = torch()
    lib = _lib.load()
    rng = np.random.default_rng(7)
    residual = rng.normal(0, 1, (64, width)).astype(np.float32)
    types = rng.normal(0, 1, (3, width)).astype(np.float32)
    gamma, beta = rng.normal(1, .1, width).astype(np.float32), rng.normal(0, .1, width).astype(np.float32)
    src_rows = np.array([0, 17, 17, 63, 2, 40, 0, 9], np.int32)      # CLS, options, ... (duplicates)
    row_question = np.array([0, 0, 0, 0, 1, 1, 2, 2], np.int32)
    question_kind = np.array([2, 0, 1], np.int32)
    live, rows = 7, 8
    selected = t.full((rows, width), float("nan"), device=gpu)
    normed = t.full((rows, width), float("nan"), device=gpu)
    args = [dev(a, gpu) for a in (residual, src_rows, row_question, question_kind, np.array([live], np.int32), types,
                                  gamma, beta)]
    check(lib.laya_op_head_gather(*[p(a) for a in args], 1e-5, p(selected), p(normed), rows, width, stream()))
    sync()
    want = residual[src_rows] + types[question_kind[row_question]]
    got = selected.cpu().numpy()
    np.testing.assert_array_equal(got[:live].view(np.uint32), want[:live].view(np.uint32))
    np.testing.assert_allclose(normed.cpu().numpy()[:live], E.layer_norm(want[:live], gamma, beta, 1e-5),
                               atol=2e-5, rtol=1e-5)
    assert np.isnan(got[live:]).all() and np.isnan(normed.cpu().numpy()[live:]).all()
    # Without type rows the scorer rows are plain copies.
    check(lib.laya_op_head_gather(p(args[0]), p(args[1]), None, None, p(args[4]), None, p(args[6]), p(args[7]), 1e-5,
                                  p(selected), p(normed), rows, width, stream()))
    sync()
    np.testing.assert_array_equal(selected.cpu().numpy()[:live].view(np.uint32),
                                  residual[src_rows[:live]].view(np.uint32))


# ---------------- MFMA GEMM ----------------

def linear(x, w, bias, out, kind, dtype, M, N, K, splits, tile):
    check(_lib.load().laya_op_linear(p(x), p(w), p(bias), p(out), kind, DTYPES[dtype][0], M, N, K, splits, tile,
                                     stream()))
    sync()


GEMM_TILES = 27  # tile ids of laya_op_linear (csrc/gemm.hip kTiles)
TILE_BN = {21: 192}  # tiles whose width is not a power of two
PERSISTENT = {26}  # tiles looping over output tiles: 16-bit epilogues without RoPE only


def ncols(N, tile):
    """N rounded down to a multiple of the tile's width (other tiles divide every N used here)."""
    bn = TILE_BN.get(tile)
    return N if bn is None else max(bn, N // bn * bn)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("tile", [t for t in range(GEMM_TILES) if t not in PERSISTENT])
def test_linear_tiles_match_fp32_product(gpu, dtype, tile):
    t = torch()
    rng = np.random.default_rng(tile)
    for M, N, K in [(96, 768, 768), (300, 512, 1024), (512, 256, 128)]:
        N = ncols(N, tile)
        x = half_round(rng.normal(0, 1, (M, K)), dtype)
        w = half_round(rng.normal(0, 1 / math.sqrt(K), (N, K)), dtype)
        out = t.full((M, N), float("nan"), device=gpu)
        linear(to16(x, dtype, gpu), to16(w, dtype, gpu), None, out, 0, dtype, M, N, K, 1, tile)
        np.testing.assert_allclose(out.cpu().numpy(), x.astype(np.float64) @ w.T.astype(np.float64),
                                   atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("kind", [1, 2])
@pytest.mark.parametrize("tile", range(GEMM_TILES))
def test_linear_16bit_epilogues_every_tile(gpu, tile, kind):
    """Bias, optional GELU and the single rounding through each tile's staged row stores, with
    rows past a tile boundary."""
    t = torch()
    rng = np.random.default_rng(100 + tile)
    M, N, K = 300, ncols(512, tile), 256
    x = half_round(rng.normal(0, 1, (M, K)), "f16")
    w = half_round(rng.normal(0, 1 / math.sqrt(K), (N, K)), "f16")
    bias = rng.normal(0, .5, N).astype(np.float32)
    out = t.full((M, N), float("nan"), dtype=t.float16, device=gpu)
    linear(to16(x, "f16", gpu), to16(w, "f16", gpu), dev(bias, gpu), out, kind, "f16", M, N, K, 1, tile)
    expected = (x.astype(np.float64) @ w.T.astype(np.float64) + bias).astype(np.float32)
    if kind == 2:
        expected = E.gelu(expected)
    np.testing.assert_allclose(from16(out), expected, atol=2e-3, rtol=2e-3)


@pytest.mark.parametrize("tile", [5, 11, 12, 14, 17, 19, 21])
@pytest.mark.parametrize("splits", [2, 3, 4])
def test_linear_split_k_partials_sum_to_the_product(gpu, splits, tile):
    t = torch()
    rng = np.random.default_rng(splits)
    M, N, K = 64, 768, 3072
    x = half_round(rng.normal(0, 1, (M, K)), "f16")
    w = half_round(rng.normal(0, 1 / math.sqrt(K), (N, K)), "f16")
    out = t.full((splits, M, N), float("nan"), device=gpu)
    linear(to16(x, "f16", gpu), to16(w, "f16", gpu), None, out, 0, "f16", M, N, K, splits, tile)
    np.testing.assert_allclose(out.sum(0).cpu().numpy(), x.astype(np.float64) @ w.T.astype(np.float64),
                               atol=1e-4, rtol=1e-4)


@pytest.mark.parametrize("kind", [1, 2, 3, 4])
@pytest.mark.parametrize("M,N,K", [(16421, 2048, 192), (30000, 768, 320), (8192, 8192, 1024)])
def test_persistent_tile_walks_many_tiles_per_workgroup(gpu, kind, M, N, K):
    """Tile 26 runs at most one workgroup per CU, each walking several 256x256 output tiles with
    the next tile's first slabs loaded during the current tile's last ones.  On 256 CUs: 520 tiles
    (two or three per workgroup) with a partial last row tile and the three-slab minimum, 354
    tiles (a count that is not a multiple of 8, so the plain tile order), and 1,024 tiles (four
    per workgroup).  Reference: torch fp32 on the same 16-bit operands."""
    t = torch()
    g = t.Generator(device=gpu).manual_seed(M + K + kind)
    x = t.randn((M, K), generator=g, device=gpu).half()
    w = (t.randn((N, K), generator=g, device=gpu) / math.sqrt(K)).half()
    bias = t.randn(N, generator=g, device=gpu) * 0.5
    ref = t.addmm(bias, x.float(), w.float().t())
    if kind == 2:
        ref = t.nn.functional.gelu(ref)
    elif kind == 3:
        ref = t.relu(ref)
    elif kind == 4:  # GeGLU over the 32-row interleave: 16 gate rows, then their 16 value rows
        groups = ref.view(M, N // 32, 2, 16)
        ref = (t.nn.functional.gelu(groups[:, :, 0]) * groups[:, :, 1]).reshape(M, N // 2)
    out = t.full((M, N // 2 if kind == 4 else N), float("nan"), dtype=t.float16, device=gpu)
    lib = _lib.load()
    check(lib.laya_op_linear(p(x), p(w), None if kind == 4 else p(bias), p(out), kind, _lib.F16, M, N, K, 1, 26,
                             stream()))
    sync()
    if kind == 4:  # the GeGLU epilogue takes no bias: compare against the product without it
        groups = t.mm(x.float(), w.float().t()).view(M, N // 32, 2, 16)
        ref = (t.nn.functional.gelu(groups[:, :, 0]) * groups[:, :, 1]).reshape(M, N // 2)
    got = out.float()
    assert t.isfinite(got).all()
    err = (got - ref).abs().max().item()
    assert err <= 2e-3 * max(1.0, ref.abs().max().item()), err


def test_persistent_qkv_walks_many_tiles_per_workgroup(gpu):
    """The head-major QKV epilogue on tile 26 with several tiles per workgroup: integer-valued
    operands make the product exact, so the layout check is bit-exact."""
    t = torch()
    rng = np.random.default_rng(26)
    M, heads = 8200, 16  # 33 row tiles x 12 column tiles = 396 tiles
    width = heads * 64
    x = rng.integers(-3, 4, (M, width)).astype(np.float32)
    w = rng.integers(-2, 3, (3 * width, width)).astype(np.float32)
    bias = rng.integers(-4, 5, 3 * width).astype(np.float32)
    q, k, vt = (t.full((heads * M * 64,), float("nan"), dtype=t.float16, device=gpu) for _ in range(3))
    d_x, d_w, d_bias = to16(x, "f16", gpu), to16(w, "f16", gpu), dev(bias, gpu)
    check(_lib.load().laya_op_qkv(p(d_x), p(d_w), p(d_bias), p(q), p(k), p(vt), None, None, None, _lib.F16, M, width,
                                  26, stream()))
    sync()
    full = x @ w.T + bias
    parts = full.reshape(M, 3, heads, 64)
    np.testing.assert_array_equal(q.cpu().numpy().reshape(heads, M, 64), parts[:, 0].transpose(1, 0, 2))
    np.testing.assert_array_equal(k.cpu().numpy().reshape(heads, M, 64), parts[:, 1].transpose(1, 0, 2))
    np.testing.assert_array_equal(vt.cpu().numpy().reshape(heads, 64, M), parts[:, 2].transpose(1, 2, 0))


def test_persistent_tile_refuses_fp32_rope_and_short_k(gpu):
    """Tile 26 stages its epilogue in one 32 KB ring buffer (16-bit outputs only), has no RoPE form
    and needs three 64-deep slabs per tile: those launches return an error instead of running."""
    t = torch()
    M, width = 512, 256
    x = t.zeros((M, 1024), dtype=t.float16, device=gpu)
    w = t.zeros((3 * width, 1024), dtype=t.float16, device=gpu)
    out32 = t.zeros((M, width), device=gpu)
    out16 = t.zeros((M, width), dtype=t.float16, device=gpu)
    lib = _lib.load()
    assert lib.laya_op_linear(p(x), p(w), None, p(out32), 0, _lib.F16, M, width, 1024, 1, 26, stream()) != 0
    assert lib.laya_op_linear(p(x), p(w), None, p(out16), 1, _lib.F16, M, width, 128, 1, 26, stream()) != 0
    assert lib.laya_op_linear(p(x), p(w), None, p(out16), 1, _lib.F16, M, width, 192, 1, 26, stream()) == 0
    q, k, vt = (t.zeros((M * width,), dtype=t.float16, device=gpu) for _ in range(3))
    cos, sin = t.ones((M, 32), device=gpu), t.zeros((M, 32), device=gpu)
    pos = t.zeros(M, dtype=t.int32, device=gpu)
    assert lib.laya_op_qkv(p(x), p(w), None, p(q), p(k), p(vt), p(cos), p(sin), p(pos), _lib.F16, M, width, 26,
                           stream()) != 0
    sync()


def test_linear_adds_bias_before_rounding(gpu):
    """tests/test_gpu.py:56-65 of the reference: (x w^T + b) rounded once."""
    t = torch()
    x = np.zeros((1, 64), np.float32)
    x[0, :2] = [1, .0006]
    w = np.ones((128, 64), np.float32)
    bias = np.full(128, -1, np.float32)
    out = t.empty((1, 128), dtype=t.float16, device=gpu)
    linear(to16(x, "f16", gpu), to16(w, "f16", gpu), dev(bias, gpu), out, 1, "f16", 1, 128, 64, 1, 6)
    x16 = x.astype(np.float16).astype(np.float32)
    oracle = (x16 @ w.T + bias).astype(np.float16)
    np.testing.assert_array_equal(out.cpu().numpy(), oracle)
    assert oracle[0, 0] != 0  # rounding before the bias would give exactly zero


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_linear_gelu_epilogue(gpu, dtype):
    t = torch()
    rng = np.random.default_rng(9)
    M, N, K = 128, 3072, 768
    x = half_round(rng.normal(0, 1, (M, K)), dtype)
    w = half_round(rng.normal(0, 2 / math.sqrt(K), (N, K)), dtype)
    bias = rng.normal(0, .5, N).astype(np.float32)
    out = t.empty((M, N), dtype=t.float16 if dtype == "f16" else t.bfloat16, device=gpu)
    linear(to16(x, dtype, gpu), to16(w, dtype, gpu), dev(bias, gpu), out, 2, dtype, M, N, K, 1, -1)
    expected = E.gelu((x.astype(np.float64) @ w.T.astype(np.float64) + bias).astype(np.float32))
    tol = 2e-3 if dtype == "f16" else 1e-2
    np.testing.assert_allclose(from16(out), expected, atol=tol, rtol=tol)


def test_sixteen_wide_mfma_tile_refuses_rope_and_geglu(gpu):
    """Tile 22 (the ring with 16x16x32 MFMAs) serves the row-major and head-major epilogues; the
    GeGLU and RoPE epilogues, which assume the 32x32 accumulator order, are refused with an error
    instead of running."""
    t = torch()
    M, width = 256, 256
    x = t.zeros((M, width), dtype=t.float16, device=gpu)
    w = t.zeros((2 * width, width), dtype=t.float16, device=gpu)
    out = t.zeros((M, width), dtype=t.float16, device=gpu)
    lib = _lib.load()
    assert lib.laya_op_linear(p(x), p(w), None, p(out), 4, _lib.F16, M, 2 * width, width, 1, 22, stream()) != 0
    wq = t.zeros((3 * width, width), dtype=t.float16, device=gpu)
    q, k, vt = (t.zeros((M * width,), dtype=t.float16, device=gpu) for _ in range(3))
    cos, sin = t.ones((M, 32), device=gpu), t.zeros((M, 32), device=gpu)
    pos = t.zeros(M, dtype=t.int32, device=gpu)
    assert lib.laya_op_qkv(p(x), p(wq), None, p(q), p(k), p(vt), p(cos), p(sin), p(pos), _lib.F16, M, width, 22,
                           stream()) != 0
    assert lib.laya_op_qkv(p(x), p(wq), None, p(q), p(k), p(vt), None, None, None, _lib.F16, M, width, 22,
                           stream()) == 0
    sync()


@pytest.mark.parametrize("tile", [0, 2, 5, 6, 7, 9, 11, 12, 13, 14, 16, 18, 19, 20, 21, 22, 26])
def test_qkv_epilogue_writes_head_major_layout(gpu, tile):
    """Integer-valued operands make the product exact, so the layout check is bit-exact."""
    t = torch()
    rng = np.random.default_rng(tile)
    M, heads = 96, 4
    width = heads * 64
    x = rng.integers(-3, 4, (M, width)).astype(np.float32)
    w = rng.integers(-2, 3, (3 * width, width)).astype(np.float32)
    bias = rng.integers(-4, 5, 3 * width).astype(np.float32)
    q, k, vt = (t.full((heads * M * 64,), float("nan"), dtype=t.float16, device=gpu) for _ in range(3))
    # Keep every operand referenced until the kernel has run: a temporary freed inside the argument
    # list returns its memory to torch's caching allocator, which hands it to the next operand.
    d_x, d_w, d_bias = to16(x, "f16", gpu), to16(w, "f16", gpu), dev(bias, gpu)
    check(_lib.load().laya_op_qkv(p(d_x), p(d_w), p(d_bias), p(q), p(k), p(vt), None, None, None, _lib.F16, M, width,
                                  tile, stream()))
    sync()
    full = x @ w.T + bias  # [M, 3*width], exact in fp32 and fp16
    parts = full.reshape(M, 3, heads, 64)
    np.testing.assert_array_equal(q.cpu().numpy().reshape(heads, M, 64), parts[:, 0].transpose(1, 0, 2))
    np.testing.assert_array_equal(k.cpu().numpy().reshape(heads, M, 64), parts[:, 1].transpose(1, 0, 2))
    np.testing.assert_array_equal(vt.cpu().numpy().reshape(heads, 64, M), parts[:, 2].transpose(1, 2, 0))


# ---------------- fused attention ----------------

def span(n):
    return -(-n // 16) * 16


@pytest.mark.parametrize("mode,waves", [(0, 1), (0, 2), (0, 4), (0, 8), (1, 2), (1, 4), (1, 8), (2, 4), (2, 8)])
@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("lengths", [[32], [7, 96], [128, 1], [250, 131], [256, 219, 145], [500], [1024, 333]])
def test_packed_attention_matches_float64(gpu, lengths, dtype, mode, waves):
    """tests/test_attention.py:12-56 of the reference (window -1): ragged packed rows, tokens past
    the last row, NaN-poisoned output, padding queries exactly zero."""
    t = torch()
    lib = _lib.load()
    h = 2
    starts = np.cumsum([0] + [span(n) for n in lengths])[:-1].astype(np.int32)
    m = span(sum(span(n) for n in lengths) + 16)
    x = half_round(np.random.default_rng(m).normal(0, 1, (m, 3, h, 64)), dtype)
    q = x[:, 0].transpose(1, 0, 2).copy()              # [h][m][64]
    k = x[:, 1].transpose(1, 0, 2).copy()
    vt = x[:, 2].transpose(1, 2, 0).copy()             # [h][64][m]
    max_tiles = m // 16
    block = lib.laya_attention_block(mode, waves)
    tiles = np.zeros(4 * max_tiles, np.int32)
    lens = np.asarray(lengths, np.int32)
    n = lib.laya_attention_tiles(starts.ctypes.data_as(ct.POINTER(ct.c_int32)), lens.ctypes.data_as(ct.POINTER(ct.c_int32)),
                                 len(lengths), m, block, tiles.ctypes.data_as(ct.POINTER(ct.c_int32)), max_tiles)
    assert n > 0
    out = t.full((m, h * 64), float("nan"), dtype=t.float16 if dtype == "f16" else t.bfloat16, device=gpu)
    args = [to16(a, dtype, gpu) for a in (q, k, vt)] + [out, dev(tiles, gpu)]

    def run():
        check(lib.laya_op_attention(*[p(a) for a in args], m, h, max_tiles, mode, waves, -1, DTYPES[dtype][0], stream()))
        sync()
        return from16(out)

    eager = run()
    out.fill_(float("nan"))
    np.testing.assert_array_equal(run(), eager)  # deterministic
    real = np.zeros(m, bool)
    atol, rtol = (6e-4, 1e-3) if dtype == "f16" else (4e-3, 8e-3)
    for start, n_tok in zip(starts, lengths):
        real[start:start + n_tok] = True
        qq, kk, vv = x[start:start + n_tok].astype(np.float64).transpose(1, 2, 0, 3)
        s = qq @ kk.transpose(0, 2, 1) / 8
        pr = np.exp(s - s.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        expected = (pr @ vv).transpose(1, 0, 2).reshape(n_tok, h * 64)
        np.testing.assert_allclose(eager[start:start + n_tok], expected, atol=atol, rtol=rtol)
    np.testing.assert_array_equal(eager[~real], 0)


# ---------------- ModernBERT-variant epilogues and local attention ----------------

def geglu_order(f):
    """Checkpoint row held by each resident row of a [2f][K] GeGLU matrix (32-row groups:
    16 gate rows, then their 16 value rows)."""
    r = np.arange(2 * f)
    group, within = r // 32, r % 32
    return np.where(within < 16, group * 16 + within, f + group * 16 + within - 16)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_linear_relu_epilogue(gpu, dtype):
    t = torch()
    rng = np.random.default_rng(21)
    M, N, K = 96, 512, 256
    x = half_round(rng.normal(0, 1, (M, K)), dtype)
    w = half_round(rng.normal(0, 1 / math.sqrt(K), (N, K)), dtype)
    bias = rng.normal(0, .5, N).astype(np.float32)
    d_x, d_w, d_b = to16(x, dtype, gpu), to16(w, dtype, gpu), dev(bias, gpu)
    out = t.empty((M, N), dtype=t.float16 if dtype == "f16" else t.bfloat16, device=gpu)
    linear(d_x, d_w, d_b, out, 3, dtype, M, N, K, 1, -1)
    expected = np.maximum(x.astype(np.float64) @ w.T.astype(np.float64) + bias, 0)
    tol = 2e-3 if dtype == "f16" else 1e-2
    np.testing.assert_allclose(from16(out), expected, atol=tol, rtol=tol)
    assert (from16(out) >= 0).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("tile", [-1, 2, 5, 7])
def test_linear_geglu_epilogue_on_interleaved_rows(gpu, dtype, tile):
    """gelu(x Wg^T) * (x Wv^T) (activate mode 2, kernels.cu:62-66) from one GEMM over the
    interleaved [2f][K] matrix; output [M][f] in feature order."""
    t = torch()
    rng = np.random.default_rng(22)
    M, f, K = 128, 1152, 256
    x = half_round(rng.normal(0, 1, (M, K)), dtype)
    w = half_round(rng.normal(0, 1.5 / math.sqrt(K), (2 * f, K)), dtype)  # checkpoint order: gate | value
    d_x, d_w = to16(x, dtype, gpu), to16(np.ascontiguousarray(w[geglu_order(f)]), dtype, gpu)
    out = t.full((M, f), float("nan"), dtype=t.float16 if dtype == "f16" else t.bfloat16, device=gpu)
    linear(d_x, d_w, None, out, 4, dtype, M, 2 * f, K, 1, tile)
    u = x.astype(np.float64) @ w.T.astype(np.float64)
    expected = E.gelu(u[:, :f].astype(np.float32)).astype(np.float64) * u[:, f:]
    tol = 3e-3 if dtype == "f16" else 2e-2
    np.testing.assert_allclose(from16(out), expected, atol=tol, rtol=tol)


@pytest.mark.parametrize("tile,heads", [(-1, 4), (2, 4), (4, 4), (7, 4), (10, 4), (11, 4), (12, 4), (13, 4), (-1, 3), (10, 3),
                                        (-1, 1)])
def test_qkv_epilogue_applies_rope_to_q_and_k(gpu, tile, heads):
    """RoPE in fp32 before the single rounding, matching the oracle's rotate-half on the same rows;
    odd head counts (3 * width not a multiple of 128) take the 128x64 tile."""
    import oracle.modernbert as MB
    t = torch()
    rng = np.random.default_rng(23)
    M = 160
    width = heads * 64
    x = half_round(rng.normal(0, 1, (M, width)), "f16")
    w = half_round(rng.normal(0, 1 / math.sqrt(width), (3 * width, width)), "f16")
    positions = np.concatenate([np.arange(96), np.arange(64)]).astype(np.int32)  # two packed sequences
    cos, sin = MB.rope_tables(10000.0, 128)
    q, k, vt = (t.full((heads * M * 64,), float("nan"), dtype=t.float16, device=gpu) for _ in range(3))
    d_x, d_w, d_c, d_s, d_p = to16(x, "f16", gpu), to16(w, "f16", gpu), dev(cos, gpu), dev(sin, gpu), dev(positions, gpu)
    check(_lib.load().laya_op_qkv(p(d_x), p(d_w), None, p(q), p(k), p(vt), p(d_c), p(d_s), p(d_p), _lib.F16, M, width,
                                  tile, stream()))
    sync()
    full = (x.astype(np.float64) @ w.T.astype(np.float64)).astype(np.float32).reshape(M, 3, heads, 64)
    cq, sq = cos[positions], sin[positions]
    want_q = MB.rope(full[:, 0], cq, sq).transpose(1, 0, 2)
    want_k = MB.rope(full[:, 1], cq, sq).transpose(1, 0, 2)
    np.testing.assert_allclose(from16(q).reshape(heads, M, 64), want_q, atol=3e-3, rtol=2e-3)
    np.testing.assert_allclose(from16(k).reshape(heads, M, 64), want_k, atol=3e-3, rtol=2e-3)
    np.testing.assert_allclose(from16(vt).reshape(heads, 64, M), full[:, 2].transpose(1, 2, 0), atol=3e-3, rtol=2e-3)


@pytest.mark.parametrize("mode,waves", [(0, 2), (0, 4), (0, 8), (1, 2), (1, 4), (1, 8), (2, 4), (2, 8)])
@pytest.mark.parametrize("lengths", [[250, 131], [500], [1024, 333], [40]])
def test_local_window_attention_matches_float64(gpu, lengths, mode, waves):
    """Local layers (kernels.cu:106-107): each query sees keys with |q - k| <= 64 of its sequence;
    blocks outside every query's window are skipped, partly masked ones masked per lane."""
    t = torch()
    lib = _lib.load()
    h, window = 2, 64
    starts = np.cumsum([0] + [span(n) for n in lengths])[:-1].astype(np.int32)
    m = span(sum(span(n) for n in lengths) + 16)
    x = half_round(np.random.default_rng(m + 1).normal(0, 1, (m, 3, h, 64)), "f16")
    q = x[:, 0].transpose(1, 0, 2).copy()
    k = x[:, 1].transpose(1, 0, 2).copy()
    vt = x[:, 2].transpose(1, 2, 0).copy()
    max_tiles = m // 16
    tiles = np.zeros(4 * max_tiles, np.int32)
    lens = np.asarray(lengths, np.int32)
    n = lib.laya_attention_tiles(starts.ctypes.data_as(ct.POINTER(ct.c_int32)), lens.ctypes.data_as(ct.POINTER(ct.c_int32)),
                                 len(lengths), m, lib.laya_attention_block(mode, waves),
                                 tiles.ctypes.data_as(ct.POINTER(ct.c_int32)), max_tiles)
    assert n > 0
    out = t.full((m, h * 64), float("nan"), dtype=t.float16, device=gpu)
    args = [to16(a, "f16", gpu) for a in (q, k, vt)] + [out, dev(tiles, gpu)]
    check(lib.laya_op_attention(*[p(a) for a in args], m, h, max_tiles, mode, waves, window, _lib.F16, stream()))
    sync()
    got = from16(out)
    real = np.zeros(m, bool)
    for start, n_tok in zip(starts, lengths):
        real[start:start + n_tok] = True
        qq, kk, vv = x[start:start + n_tok].astype(np.float64).transpose(1, 2, 0, 3)
        s = qq @ kk.transpose(0, 2, 1) / 8
        idx = np.arange(n_tok)
        s = np.where(np.abs(idx[:, None] - idx[None, :]) > window, -np.inf, s)
        pr = np.exp(s - s.max(-1, keepdims=True))
        pr /= pr.sum(-1, keepdims=True)
        expected = (pr @ vv).transpose(1, 0, 2).reshape(n_tok, h * 64)
        np.testing.assert_allclose(got[start:start + n_tok], expected, atol=6e-4, rtol=1e-3)
    np.testing.assert_array_equal(got[~real], 0)
