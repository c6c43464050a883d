"""GPU parity of the dequant / GEMM / matvec path against the oracle (through the C ABI).

Bar: dequant is bit-exact (fp16 payloads identical); GEMMs match an fp64 product
of the same fp16 activations and the exact RNE16 weights to within the fp16
output rounding plus fp32 accumulation-order noise; the fp32 matvec follows the
reference's own thresholds (LinearExecutorTests.swift:411-414,
MetalExecutionTests.swift:110,165).
"""

import numpy as np
import pytest
import torch

import animaxs_amd
from animaxs_amd import AnimaError, LinearExecutor, QuantizedLinearWeightBuffers
from oracle import inputs, quant
from tests.helpers import dev, device_weight

pytestmark = pytest.mark.gpu


def _dequant_gpu(ctx, w, out_stride=None, guard=32):
    qw, keep = device_weight(w)
    stride = out_stride or w["cols"]
    n = (w["rows"] - 1) * stride + w["cols"]
    out = torch.full((n + guard,), float("nan"), dtype=torch.float16, device="cuda")
    LinearExecutor.encode_dequant(ctx, qw, out, stride)
    torch.cuda.synchronize()
    bits = out.cpu().numpy().view(np.uint16)
    assert np.all(bits[n:] == np.float16(np.nan).view(np.uint16)), "kernel wrote past the logical output"
    rows = np.stack([bits[r * stride: r * stride + w["cols"]] for r in range(w["rows"])])
    return rows


def _wdict(storage, packed, scale_bits, zero_bits, rows, cols, stride):
    return {"storage": storage, "packed": np.asarray(packed, np.uint8), "scale_bits": np.asarray(scale_bits, np.uint16),
            "zero_bits": np.asarray(zero_bits, np.uint16), "rows": rows, "cols": cols, "row_stride": stride}


def test_w4_kernel_known_answer(ctx):
    """MetalExecutionTests.swift:28-65: 0x6E, scale 0.5, zero -0.25 -> 6.75, 2.75."""
    w = _wdict(0, [0x6E], np.array([0.5], np.float16).view(np.uint16), np.array([-0.25], np.float16).view(np.uint16),
               1, 2, 1)
    bits = _dequant_gpu(ctx, w)
    assert bits.view(np.float16).astype(np.float32).tolist() == [[6.75, 2.75]]


def test_row_aware_dequant_bit_exact(ctx):
    """MetalExecutionTests.swift:170-257 shapes (W4 [2,68], W8 [2,65]) with the guard tail."""
    rows, cols = 2, 68
    q = np.array([[(r * 7 + c) & 15 for c in range(cols)] for r in range(rows)], np.uint8)
    s = np.array([0.5, 0.25, 1.0, 2.0], np.float16).view(np.uint16)
    z = np.array([-1, 1, 3, -2], np.float16).view(np.uint16)
    w4 = _wdict(0, quant.pack_w4(q), s, z, rows, cols, 34)
    assert np.array_equal(_dequant_gpu(ctx, w4), quant.dequant_to_half(0, w4["packed"], s, z, rows, cols, 34))
    cols = 65
    p8 = np.array([(i * 13) & 255 for i in range(rows * cols)], np.uint8)
    s8 = np.array([0.125, 0.5, 0.25, 2], np.float16).view(np.uint16)
    z8 = np.array([-2, 1, 4, -3], np.float16).view(np.uint16)
    w8 = _wdict(1, p8, s8, z8, rows, cols, cols)
    assert np.array_equal(_dequant_gpu(ctx, w8), quant.dequant_to_half(1, p8, s8, z8, rows, cols, cols))


@pytest.mark.parametrize("storage", [0, 1])
def test_dequant_random_bit_exact_with_subnormals_and_padding(ctx, storage):
    rng = np.random.default_rng(11 + storage)
    rows, cols = 37, 200
    stride = ((cols + 1) // 2 + 5) if storage == 0 else cols + 3
    groups = (cols + 63) // 64
    packed = rng.integers(0, 256, size=(rows, stride), dtype=np.uint8)
    # mix of normal, subnormal and negative fp16 payloads (MetalExecutionTests.swift:115-168 class)
    s = rng.integers(0, 0x7BFF, size=(rows, groups)).astype(np.uint16)
    s[::3] = rng.integers(1, 0x03FF, size=s[::3].shape)
    z = rng.integers(0, 0xFBFF, size=(rows, groups)).astype(np.uint16)
    z[z >= 0x7C00] &= 0x83FF
    w = _wdict(storage, packed, s, z, rows, cols, stride)
    got = _dequant_gpu(ctx, w, out_stride=cols + 8)
    ref = quant.dequant_to_half(storage, packed, s, z, rows, cols, stride)
    bad = np.argwhere(got != ref)
    for r, c in bad[:8]:
        g = r * groups + c // 64
        print(f"MISMATCH r={r} c={c} got={got[r, c]:#06x} ref={ref[r, c]:#06x} "
              f"scale={s.reshape(-1)[g]:#06x} zero={z.reshape(-1)[g]:#06x}", flush=True)
    assert len(bad) == 0


def _gemm_ref(x16: torch.Tensor, w: dict) -> torch.Tensor:
    """fp64 product of the fp16 activations and the exact RNE16 dequantized weights."""
    wh = quant.dequant_to_half(w["storage"], w["packed"], w["scale_bits"], w["zero_bits"], w["rows"], w["cols"],
                               w["row_stride"]).view(np.float16).astype(np.float64)
    return torch.from_numpy(x16.double().numpy() @ wh.T)


def _check_gemm(y: torch.Tensor, ref: torch.Tensor, label: str):
    y = y.double().cpu()
    # fp16 output rounding (half an ulp) + fp32 accumulation noise
    tol = ref.abs() * 2.0 ** -10 + 1e-3 * float(ref.abs().max())
    err = (y - ref).abs()
    bad = int((err > tol).sum())
    print(f"GEMM {label}: max_err={float(err.max()):.3e} max_ref={float(ref.abs().max()):.3e} "
          f"mean_rel={float(err.sum() / ref.abs().sum()):.3e}", flush=True)
    assert bad == 0, f"{label}: {bad} elements outside tolerance"
    assert float(err.sum() / ref.abs().sum()) < 1e-3


@pytest.mark.parametrize("backend", ["auto", "dequantizedGEMM"])
@pytest.mark.parametrize("M,N,K", [(4096, 2048, 2048), (512, 2048, 1024), (300, 8192 // 4, 8192), (1, 2048, 2048),
                                   (16, 8192, 2048), (64, 2048, 8192)])
def test_w4_gemm_block_shapes(ctx, backend, M, N, K):
    d = inputs.small_m_gemm(M, N, K)
    qw, keep = device_weight(d["w"])
    x = dev(d["x"])
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx, backend=backend).execute(x, qw, y, M)
    torch.cuda.synchronize()
    _check_gemm(y, _gemm_ref(d["x"], d["w"]), f"W4 {backend} M{M} N{N} K{K}")


@pytest.mark.parametrize("storage", [0, 1])
@pytest.mark.parametrize("M,N,K", [(65, 256, 64), (130, 520, 320), (257, 1000, 448), (1000, 2056, 1024),
                                   (200, 300, 512), (129, 768, 1536), (383, 520, 4608),
                                   (4196, 8192, 512), (4300, 8256, 1024), (4196, 8192, 576)])
def test_tiled_gemm_ragged_shapes_and_both_dequant_roundings(ctx, storage, M, N, K):
    """The tiled GEMM for M > 64 with K a multiple of 64: partial row and column tiles, a
    single K block, odd block counts (the workgroup's two K halves get unequal shares), the
    M-split form of wide launches (256-row tiles: M=4196 leaves the second 128-row half of the
    last tile row wholly past M, M=4300 partly; N=8256 a 64-column last tile; K=576 has no
    scale windows), and
    per-group scale/zero pairs chosen per 64-row block so that whole waves take the
    one-rounding packed dequant (symmetric or zero offset) or the fp32 fallback (offset 2^-14
    of the scale: q*s + z no longer exact in fp32)."""
    rng = np.random.default_rng(1000 * storage + M + N + K)
    groups = K // 64
    scale = (rng.random((N, groups)) * 0.015 + 0.005).astype(np.float16)
    kind = np.repeat(rng.integers(0, 3, ((N + 63) // 64, groups)), 64, axis=0)[:N]
    sign = np.where(rng.random((N, groups)) < 0.5, -1.0, 1.0)
    qmid = 8.0 if storage == 0 else 128.0
    zero = np.where(kind == 0, -qmid * scale.astype(np.float64),
                    np.where(kind == 1, scale.astype(np.float64) * 2.0 ** -14 * sign, 0.0)).astype(np.float16)
    if storage == 0:
        packed = quant.pack_w4(rng.integers(0, 16, (N, K)).astype(np.uint8))
        stride = K // 2
    else:
        packed = rng.integers(0, 256, (N, K)).astype(np.uint8)
        stride = K
    w = _wdict(storage, packed, scale.view(np.uint16), zero.view(np.uint16), N, K, stride)
    x = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float16))
    qw, keep = device_weight(w)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx).execute(dev(x), qw, y, M)
    torch.cuda.synchronize()
    _check_gemm(y, _gemm_ref(x, w), f"tiled s{storage} M{M} N{N} K{K}")


def test_w8_padded_stride_tail_tile_and_guards(ctx):
    """LinearExecutorTests.swift:33-103: W8, M=133 N=16 K=16, packed stride 20, byte offsets 32,
    guard bytes on both sides of the output untouched."""
    m, n, k, stride, pre = 133, 16, 16, 20, 32
    xv = np.array([[((r * 3 + c * 5) % 17 - 8) / 8 for c in range(k)] for r in range(m)], np.float16)
    packed = np.full(pre + n * stride + 32, 0xEE, np.uint8)
    for r in range(n):
        for c in range(k):
            packed[pre + r * stride + c] = (r * 19 + c * 7) & 31
    sc = np.zeros(pre // 2 + n + 16, np.float16)
    ze = np.zeros(pre // 2 + n + 16, np.float16)
    sc[pre // 2: pre // 2 + n] = [(r + 1) / 64 for r in range(n)]
    ze[pre // 2: pre // 2 + n] = [(r - 3) / 16 for r in range(n)]
    xbuf = np.concatenate([np.full(pre // 2, 7, np.float16), xv.reshape(-1), np.full(16, 7, np.float16)])
    out = torch.full((pre // 2 + m * n + 16,), 0, dtype=torch.int16)
    out.fill_(0x7B7B)
    out_d = dev(out)
    P, S, Z, X = dev(torch.from_numpy(packed)), dev(torch.from_numpy(sc.view(np.int16))), \
        dev(torch.from_numpy(ze.view(np.int16))), dev(torch.from_numpy(xbuf))
    qw = QuantizedLinearWeightBuffers(1, P, S, Z, n, k, stride, packed_offset=pre, scale_offset=pre, zero_offset=pre)
    LinearExecutor(ctx).execute(X, qw, out_d, m, input_offset=pre, output_offset=pre)
    torch.cuda.synchronize()
    o = out_d.cpu()
    assert torch.all(o[: pre // 2] == 0x7B7B) and torch.all(o[pre // 2 + m * n:] == 0x7B7B)
    y = o[pre // 2: pre // 2 + m * n].numpy().view(np.float16).astype(np.float64).reshape(m, n)
    w = _wdict(1, packed[pre: pre + n * stride], sc[pre // 2: pre // 2 + n].view(np.uint16),
               ze[pre // 2: pre // 2 + n].view(np.uint16), n, k, stride)
    ref = _gemm_ref(torch.from_numpy(xv), w).numpy()
    assert np.abs(y - ref).max() <= 0.025


def test_w4_nibble_order_and_padded_rows(ctx):
    """LinearExecutorTests.swift:105-155: W4 M=3 N=16 K=16, packed stride 12 (pad 0xCC)."""
    m, n, k, stride = 3, 16, 16, 12
    xv = np.array([((i * 11) % 13 - 6) / 4 for i in range(m * k)], np.float16).reshape(m, k)
    packed = np.full((n, stride), 0xCC, np.uint8)
    for r in range(n):
        for c in range(k):
            q = (r * 5 + c * 3) & 15
            b = packed[r, c // 2]
            packed[r, c // 2] = ((b & 0xF0) | q) if c % 2 == 0 else ((b & 0x0F) | (q << 4))
    sc = np.full(n, 0.125, np.float16).view(np.uint16)
    ze = np.full(n, -0.5, np.float16).view(np.uint16)
    w = _wdict(0, packed, sc, ze, n, k, stride)
    qw, keep = device_weight(w)
    y = torch.zeros((m, n), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx, tile_rows=2).execute(dev(torch.from_numpy(xv)), qw, y, m)
    torch.cuda.synchronize()
    ref = _gemm_ref(torch.from_numpy(xv), w)
    assert float((y.double().cpu() - ref).abs().max()) <= 0.015


def test_fp16_storage_gemm(ctx):
    g = torch.Generator().manual_seed(5)
    M, N, K = 257, 300, 192
    x = torch.randn(M, K, generator=g).half()
    w16 = (torch.randn(N, K, generator=g) * 0.05).half()
    qw = QuantizedLinearWeightBuffers(2, dev(w16), dev(w16), dev(w16), N, K, K)
    y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx).execute(dev(x), qw, y, M)
    torch.cuda.synchronize()
    ref = torch.from_numpy(x.double().numpy() @ w16.double().numpy().T)
    _check_gemm(y, ref, "FP16 storage")


def test_linear_rejects_undersized_stride(ctx):
    """LinearExecutorTests.swift:157-168."""
    buf = torch.zeros(64, dtype=torch.uint8, device="cuda")
    qw = QuantizedLinearWeightBuffers(0, buf, buf, buf, 1, 16, 7)
    with pytest.raises(AnimaError) as e:
        LinearExecutor(ctx).encode(buf, qw, buf, 1)
    assert "row stride is too small" in e.value.message


def test_matvec_w8_row_boundary_and_subnormal_metadata(ctx):
    """MetalExecutionTests.swift:67-168: K=65 row boundary; fp16-subnormal scale/zero."""
    rows, cols = 2, 65
    cases = [
        (np.array([(i * 17 + 3) & 255 for i in range(rows * cols)], np.uint8),
         np.array([0.125, 0.5, 0.25, 2.0], np.float16).view(np.uint16),
         np.array([-2.0, 1.0, 4.0, -3.0], np.float16).view(np.uint16),
         np.array([(c % 11) * 0.125 - 0.5 for c in range(cols)], np.float32), 2e-3),
        (np.array([(i * 29 + 17) & 255 for i in range(rows * cols)], np.uint8),
         np.array([0x0001, 0x03FF, 0x0011, 0x0200], np.uint16),
         np.array([0x8001, 0x0002, 0x8010, 0x03FF], np.uint16),
         np.array([((c % 13) - 6) * 0.25 for c in range(cols)], np.float32), 2e-6),
    ]
    for packed, s, z, x, tol in cases:
        w = _wdict(1, packed, s, z, rows, cols, cols)
        qw, keep = device_weight(w)
        y = torch.zeros(rows, dtype=torch.float32, device="cuda")
        LinearExecutor.encode_matvec(ctx, qw, dev(torch.from_numpy(x)), y)
        torch.cuda.synchronize()
        ref = quant.dequant_w8_matrix(packed, s, z, rows, cols).astype(np.float64) @ x.astype(np.float64)
        assert np.abs(y.cpu().numpy() - ref).max() <= tol


@pytest.mark.parametrize("K", [2048, 8192])
def test_matvec_w4_precision(ctx, K):
    """LinearExecutorTests.swift:308-415 generator: direct matvec maxAbs < 1e-3 vs fp64."""
    n, groups, stride = 16, K // 64, K // 2
    state = (0xA51A0000 + K) & 0xFFFFFFFF
    norm = 1 / np.sqrt(K)
    xin = np.zeros(K, np.float32)
    for c in range(K):
        state = (state * 1664525 + 1013904223) & 0xFFFFFFFF
        xin[c] = ((int((state >> 16) % 2001) - 1000) / 1000) * norm
    packed = np.zeros((n, stride), np.uint8)
    sc = np.zeros((n, groups), np.float16)
    ze = np.zeros((n, groups), np.float16)
    for r in range(n):
        for g in range(groups):
            sc[r, g] = (1 + (r + g) % 3) / 64
            ze[r, g] = ((r + g) % 5 - 2) / 16
        for c in range(K):
            q = (r * 11 + c * 7 + c // 64 * 3) & 15
            packed[r, c // 2] |= q if c % 2 == 0 else q << 4
    w = _wdict(0, packed, sc.view(np.uint16), ze.view(np.uint16), n, K, stride)
    qw, keep = device_weight(w)
    y = torch.zeros(n, dtype=torch.float32, device="cuda")
    LinearExecutor.encode_matvec(ctx, qw, dev(torch.from_numpy(xin)), y)
    torch.cuda.synchronize()
    ref = quant.dequant_w4_matrix(packed, sc.view(np.uint16), ze.view(np.uint16), n, K).astype(np.float64) @ xin.astype(np.float64)
    got = y.cpu().numpy().astype(np.float64)
    assert np.abs(got - ref).max() < 1e-3
    cos = got @ ref / (np.linalg.norm(got) * np.linalg.norm(ref))
    assert cos > 0.999999


def _affine_weight(storage: int, N: int, K: int, seed: int, pad: int = 0) -> dict:
    """Random affine weight (codes, fp16 scale/zero) in the pack layout, optional row padding."""
    rng = np.random.default_rng(seed)
    groups = (K + 63) // 64
    s = (rng.random((N, groups)) * 0.02 + 0.002).astype(np.float16).view(np.uint16)
    z = ((rng.random((N, groups)) - 0.5) * 0.2).astype(np.float16).view(np.uint16)
    if storage == 0:
        q = rng.integers(0, 16, (N, K)).astype(np.uint8)
        stride = (K + 1) // 2 + pad
        packed = quant.pack_w4(q, stride, pad_value=0xA5)
    elif storage == 1:
        stride = K + pad
        packed = np.full((N, stride), 0x5A, np.uint8)
        packed[:, :K] = rng.integers(0, 256, (N, K)).astype(np.uint8)
    else:
        stride = K + pad // 2
        w16 = np.full((N, stride), np.float16(7.0), np.float16)
        w16[:, :K] = (rng.standard_normal((N, K)) * 0.05).astype(np.float16)
        packed = w16.view(np.uint8)
    return _wdict(storage, packed, s, z, N, K, stride)


@pytest.mark.parametrize("storage", [0, 1, 2])
@pytest.mark.parametrize("M,N,K,pad", [(1, 2048, 2048, 0), (5, 1000, 384, 16), (16, 8192, 2048, 0),
                                       (17, 130, 1280, 32), (33, 2048, 1024, 0), (64, 2048, 8192, 0),
                                       (64, 4000, 2048, 16), (64, 8192, 2048, 0), (40, 8200, 1024, 16),
                                       (3, 1004, 1024, 0), (1, 2052, 8192, 0), (16, 2048, 8192, 16)])
def test_small_m_weight_stream_gemm(ctx, storage, M, N, K, pad):
    """M <= 64 with K a multiple of 128 takes the weight-streaming kernel: every storage, ragged N,
    padded row strides; the output's neighbours stay untouched."""
    w = _affine_weight(storage, N, K, seed=M * 1000 + N + K + storage, pad=pad)
    qw, keep = device_weight(w)
    g = torch.Generator().manual_seed(M + N)
    x = torch.randn(M, K, generator=g).half()
    guard = 8
    out = torch.full((M * N + 2 * guard,), float("nan"), dtype=torch.float16, device="cuda")
    print(f"SMALLM storage={storage} M={M} N={N} K={K} pad={pad}", flush=True)
    LinearExecutor(ctx).execute(dev(x), qw, out, M, output_offset=2 * guard)
    torch.cuda.synchronize()
    o = out.cpu()
    assert torch.isnan(o[:guard]).all() and torch.isnan(o[guard + M * N:]).all()
    _check_gemm(o[guard: guard + M * N].reshape(M, N), _gemm_ref(x, w), f"small-M s{storage} M{M} N{N} K{K}")


def test_small_m_unaligned_output_and_repeat(ctx):
    """An output offset of one half (not 8-byte aligned) takes the scalar store path; two calls in a
    row give identical bits (fixed-order reduction)."""
    M, N, K = 3, 260, 512
    w = _affine_weight(0, N, K, seed=11)
    qw, keep = device_weight(w)
    x = torch.randn(M, K, generator=torch.Generator().manual_seed(2)).half()
    out = torch.zeros(M * N + 1, dtype=torch.float16, device="cuda")
    ex = LinearExecutor(ctx)
    ex.execute(dev(x), qw, out, M, output_offset=2)
    first = out.clone()
    ex.execute(dev(x), qw, out, M, output_offset=2)
    torch.cuda.synchronize()
    assert torch.equal(first.view(torch.int16), out.view(torch.int16))
    assert float(out[0]) == 0.0
    _check_gemm(out[1:].reshape(M, N), _gemm_ref(x, w), "small-M unaligned")


def _one_hot_params(rng, N: int, groups: int) -> tuple:
    """fp16 scale/zero bit patterns per (row, group): ordinary values, subnormals, zeros and
    pairs whose exponents differ by up to 20 (q*s + z no longer exact in fp32)."""
    kinds = rng.integers(0, 6, (N, groups))
    s = np.zeros((N, groups), np.float16)
    z = np.zeros((N, groups), np.float16)
    base = (rng.random((N, groups)) * 0.02 + 0.001)
    gap = 2.0 ** rng.integers(9, 21, (N, groups))
    sign = np.where(rng.random((N, groups)) < 0.5, -1.0, 1.0)
    s[kinds == 0] = base[kinds == 0]
    z[kinds == 0] = (-8 * base * sign)[kinds == 0]
    s[kinds == 1] = (base * 64)[kinds == 1]                         # |z| far below s
    z[kinds == 1] = (base * 64 / gap * sign)[kinds == 1]
    s[kinds == 2] = (base / 64)[kinds == 2]                         # |z| far above s
    z[kinds == 2] = (base / 64 * gap * sign)[kinds == 2]
    sb, zb = s.view(np.uint16), z.view(np.uint16)
    sub = kinds == 3                                                # subnormal scale / zero
    sb[sub] = rng.integers(1, 0x400, int(sub.sum())).astype(np.uint16)
    zb[sub] = (rng.integers(1, 0x400, int(sub.sum())) | (rng.integers(0, 2, int(sub.sum())) << 15)).astype(np.uint16)
    s[kinds == 4] = base[kinds == 4]                                # zero offset
    z[kinds == 4] = 0
    s[kinds == 5] = 0                                               # zero scale
    z[kinds == 5] = (base * sign)[kinds == 5]
    return sb.copy(), zb.copy()


@pytest.mark.parametrize("storage", [0, 1])
@pytest.mark.parametrize("M", [5, 16, 64, 128])
def test_gemm_dequant_bit_exact_via_one_hot(ctx, storage, M):
    """Row m of X is one-hot at column k_m, so y[m, n] = deq(W)[n, k_m] exactly (a single
    1*w product in fp32): the GEMM's in-register dequantization must reproduce the oracle's
    RNE16(fl32(q*s + z)) bit for bit, including the fallback taken when q*s + z is not exact in
    fp32.  M=5 and 16 run the weight-streaming kernel with per-lane scale/zero loads (and X rows
    past M read as zeros through the bounded loads), M=64 that kernel with scale/zero staged in
    LDS, M=128 the tiled GEMM."""
    rng = np.random.default_rng(40 + storage + M)
    N, K = 384, 1024
    groups = K // 64
    sb, zb = _one_hot_params(rng, N, groups)
    if storage == 0:
        packed = quant.pack_w4(rng.integers(0, 16, (N, K)).astype(np.uint8))
        stride = K // 2
    else:
        packed = rng.integers(0, 256, (N, K)).astype(np.uint8)
        stride = K
    w = _wdict(storage, packed, sb, zb, N, K, stride)
    ks = rng.choice(K, M, replace=False)
    x = np.zeros((M, K), np.float16)
    x[np.arange(M), ks] = 1.0
    qw, keep = device_weight(w)
    y = torch.zeros((M, N), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx).execute(dev(torch.from_numpy(x)), qw, y, M)
    torch.cuda.synchronize()
    got = y.cpu().numpy()
    want = quant.dequant_to_half(storage, packed, sb, zb, N, K, stride).view(np.float16)[:, ks].T
    finite = np.isfinite(want)
    mism = np.argwhere(finite & (got != want))
    for m, n in mism[:8]:
        g = n * groups + ks[m] // 64
        print(f"MISMATCH m={m} n={n} k={ks[m]} got={got[m, n]!r} want={want[m, n]!r} "
              f"scale={sb.reshape(-1)[g]:#06x} zero={zb.reshape(-1)[g]:#06x}", flush=True)
    assert len(mism) == 0
    assert finite.mean() > 0.99


@pytest.mark.parametrize("storage,M,N,K", [(0, 256, 2048, 2048), (1, 130, 520, 320), (0, 257, 1000, 448),
                                           (1, 129, 770, 128), (0, 32, 512, 512), (2, 96, 256, 256),
                                           (0, 100, 300, 200), (0, 4096, 8192, 256)])
def test_linear_epilogues_equal_two_step(ctx, storage, M, N, K):
    """anima_linear_encode_epilogue: the tiled GEMM's fused GELU / gate-add output stage (M > 64,
    W4/W8, K a multiple of 64; N % 4 != 0 takes its element-wise stores) and the two-kernel
    fallback (small M, fp16 storage, K not a multiple of 64) give the same bits as the linear
    followed by dit_gelu_half_inplace / gate_add_half_f32 / add_half_into_float."""
    from animaxs_amd import BlockOps
    w = _affine_weight(storage, N, K, seed=7 * M + N + K + storage)
    qw, keep = device_weight(w)
    g = torch.Generator().manual_seed(M * 3 + N)
    x = dev(torch.randn(M, K, generator=g).half())
    lin, ops = LinearExecutor(ctx), BlockOps(ctx)
    print(f"EPILOGUE storage={storage} M={M} N={N} K={K}", flush=True)

    y_ref = torch.empty(M * N, dtype=torch.float16, device="cuda")
    lin.encode(x, qw, y_ref, M)
    ops.gelu_half_inplace(y_ref, M * N)
    y = torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda")
    lin.encode_epilogue(x, qw, y, M, "gelu")

    res0 = torch.randn(M * N, generator=g)
    gate = dev(torch.randn(N, generator=g))
    branch = torch.empty(M * N, dtype=torch.float16, device="cuda")
    r_ref = dev(res0.clone())
    lin.encode(x, qw, branch, M)
    ops.gate_add_half_f32(r_ref, branch, gate, N, M * N)
    r = dev(res0.clone())
    lin.encode_epilogue(x, qw, torch.empty_like(branch), M, "gate_add", residual=r, gate=gate)
    # residual add (add_half_into_float); M=256 N=2048 K=2048 runs split over K in both forms
    r2_ref = dev(res0.clone())
    ops.add_half_into_float(r2_ref, branch, M * N)
    r2 = dev(res0.clone())
    lin.encode_epilogue(x, qw, torch.empty_like(branch), M, "residual_add", residual=r2)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), y_ref.view(torch.int16))
    assert torch.equal(r.view(torch.int32), r_ref.view(torch.int32))
    assert torch.equal(r2.view(torch.int32), r2_ref.view(torch.int32))
    assert not torch.equal(r.cpu(), res0)


def test_linear_epilogue_rejects_bad_arguments(ctx):
    w = _affine_weight(0, 256, 256, seed=5)
    qw, keep = device_weight(w)
    x = torch.zeros(128, 256, dtype=torch.float16, device="cuda")
    y = torch.empty(128, 256, dtype=torch.float16, device="cuda")
    lin = LinearExecutor(ctx)
    with pytest.raises(AnimaError) as e:
        lin.encode_epilogue(x, qw, y, 128, "gate_add", residual=torch.zeros(128 * 256 - 1, device="cuda"),
                            gate=torch.zeros(256, device="cuda"))
    assert "out of bounds" in e.value.message
    with pytest.raises(AnimaError):
        lin.encode_epilogue(x, qw, y, 128, "gate_add", residual=torch.zeros(128 * 256, device="cuda"), gate=None)


@pytest.mark.parametrize("storage", [0, 1, 2])
@pytest.mark.parametrize("N,K,pad", [(6144, 256, 0), (256, 2048, 0), (33, 96, 16), (7, 4096, 0), (5, 130, 0)])
def test_matvec_vectorised_every_storage(ctx, storage, N, K, pad):
    """The fp32 matvec's 16-byte chunk form (8 to 64 lanes per row, several rows per wave, padded
    strides) and its scalar form (K=130: not a multiple of the chunk) against an fp64 product of
    the fp32 dequantised weights."""
    w = _affine_weight(storage, N, K, seed=N + K + storage, pad=pad)
    qw, keep = device_weight(w)
    x = torch.randn(K, generator=torch.Generator().manual_seed(K)).float()
    y = torch.full((N + 4,), float("nan"), device="cuda")
    print(f"MATVEC storage={storage} N={N} K={K} pad={pad}", flush=True)
    LinearExecutor.encode_matvec(ctx, qw, dev(x), y)
    torch.cuda.synchronize()
    wf = quant.dequant_matrix_f32(storage, w["packed"], w["scale_bits"], w["zero_bits"], N, K,
                                  w["row_stride"]).astype(np.float64)
    xd = x.double().numpy()
    ref = wf @ xd
    got = y.cpu().numpy().astype(np.float64)
    assert np.isnan(got[N:]).all()
    bound = 1e-5 * (np.abs(wf) @ np.abs(xd)) + 1e-6
    assert (np.abs(got[:N] - ref) <= bound).all(), float(np.abs(got[:N] - ref).max())


@pytest.mark.parametrize("storage,M,Ns,K", [(0, 4096 + 40, (2048, 1024, 1024), 1024), (1, 130, (520, 256), 320),
                                            (0, 512, (2048, 2048), 1024), (0, 257, (1000, 300, 1030), 448),
                                            (0, 48, (512, 256), 512), (1, 200, (256, 256), 200),
                                            (0, 4096, (8192, 2048), 256)])
def test_linear_group_equals_separate_encodes(ctx, storage, M, Ns, K):
    """anima_linear_encode_group: one ping-pong launch over 2-3 weights of different N (tile ->
    problem mapping, ragged M and N) gives the bits of separate encodes; groups the tiled GEMM
    does not take (small M, K not a multiple of 64) and groups with a member that its own
    encode runs in the M-split form (M=4096 N=8192) fall back to separate encodes."""
    ws = [_affine_weight(storage, N, K, seed=N + K + i) for i, N in enumerate(Ns)]
    qws, keeps = zip(*[device_weight(w) for w in ws])
    x = dev(torch.randn(M, K, generator=torch.Generator().manual_seed(M + K)).half())
    lin = LinearExecutor(ctx)
    refs = []
    for qw, N in zip(qws, Ns):
        y = torch.empty(M * N, dtype=torch.float16, device="cuda")
        lin.encode(x, qw, y, M)
        refs.append(y)
    outs = [torch.full((M * N,), float("nan"), dtype=torch.float16, device="cuda") for N in Ns]
    print(f"GROUP storage={storage} M={M} Ns={Ns} K={K}", flush=True)
    lin.encode_group(x, list(qws), outs, M)
    torch.cuda.synchronize()
    for r, o in zip(refs, outs):
        assert torch.equal(r.view(torch.int16), o.view(torch.int16))


@pytest.mark.parametrize("storage,M,N,K,hd", [(0, 300, 384, 512, 128), (1, 1000, 2048, 1024, 128),
                                              (0, 4096 + 40, 2048, 2048, 128), (0, 48, 384, 512, 128),
                                              (0, 300, 384, 512, 64), (2, 100, 256, 256, 128),
                                              (0, 4096 + 40, 8192, 256, 128)])
def test_linear_head_rmsnorm_matches_encode_then_norm(ctx, storage, M, N, K, hd):
    """anima_linear_encode_head_rmsnorm: the tiled GEMM's per-head RMSNorm output stage (M > 64,
    W4/W8, head_dim 128; ragged M, N = 384 leaves a 256-column tile half used; N = 8192 runs the
    M-split form's 256-row tiles) and the in-place
    second pass (small M, head_dim 64, fp16 storage) against plain encode followed by the oracle's
    per-head RMSNorm (rmsnorm_heads_half, AnimaKernels.metal:660-689) of those fp16 outputs: within
    one fp16 ulp (the sum of squares is reduced in another order)."""
    from oracle import norms
    w = _affine_weight(storage, N, K, seed=11 * M + N + K + storage + hd)
    qw, keep = device_weight(w)
    g = torch.Generator().manual_seed(M + N + hd)
    x = dev(torch.randn(M, K, generator=g).half())
    nw = (torch.rand(hd, generator=g) * 0.4 + 0.8).half()
    lin = LinearExecutor(ctx)
    print(f"HEAD_RMSNORM storage={storage} M={M} N={N} K={K} hd={hd}", flush=True)
    y0 = torch.empty(M, N, dtype=torch.float16, device="cuda")
    lin.encode(x, qw, y0, M)
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    lin.encode_head_rmsnorm(x, qw, y, M, dev(nw), head_dim=hd, eps=1e-6)
    torch.cuda.synchronize()
    ref = norms.rms_norm(y0.cpu().float().reshape(M, N // hd, hd), nw, 1e-6).reshape(M, N)
    got = y.cpu().float()
    assert torch.isfinite(got).all()
    err = (got - ref).abs()
    ulp = torch.clamp(ref.abs(), min=2.0 ** -14) * 2.0 ** -10
    print(f"HEAD_RMSNORM max_err={float(err.max()):.3e} max_err/ulp={float((err / ulp).max()):.2f}", flush=True)
    assert bool((err <= ulp * 1.01).all())


def test_split_k_merge_with_odd_element_count(ctx):
    """M*N odd (101 x 1001, K = 2048: four tiles, so the GEMM splits K in two): the split-K
    merge must take its element-wise path, whose reads of split s >= 1 are then not
    16-byte aligned."""
    M, N, K = 101, 1001, 2048
    d = inputs.small_m_gemm(M, N, K, seed=77)
    qw, keep = device_weight(d["w"])
    y = torch.full((M, N), float("nan"), dtype=torch.float16, device="cuda")
    LinearExecutor(ctx).execute(dev(d["x"]), qw, y, M)
    torch.cuda.synchronize()
    _check_gemm(y, _gemm_ref(d["x"], d["w"]), f"split-K odd M{M} N{N} K{K}")
