"""CPU: W4/W8 dequantization oracle and the library's C decoders against the reference's
known answers (AnimaXSTests/QuantDecoderTests.swift, MetalExecutionTests.swift) and
against independent fp64 arithmetic.  No GPU needed."""

from __future__ import annotations

import numpy as np
import pytest

from oracle import quant as Q


def f16bits(values) -> np.ndarray:
    return np.asarray(values, dtype=np.float16).view(np.uint16)


@pytest.fixture(scope="module")
def lib_decoders():
    import animaxs_amd
    return animaxs_amd.QuantDecoders


def decoders(lib):
    """The oracle and the library's CPU decoders share every known-answer test."""
    return {"oracle": Q, "lib": lib}


# --- QuantDecoderTests.swift known answers, run on both decoders ---------------------

def _w4(impl, *a, **k):
    return impl.dequant_w4(*a, **k)


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w4_even_index_low_nibble(who, lib_decoders):
    # QuantDecoderTests.swift:23-28: 0x6E -> low nibble 14 (even K), high 6 (odd K)
    impl = decoders(lib_decoders)[who]
    s = 0.0004537
    out = impl.dequant_w4(bytes([0x6E]), f16bits([s]), f16bits([0.0]), 2)
    s16 = float(np.float16(s))
    assert out[0] == pytest.approx(14 * s16, abs=1e-6)
    assert out[1] == pytest.approx(6 * s16, abs=1e-6)
    assert abs(out[0] - 14 * s) < 1e-4 and abs(out[1] - 6 * s) < 1e-4


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w4_equation(who, lib_decoders):
    # QuantDecoderTests.swift:30-34: q=10, scale 0.5, zero -0.25 -> 4.75 (exact)
    impl = decoders(lib_decoders)[who]
    out = impl.dequant_w4(bytes([0x0A]), f16bits([0.5]), f16bits([-0.25]), 1)
    assert out[0] == 4.75


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w4_group_indexing_along_k(who, lib_decoders):
    # QuantDecoderTests.swift:36-44: index 64 switches to scale[1]
    impl = decoders(lib_decoders)[who]
    full = bytearray(64)
    full[0] = 0x07
    full[32] = 0x03
    out = impl.dequant_w4(bytes(full), f16bits([1.0, 2.0]), f16bits([0.0, 0.0]), 65)
    assert out[0] == 7.0 and out[64] == 6.0
    assert np.all(out[1:64] == 0.0)


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w4_matrix_groups_reset_each_row(who, lib_decoders):
    # QuantDecoderTests.swift:46-60: two rows of 68 -> groups reset per row
    impl = decoders(lib_decoders)[who]
    out = impl.dequant_w4_matrix(bytes([0x11] * (2 * 34)), f16bits([1, 10, 100, 1000]), f16bits([0, 0, 0, 0]), 2, 68)
    out = np.asarray(out).reshape(-1)
    assert out[0] == 1.0 and out[64] == 10.0 and out[68] == 100.0 and out[68 + 64] == 1000.0


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w8_equation_and_groups(who, lib_decoders):
    # QuantDecoderTests.swift:64-79
    impl = decoders(lib_decoders)[who]
    out = impl.dequant_w8(bytes([10, 20]), f16bits([0.5, 0.25]), f16bits([-1.0, 2.0]), 2)
    assert out[0] == 4.0 and out[1] == 9.0
    data = bytearray(65)
    data[0], data[64] = 5, 9
    out = impl.dequant_w8(bytes(data), f16bits([1.0, 10.0]), f16bits([0.0, 0.0]), 65)
    assert out[0] == 5.0 and out[64] == 90.0


@pytest.mark.parametrize("who", ["oracle", "lib"])
def test_w8_matrix_groups_reset_each_row(who, lib_decoders):
    # QuantDecoderTests.swift:81-93
    impl = decoders(lib_decoders)[who]
    out = impl.dequant_w8_matrix(bytes([1] * 130), f16bits([1, 10, 100, 1000]), f16bits([0, 0, 0, 0]), 2, 65)
    out = np.asarray(out).reshape(-1)
    assert out[0] == 1.0 and out[64] == 10.0 and out[65] == 100.0 and out[65 + 64] == 1000.0


def test_fp16_read(lib_decoders):
    # QuantDecoderTests.swift:97-103
    bits = f16bits([1.5, -2.25, 0.0, 65504.0])
    for out in (Q.fp16_bits_to_f32(bits), lib_decoders.fp16_to_float32(bits, 4)):
        assert list(out) == [1.5, -2.25, 0.0, 65504.0]


def test_fp16_read_all_patterns(lib_decoders):
    """Every binary16 bit pattern (subnormals, infinities, NaNs) decodes like numpy."""
    bits = np.arange(65536, dtype=np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    for got in (Q.fp16_bits_to_f32(bits), lib_decoders.fp16_to_float32(bits, 65536)):
        assert np.array_equal(got.view(np.uint32)[~np.isnan(want)], want.view(np.uint32)[~np.isnan(want)])
        assert np.all(np.isnan(got[np.isnan(want)]))


# --- MetalExecutionTests.swift known answers (the to-half kernel's values) ------------

def test_w4_to_half_kernel_values():
    # MetalExecutionTests.swift:28-65: 0x6E, scale 0.5, zero -0.25 -> 6.75, 2.75
    h = Q.dequant_to_half(Q.STORAGE_W4, np.array([[0x6E]], np.uint8), f16bits([0.5]), f16bits([-0.25]), 1, 2)
    assert list(h.view(np.float16).astype(np.float32).ravel()) == [6.75, 2.75]


def _row_aware_w4():
    rows, cols, stride = 2, 68, 34
    q = np.array([[(r * 7 + c) & 15 for c in range(cols)] for r in range(rows)], np.uint8)
    return q, Q.pack_w4(q, stride), f16bits([0.5, 0.25, 1.0, 2.0]), f16bits([-1, 1, 3, -2])


def test_w4_row_aware_bit_patterns():
    # MetalExecutionTests.swift:170-196: expected = Float16(q*s + z) per element
    q, packed, s, z = _row_aware_w4()
    got = Q.dequant_to_half(Q.STORAGE_W4, packed, s, z, 2, 68)
    sf, zf = s.view(np.float16).astype(np.float64), z.view(np.float16).astype(np.float64)
    for r in range(2):
        for c in range(68):
            g = r * 2 + c // 64
            assert got[r, c] == np.float16(q[r, c] * sf[g] + zf[g]).view(np.uint16)


def test_w8_row_aware_bit_patterns():
    # MetalExecutionTests.swift:198-216
    rows, cols = 2, 65
    packed = np.array([(i * 13) & 255 for i in range(rows * cols)], np.uint8).reshape(rows, cols)
    s, z = f16bits([0.125, 0.5, 0.25, 2]), f16bits([-2, 1, 4, -3])
    got = Q.dequant_to_half(Q.STORAGE_W8, packed, s, z, rows, cols)
    sf, zf = s.view(np.float16).astype(np.float64), z.view(np.float16).astype(np.float64)
    for r in range(rows):
        for c in range(cols):
            g = r * 2 + c // 64
            assert got[r, c] == np.float16(packed[r, c] * sf[g] + zf[g]).view(np.uint16)


def _w8_matvec_expected(packed, sbits, zbits, x, rows, cols):
    """fp64 restatement of the expectation loop of MetalExecutionTests.swift:94-103."""
    s = np.asarray(sbits, np.uint16).view(np.float16).astype(np.float64)
    z = np.asarray(zbits, np.uint16).view(np.float16).astype(np.float64)
    out = np.zeros(rows)
    for r in range(rows):
        for c in range(cols):
            g = r * 2 + c // 64
            out[r] += x[c] * (float(packed[r * cols + c]) * s[g] + z[g])
    return out


@pytest.mark.parametrize("case", ["row_boundary", "subnormal"])
def test_w8_matvec_expectation(case):
    # MetalExecutionTests.swift:67-168: the oracle's decode times x matches the fp64
    # expectation within the reference's tolerances (2e-3, and 2e-6 for subnormals)
    rows, cols = 2, 65
    if case == "row_boundary":
        packed = np.array([(i * 17 + 3) & 255 for i in range(rows * cols)], np.uint8)
        sbits, zbits = f16bits([0.125, 0.5, 0.25, 2.0]), f16bits([-2.0, 1.0, 4.0, -3.0])
        x = np.array([(c % 11) * 0.125 - 0.5 for c in range(cols)], np.float32)
        tol = 2e-3
    else:
        packed = np.array([(i * 29 + 17) & 255 for i in range(rows * cols)], np.uint8)
        sbits = np.array([0x0001, 0x03FF, 0x0011, 0x0200], np.uint16)
        zbits = np.array([0x8001, 0x0002, 0x8010, 0x03FF], np.uint16)
        x = np.array([((c % 13) - 6) * 0.25 for c in range(cols)], np.float32)
        tol = 2e-6
    w = Q.dequant_w8_matrix(packed.reshape(rows, cols), sbits, zbits, rows, cols)
    # subnormal scales must not be flushed: the decoded weights are not all zero-offset
    assert np.any(w != 0)
    got = w.astype(np.float32) @ x
    want = _w8_matvec_expected(packed, sbits, zbits, x, rows, cols)
    assert np.max(np.abs(got - want)) <= tol


# --- exhaustive / invariant checks ----------------------------------------------------

def test_w4_value_exact_for_every_q_and_random_params():
    """fl32(q*s + z) equals the fp64 value rounded once to fp32 for every nibble: q*s is
    exact in fp32, so contraction to an FMA cannot change a bit."""
    rng = np.random.default_rng(7)
    sb = rng.integers(0, 0x7C00, 4096).astype(np.uint16)     # finite non-negative scales
    zb = rng.integers(0, 0x10000, 4096).astype(np.uint16)
    zb = zb[(zb & 0x7C00) != 0x7C00][:2048]
    sb = sb[: len(zb)]
    s = sb.view(np.float16).astype(np.float64)
    z = zb.view(np.float16).astype(np.float64)
    for q in range(16):
        exact = (q * s + z).astype(np.float32)
        byte = np.full(1, q | (q << 4), np.uint8)
        for i in range(0, len(sb), 256):
            got = np.array([Q.dequant_w4(byte, sb[j:j + 1], zb[j:j + 1], 1)[0] for j in range(i, i + 4)])
            assert np.array_equal(got.view(np.uint32), exact[i:i + 4].view(np.uint32))
        # vectorised over all parameter pairs with the matrix decoder
        packed = np.full((len(sb), 1), q | (q << 4), np.uint8)
        got = Q.dequant_w4_matrix(packed, sb, zb, len(sb), 2)
        assert np.array_equal(got[:, 0].view(np.uint32), exact.view(np.uint32))


def test_w8_value_exact_for_every_q():
    rng = np.random.default_rng(8)
    sb = rng.integers(0, 0x7C00, 512).astype(np.uint16)
    zb = rng.integers(0, 0x7C00, 512).astype(np.uint16) | (rng.integers(0, 2, 512).astype(np.uint16) << 15)
    s = sb.view(np.float16).astype(np.float64)
    z = zb.view(np.float16).astype(np.float64)
    q = np.arange(256, dtype=np.uint8)
    packed = np.tile(q, (512, 1))
    # one group per row: cols = 64 uses only group 0 -> decode 4 rows of 64 per param
    got = Q.dequant_w8_matrix(packed[:, :64], sb, zb, 512, 64)
    exact = (q[None, :64].astype(np.float64) * s[:, None] + z[:, None]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), exact.view(np.uint32))
    got = Q.dequant_w8_matrix(packed[:, 192:], sb, zb, 512, 64)
    exact = (q[None, 192:].astype(np.float64) * s[:, None] + z[:, None]).astype(np.float32)
    assert np.array_equal(got.view(np.uint32), exact.view(np.uint32))


def test_symmetric_w4_reproduces_centered_codes():
    """Symmetric data (zero = -8*scale) decodes to exactly (q - 8) * scale."""
    rng = np.random.default_rng(9)
    rows, cols = 16, 200
    q = rng.integers(0, 16, (rows, cols)).astype(np.uint8)
    groups = (cols + 63) // 64
    s = (rng.random((rows, groups)) * 0.01 + 1e-3).astype(np.float16)
    z = (-8.0 * s.astype(np.float32)).astype(np.float16)
    assert np.all(z.astype(np.float32) == -8.0 * s.astype(np.float32))  # exact in fp16
    got = Q.dequant_w4_matrix(Q.pack_w4(q), s.view(np.uint16), z.view(np.uint16), rows, cols)
    gidx = np.arange(cols) // 64
    want = (q.astype(np.float64) - 8.0) * s.astype(np.float64)[:, gidx]
    assert np.array_equal(got, want.astype(np.float32))


def test_padded_row_stride_and_odd_cols():
    rng = np.random.default_rng(10)
    rows, cols = 5, 131
    q = rng.integers(0, 16, (rows, cols)).astype(np.uint8)
    groups = 3
    s = rng.random((rows, groups)).astype(np.float16).view(np.uint16)
    z = (rng.random((rows, groups)) - 0.5).astype(np.float16).view(np.uint16)
    tight = Q.dequant_w4_matrix(Q.pack_w4(q), s, z, rows, cols)
    padded = Q.dequant_w4_matrix(Q.pack_w4(q, 80, pad_value=0xFF), s, z, rows, cols, row_stride=80)
    assert np.array_equal(tight, padded)
    # the flat decoder on one row equals the matrix decoder's row
    for r in range(rows):
        flat = Q.dequant_w4(Q.pack_w4(q[r:r + 1]).ravel(), s.reshape(rows, groups)[r], z.reshape(rows, groups)[r], cols)
        assert np.array_equal(flat, tight[r])


def test_lib_decoders_match_oracle_random(lib_decoders):
    rng = np.random.default_rng(11)
    rows, cols = 7, 300
    groups = (cols + 63) // 64
    q = rng.integers(0, 16, (rows, cols)).astype(np.uint8)
    s = rng.integers(0, 0x7C00, rows * groups).astype(np.uint16)
    z = rng.integers(0, 0x7C00, rows * groups).astype(np.uint16) | 0x8000
    packed = Q.pack_w4(q)
    a = Q.dequant_w4_matrix(packed, s, z, rows, cols)
    b = lib_decoders.dequant_w4_matrix(packed.ravel(), s, z, rows, cols)
    assert np.array_equal(a.view(np.uint32), np.asarray(b).view(np.uint32))
    p8 = rng.integers(0, 256, (rows, cols)).astype(np.uint8)
    a = Q.dequant_w8_matrix(p8, s, z, rows, cols)
    b = lib_decoders.dequant_w8_matrix(p8.ravel(), s, z, rows, cols)
    assert np.array_equal(a.view(np.uint32), np.asarray(b).view(np.uint32))


# --- LinearExecutorTests.swift cases restated on the oracle --------------------------

def _linear_oracle(x16, storage, packed, sbits, zbits, rows, cols, stride):
    w = Q.dequant_to_half(storage, packed, sbits, zbits, rows, cols, stride).view(np.float16).astype(np.float64)
    return x16.astype(np.float64) @ w.T


def test_w8_padded_stride_linear_case():
    # LinearExecutorTests.swift:33-100: M=133, N=16, K=16, packed stride 20 (pad 0xEE)
    m, n, k, stride = 133, 16, 16, 20
    x = np.array([[np.float16((((r * 3 + c * 5) % 17) - 8) / 8) for c in range(k)] for r in range(m)])
    packed = np.full((n, stride), 0xEE, np.uint8)
    deq = np.zeros((n, k))
    s = np.array([np.float16((r + 1) / 64) for r in range(n)])
    z = np.array([np.float16((r - 3) / 16) for r in range(n)])
    for r in range(n):
        for c in range(k):
            q = (r * 19 + c * 7) & 31
            packed[r, c] = q
            deq[r, c] = float(np.float16(q * float(s[r]) + float(z[r])))
    want = x.astype(np.float64) @ deq.T
    got = _linear_oracle(x, Q.STORAGE_W8, packed, s.view(np.uint16), z.view(np.uint16), n, k, stride)
    assert np.max(np.abs(got - want)) == 0.0


def test_w4_nibble_order_padded_rows_linear_case():
    # LinearExecutorTests.swift:102-148: M=3, N=16, K=16, packed stride 12 (pad 0xCC)
    m, n, k, stride = 3, 16, 16, 12
    x = np.array([np.float16(((i * 11) % 13 - 6) / 4) for i in range(m * k)]).reshape(m, k)
    packed = np.full((n, stride), 0xCC, np.uint8)
    deq = np.zeros((n, k))
    for r in range(n):
        for c in range(k):
            q = (r * 5 + c * 3) & 15
            b = packed[r, c // 2]
            packed[r, c // 2] = (b & 0xF0) | q if c % 2 == 0 else (b & 0x0F) | (q << 4)
            deq[r, c] = float(np.float16(q * 0.125 - 0.5))
    s = np.full(n, np.float16(0.125)).view(np.uint16)
    z = np.full(n, np.float16(-0.5)).view(np.uint16)
    want = x.astype(np.float64) @ deq.T
    got = _linear_oracle(x, Q.STORAGE_W4, packed, s, z, n, k, stride)
    assert np.max(np.abs(got - want)) == 0.0


# --- the exactness condition the GEMM kernels use to round once -----------------------

def _unit_exp(bits):
    e = (bits.astype(np.int32) >> 10) & 31
    return np.maximum(e, 1)


@pytest.mark.parametrize("qbits", [4, 8])
def test_one_rounding_condition_implies_fp32_exact(qbits):
    """The GEMMs round q*s + z once (straight to fp16) when the fp16 unit exponents of s and z
    differ by d with -12 <= d <= 12 - qbits (or s or z is zero).  Under that condition q*s + z
    must be exactly representable in fp32 for every code q, so one rounding equals the
    reference's fp32-then-fp16 rounding.  Checked on 400k random finite (s, z) pairs plus the
    boundary exponents."""
    rng = np.random.default_rng(qbits)
    n = 400_000
    sb = rng.integers(0, 0x10000, n).astype(np.uint16)
    zb = rng.integers(0, 0x10000, n).astype(np.uint16)
    # add pairs exactly at and just outside the boundary
    es = rng.integers(1, 31, 20000)
    for d in (-13, -12, 12 - qbits, 13 - qbits):
        ez = es - d
        ok = (ez >= 1) & (ez <= 30)
        m1 = rng.integers(0, 1024, int(ok.sum()))
        m2 = rng.integers(0, 1024, int(ok.sum()))
        sb = np.concatenate([sb, ((es[ok] << 10) | m1).astype(np.uint16)])
        zb = np.concatenate([zb, ((ez[ok] << 10) | m2 | (rng.integers(0, 2, int(ok.sum())) << 15)).astype(np.uint16)])
    finite = ((sb & 0x7C00) != 0x7C00) & ((zb & 0x7C00) != 0x7C00)
    sb, zb = sb[finite], zb[finite]
    d = _unit_exp(sb) - _unit_exp(zb)
    zero = ((sb & 0x7FFF) == 0) | ((zb & 0x7FFF) == 0)
    cond = zero | ((d >= -12) & (d <= 12 - qbits))
    s = sb.view(np.float16).astype(np.float64)
    z = zb.view(np.float16).astype(np.float64)
    inexact_seen = False
    for q in (0, 1, 2, 3, 7, 15) + ((100, 255) if qbits == 8 else ()):
        exact = q * s + z                       # exact in fp64 (< 53 bits)
        rep = exact.astype(np.float32).astype(np.float64) == exact
        assert np.all(rep[cond]), (qbits, q)
        inexact_seen |= bool(np.any(~rep[~cond]))
    assert inexact_seen                          # the condition is not vacuous
