"""The numerical-health probe on the CPU: the oracle pinned to the reference's known
answers (AnimaXSTests/NumericalMonitorTests.swift) and closed forms, the host-side slot
decoding (NumericalMonitor.Stats), and the C ABI's argument checks (nothing launches)."""

import numpy as np
import pytest

import animaxs_amd
from animaxs_amd import AnimaError, ProbeStats, _abi
from animaxs_amd._abi import call
from oracle import probe as oprobe

F32_BITS = lambda v: int(np.float32(v).view(np.uint32))  # noqa: E731


def test_float_to_half_probe_known_answers():
    """NumericalMonitorTests.swift:83-123: the fp32 input of float_to_half_probe raises every
    flag, the first offender is the NaN at index 2 and the max over the finite values is
    70000 (65504 itself is not an overflow)."""
    v = np.array([1.0, -1.0, np.nan, np.inf, -np.inf, 70_000.0, 65504.0, 0.5], np.float32)
    flags, maxbits, first = oprobe.probe_stats(v)
    assert flags == oprobe.FLAG_NAN | oprobe.FLAG_POS_INF | oprobe.FLAG_NEG_INF | oprobe.FLAG_HALF_OVERFLOW
    assert first == 2
    assert maxbits == F32_BITS(70_000.0)


def test_standalone_pass_known_answers():
    """NumericalMonitorTests.swift:167-189: the fp16 pass sees NaN and +Inf with the first
    offender at 1; the fp32 pass sees -Inf and the 80000 overflow, max 80000."""
    f16 = oprobe.probe_stats(np.array([1.0, np.nan, 3.0, np.inf], np.float16))
    assert f16[0] == oprobe.FLAG_NAN | oprobe.FLAG_POS_INF and f16[2] == 1 and f16[1] == F32_BITS(3.0)
    f32 = oprobe.probe_stats(np.array([-2.0, 4.0, 80_000.0, -np.inf], np.float32))
    assert f32[0] == oprobe.FLAG_NEG_INF | oprobe.FLAG_HALF_OVERFLOW
    assert f32[1] == F32_BITS(80_000.0) and f32[2] == 2


def test_probe_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal(1000).astype(np.float32)
    assert oprobe.probe_stats(x) == (0, F32_BITS(np.abs(x).max()), oprobe.NO_INDEX)
    # 65504 is the largest finite fp16; the next fp32 above it overflows fp16
    edge = np.array([65504.0, np.nextafter(np.float32(65504.0), np.float32(np.inf))], np.float32)
    assert oprobe.probe_stats(edge)[0] == oprobe.FLAG_HALF_OVERFLOW and oprobe.probe_stats(edge)[2] == 1
    assert oprobe.probe_stats(np.array([-0.0, 0.0], np.float32)) == (0, 0, oprobe.NO_INDEX)
    for k in (0, 17, 998):
        y = x.copy()
        y[k] = np.nan
        y[-1] = -np.inf
        flags, _, first = oprobe.probe_stats(y)
        assert first == k and flags == oprobe.FLAG_NAN | oprobe.FLAG_NEG_INF
    only_bad = np.array([np.nan, np.inf], np.float16)
    assert oprobe.probe_stats(only_bad)[1] == 0


def test_slot_accumulation():
    a = oprobe.probe_stats(np.array([1.0, np.inf], np.float32))
    b = oprobe.probe_stats(np.array([np.nan, 5.0, 2.0], np.float32))
    acc = oprobe.accumulate(oprobe.accumulate(oprobe.EMPTY_SLOT, a), b)
    assert acc == (oprobe.FLAG_POS_INF | oprobe.FLAG_NAN, F32_BITS(5.0), 0)


def test_stats_condition_decoding():
    """NumericalMonitorTests.swift:34-51."""
    assert not ProbeStats().has_issue
    assert ProbeStats().condition == "non-finite value detected"
    cases = {1: "NaN detected", 2: "positive Inf detected", 4: "negative Inf detected",
             16: "residual became NaN", 32: "residual became non-finite",
             8: "value exceeded FP16 finite range"}
    for flags, text in cases.items():
        assert ProbeStats(flags=flags).condition == text
    s = ProbeStats.from_words([3, F32_BITS(70_000.0), 2, 0])
    assert s.has_nan and s.has_pos_inf and not s.has_neg_inf and s.max_abs == 70_000.0 and s.first_index == 2
    assert len(animaxs_amd.NumericalMonitor.PROBES) * 16 == 512   # the reference's 512-byte buffer


FAKE = 0x10000  # placeholder device address; validation fails before it is used


@pytest.fixture(scope="module")
def ctx():
    c = animaxs_amd.Context(0)
    yield c
    c.close()


def _expect(status, fragment, *args):
    with pytest.raises(AnimaError) as ei:
        call(*args)
    assert ei.value.status == status and fragment in ei.value.message, ei.value


def test_probe_argument_checks(ctx):
    B = _abi.Buffer
    vals, stats = B(FAKE, 1 << 20), B(FAKE, 64)
    enc = "anima_numerics_probe_encode"
    _expect(_abi.E_INVALID_ARGUMENT, "dtype", enc, ctx.handle, vals, 0, 16, 2, stats, 0)
    _expect(_abi.E_INVALID_SHAPE, "count and offset", enc, ctx.handle, vals, 0, -1, 0, stats, 0)
    _expect(_abi.E_INVALID_SHAPE, "below 0xFFFFFFFF", enc, ctx.handle, vals, 0, 0xFFFFFFFF, 0, stats, 0)
    _expect(_abi.E_INVALID_ARGUMENT, "slot", enc, ctx.handle, vals, 0, 16, 0, stats, -1)
    _expect(_abi.E_OUT_OF_BOUNDS, "values", enc, ctx.handle, vals, (1 << 19) - 4, 8, 0, stats, 0)
    _expect(_abi.E_OUT_OF_BOUNDS, "stats", enc, ctx.handle, vals, 0, 16, 1, stats, 4)
    _expect(_abi.E_MISALIGNED, "aligned", enc, ctx.handle, B(FAKE + 2, 1 << 20), 0, 16, 1, stats, 0)
    _expect(_abi.E_INVALID_SHAPE, "slots", "anima_numerics_probe_reset_encode", ctx.handle, stats, -1)
    _expect(_abi.E_OUT_OF_BOUNDS, "stats", "anima_numerics_probe_reset_encode", ctx.handle, stats, 5)
    call(enc, ctx.handle, vals, 0, 0, 0, stats, 3)                     # count 0: nothing to do
    call("anima_numerics_probe_reset_encode", ctx.handle, stats, 0)     # no slots: nothing to do
