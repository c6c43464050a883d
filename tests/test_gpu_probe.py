"""GPU parity of the numerical-health probe pass (anima_numerics_probe_encode) with the
oracle: the reference's known answers, random fp16/fp32 buffers with NaN/Inf/overflow
planted at chosen indices (16-byte chunked and element-wise paths, ragged tails, grid
strides), slot accumulation across passes and slots, and the reset.  Bit-exact: the slot
words are integers."""

import numpy as np
import pytest
import torch

from animaxs_amd import NumericalMonitor
from oracle import probe as oprobe

pytestmark = pytest.mark.gpu


def _words(mon, slot):
    torch.cuda.synchronize()
    w = mon.buffer[4 * slot:4 * slot + 4].cpu().numpy().view(np.uint32)
    return int(w[0]), int(w[1]), int(w[2])


def test_reset_and_known_answers(ctx):
    """NumericalMonitorTests.swift:167-189 through the device pass: the fp16 buffer into
    selfQToken, the fp32 buffer into velocity; every other slot stays empty."""
    mon = NumericalMonitor(ctx)
    for s in range(mon.slots):
        assert _words(mon, s) == oprobe.EMPTY_SLOT
    h = torch.tensor([1.0, float("nan"), 3.0, float("inf")], dtype=torch.float16, device="cuda")
    f = torch.tensor([-2.0, 4.0, 80_000.0, float("-inf")], dtype=torch.float32, device="cuda")
    mon.encode_probe(h, "selfQToken")
    mon.encode_probe(f, "velocity")
    q, v = mon.stats("selfQToken"), mon.stats("velocity")
    assert q.has_nan and q.has_pos_inf and q.first_index == 1 and q.max_abs == 3.0
    assert v.has_neg_inf and v.has_half_overflow and v.max_abs == 80_000.0 and v.first_index == 2
    for name in mon.PROBES:
        if name not in ("selfQToken", "velocity"):
            assert _words(mon, mon.slot(name)) == oprobe.EMPTY_SLOT, name
    mon.begin_run()
    assert _words(mon, mon.slot("velocity")) == oprobe.EMPTY_SLOT


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
@pytest.mark.parametrize("count,offset,plants", [
    (1, 0, []),
    (7, 0, [(3, "nan")]),                                  # one 16-byte chunk short: element path only
    (4099, 0, [(4098, "-inf")]),                           # offender in the ragged tail
    (4096 * 3 + 5, 1, [(5000, "over"), (12000, "nan")]),   # offset 1: element-wise path
    (3_000_001, 0, [(2_999_000, "inf"), (1_700_000, "over"), (2_500_000, "nan")]),  # grid stride
    (2_000_000, 8, []),                                     # all finite: max only, no flag
])
def test_pass_matches_oracle(ctx, dtype, count, offset, plants):
    g = torch.Generator().manual_seed(count + offset)
    x = (torch.randn(count + offset, generator=g) * 1000).to(dtype)
    for i, kind in plants:
        val = {"nan": float("nan"), "inf": float("inf"), "-inf": float("-inf"),
               "over": 70_000.0 if dtype == torch.float32 else float("inf")}[kind]
        x[offset + i] = val
    print(f"PROBE dtype={dtype} count={count} offset={offset} plants={plants}", flush=True)
    mon = NumericalMonitor(ctx, slots=2)
    xd = x.cuda()
    mon.encode_probe(xd, 1, count=count, offset=offset)
    assert _words(mon, 1) == oprobe.probe_stats(x[offset:offset + count].numpy())
    assert _words(mon, 0) == oprobe.EMPTY_SLOT


def test_passes_accumulate_in_a_slot(ctx):
    """Three passes into one slot give the OR of the flags, the max of the maxima and the
    min of the first indices; a pass into another slot leaves it alone."""
    g = torch.Generator().manual_seed(11)
    a = torch.randn(50_000, generator=g)
    a[40_000] = float("inf")
    b = (torch.randn(30_000, generator=g) * 5).half()
    b[123] = float("nan")
    c = torch.randn(70_000, generator=g) * 1e6          # most |v| above 65504: the overflow flag
    mon = NumericalMonitor(ctx, slots=3)
    dev = [t.cuda() for t in (a, b, c)]
    for t in dev:
        mon.encode_probe(t, 2)
    mon.encode_probe(dev[0], 0)
    want = oprobe.EMPTY_SLOT
    for t in (a, b, c):
        want = oprobe.accumulate(want, oprobe.probe_stats(t.numpy()))
    assert _words(mon, 2) == want
    assert _words(mon, 0) == oprobe.probe_stats(a.numpy())
    assert _words(mon, 1) == oprobe.EMPTY_SLOT
