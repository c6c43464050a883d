"""Numerical-health probe statistics.  TEST INFRASTRUCTURE ONLY (the HIP probe pass is
checked against it; the product never calls it).

Restates one standalone pass of probe_f16_stats / probe_f32_stats
(AnimaKernels.metal:1921-2040) over a whole buffer, as NumericalMonitor reads the slot
(NumericalMonitor.swift:136-170):
- flags: bit0 a NaN, bit1 a +Inf, bit2 a -Inf, bit3 a finite |v| > 65504
  (AnimaKernels.metal:295-301);
- max |v| over the finite values as fp32 bits, 0 when there is none;
- the first index that set a flag, 0xFFFFFFFF when none did.
Slots accumulate passes: flags OR, max of the max, min of the first index
(the relaxed atomics of :1968-1976)."""

from __future__ import annotations

import numpy as np

FLAG_NAN, FLAG_POS_INF, FLAG_NEG_INF, FLAG_HALF_OVERFLOW = 1, 2, 4, 8
NO_INDEX = 0xFFFFFFFF
EMPTY_SLOT = (0, 0, NO_INDEX)   # beginRun (NumericalMonitor.swift:205-212)


def probe_stats(values) -> tuple[int, int, int]:
    """(flags, max |v| fp32 bits, first index) of one pass over an fp16 or fp32 array."""
    x = np.asarray(values).astype(np.float32).ravel()   # fp16 -> fp32 is exact
    nan = np.isnan(x)
    inf = np.isinf(x)
    finite = ~(nan | inf)
    mag = np.abs(x)
    over = finite & (mag > np.float32(65504.0))
    flags = ((FLAG_NAN if nan.any() else 0) | (FLAG_POS_INF if (inf & (x > 0)).any() else 0)
             | (FLAG_NEG_INF if (inf & (x < 0)).any() else 0) | (FLAG_HALF_OVERFLOW if over.any() else 0))
    bad = np.flatnonzero(nan | inf | over)
    first = int(bad[0]) if bad.size else NO_INDEX
    maxbits = int(mag[finite].max().view(np.uint32)) if finite.any() else 0
    return flags, maxbits, first


def accumulate(slot: tuple[int, int, int], one_pass: tuple[int, int, int]) -> tuple[int, int, int]:
    """A slot after another pass into it."""
    return slot[0] | one_pass[0], max(slot[1], one_pass[1]), min(slot[2], one_pass[2])
