"""CPU checks of integer arithmetic the HIP kernels do in float.

The layer-resident kernel divides small non-negative integers by a run-time
divisor d as trunc((n + 0.5) * inv) with inv the hardware reciprocal of d
(lich_amd/csrc/ipc_resident.hip, qdiv).  The reciprocal is within one ulp of
1/d; this checks, in float32 arithmetic, that the quotient is exact for every
inv within one ulp of 1/d over the divisors and numerators the kernel uses
(tile counts and the batch: d <= 256, n < 2^17)."""
import numpy as np


def test_qdiv_is_exact_for_reciprocals_within_one_ulp():
    n = np.arange(1 << 17, dtype=np.int64)
    nf = (n.astype(np.float32) + np.float32(0.5)).astype(np.float32)
    for d in range(1, 257):
        exact = np.float32(1.0) / np.float32(d)
        for inv in (np.nextafter(exact, np.float32(0)), exact, np.nextafter(exact, np.float32(1))):
            q = (nf * np.float32(inv)).astype(np.float32).astype(np.int64)  # truncation, as (int) on the device
            assert np.array_equal(q, n // d), (d, inv)
