"""Host-side helpers of the product package, on the CPU."""
import numpy as np

import oracle


def test_rope_tables_match_oracle():
    """relux_amd.rope_tables (rope.go:50-75) against the oracle's C tables."""
    from relux_amd import rope_tables
    for D, base, n in ((16, 10000.0, 64), (128, 10000.0, 4096), (64, 500000.0, 300)):
        c, s = rope_tables(D, base, n, "cpu")
        oc, os_ = oracle.rope_tables(D, base, n)
        oc, os_ = oc.reshape(n, D // 2), os_.reshape(n, D // 2)
        # numpy's f64 cos/sin may differ from libm by an ulp before the f32
        # rounding; allow one f32 ulp.
        np.testing.assert_array_max_ulp(c.numpy(), oc, maxulp=1)
        np.testing.assert_array_max_ulp(s.numpy(), os_, maxulp=1)
        assert (c.numpy() == oc).mean() > 0.999
