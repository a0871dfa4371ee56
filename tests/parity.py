"""BF16 comparison helpers for parity tests.

The parity bar: the BF16 output is within 1 BF16
ulp of the CPU oracle, or -- where the accumulation order differs -- the
relative L2 error is <= 1e-2 with cosine similarity >= 0.9999.  The
reference's own test tolerance (allclose rtol .01, atol .001 against an FP64
oracle, tests/fp8_tensor_test.cpp:23-26) is checked as well.
"""
import numpy as np


def bf16_to_f32(bits):
    return (np.asarray(bits, np.uint16).astype(np.uint32) << 16).view(np.float32)


def ulp_distance(a_bits, b_bits):
    """Distance in BF16 ulps along the ordered integer line (sign-magnitude
    mapped to two's complement); +0 and -0 are 0 apart."""
    def ordered(b):
        b = np.asarray(b, np.uint16).astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7fff), b)
    return np.abs(ordered(a_bits) - ordered(b_bits))


def stats(got_bits, ref_bits):
    g = bf16_to_f32(got_bits).astype(np.float64).ravel()
    r = bf16_to_f32(ref_bits).astype(np.float64).ravel()
    u = ulp_distance(got_bits, ref_bits).ravel()
    diff = np.linalg.norm(g - r)
    nr = np.linalg.norm(r)
    rel = diff / nr if nr > 0 else (0.0 if diff == 0 else np.inf)
    ng = np.linalg.norm(g)
    cos = float(g @ r / (ng * nr)) if ng > 0 and nr > 0 else (1.0 if diff == 0 else 0.0)
    return {
        "max_ulp": int(u.max()) if u.size else 0,
        "frac_le1ulp": float((u <= 1).mean()) if u.size else 1.0,
        "exact": float((u == 0).mean()) if u.size else 1.0,
        "rel_l2": float(rel),
        "cos": cos,
        "max_abs": float(np.abs(g - r).max()) if g.size else 0.0,
        "finite": bool(np.isfinite(g).all()),
    }


def assert_parity(got_bits, ref_bits, what="", min_exact=0.9, elementwise=True):
    """min_exact: fraction of outputs that must be bit-identical to the oracle.
    Kernels that keep the reference rounding point bf16(decode*scale) differ
    from the FP64 oracle only where the FP32 sum lands next to a BF16 rounding
    boundary, so nearly all outputs match exactly; pass None for paths whose
    accumulation order legitimately differs more."""
    s = stats(got_bits, ref_bits)
    assert s["finite"], f"{what}: non-finite output {s}"
    ok = s["max_ulp"] <= 1 or (s["rel_l2"] <= 1e-2 and s["cos"] >= 0.9999)
    assert ok, f"{what}: parity failed {s}"
    if min_exact is not None:
        assert s["exact"] >= min_exact, f"{what}: only {s['exact']:.4f} bit-exact {s}"
    if not elementwise:
        return s
    g = bf16_to_f32(got_bits).astype(np.float64)
    r = bf16_to_f32(ref_bits).astype(np.float64)
    assert np.allclose(g, r, rtol=0.01, atol=0.001), f"{what}: allclose(.01,.001) failed {s}"
    return s
