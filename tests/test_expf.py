"""The exponential of the exact-order mode against the x86 reference build's exp.

The reference's x86 build takes softmax and SwiGLU exponentials from the platform libm
(f32::exp, real_llm.rs:9595 and 9803): glibc's expf, which the oracle calls.  The
library's routine (k2t_expf_host, the same source as the device code) is compared with
it over every one of the 2^32 fp32 bit patterns: NaNs, infinities, subnormal results
and both overflow limits included.  A bit-exact match over the whole domain is the
only claim, so the check is exhaustive rather than sampled."""
import ctypes as C

import numpy as np

import k2t
import oracle as O


def _host_fn():
    return C.cast(k2t.lib().k2t_expf_host, C.c_void_p).value


def test_expf_host_matches_libm_on_every_fp32_input():
    first = C.c_uint32()
    bad = O.lib().or_expf_mismatches(_host_fn(), 0, 1 << 32, 8, C.byref(first))
    assert bad == 0, f"{bad} inputs differ from libm expf, first bit pattern {first.value:#010x}"


def test_mismatch_counter_detects_a_wrong_routine():
    # a routine that is off by one ulp on part of a range must be counted exactly there
    F = C.CFUNCTYPE(C.c_float, C.c_float)

    def off(x):
        y = np.float32(np.exp(np.float64(x)))
        return float(np.nextafter(y, np.float32(np.inf))) if x > 1.0 else float(y)

    cb = F(off)
    lo = int(np.float32(1.0).view(np.uint32)) - 2000  # 2000 inputs below 1, then 1 and above
    first = C.c_uint32()
    bad = O.lib().or_expf_mismatches(C.cast(cb, C.c_void_p).value, lo, lo + 4000, 1, C.byref(first))
    above = int(np.sum(np.arange(lo, lo + 4000, dtype=np.uint32).view(np.float32) > 1.0))
    assert above > 0
    # every input above 1 differs; below 1, exp rounded from double may still equal expf
    assert bad >= above
    assert lo <= first.value < lo + 4000


def test_expf_host_special_values():
    f = k2t.lib().k2t_expf_host
    assert f(0.0) == 1.0
    assert f(-0.0) == 1.0
    assert f(float("inf")) == float("inf")
    assert f(float("-inf")) == 0.0
    assert np.isnan(f(float("nan")))
    assert f(89.0) == float("inf")
    assert f(-104.0) == 0.0
