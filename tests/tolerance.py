"""The floating-point bar for the dequantised (fp16-output) paths.

north_star: max relative error <= 1e-2 with fp16 output. Relative error is
taken per element against the f64 ground truth, with the denominator floored
twice over: at 0.1 x the RMS of the reference outputs (outputs are sums of
thousands of signed terms, so some land near zero where any change of
summation order is an unbounded *relative* change) and, as the reference's
own tests do, at 0.1 (crates/minicpm-v/src/quant.rs:552; :313 floors at
1e-3 for its f32 CPU route); both measures must stay within 1e-2.
"""
import os

import numpy as np

FP16_REL_TOL = 1e-2

# The reference's own floor for its fp16 checks: |ref|.max(0.1)
# (crates/minicpm-v/src/quant.rs:552), whose Metal FP16 route it holds to
# 5e-2 (:556).
REF_CLAMP = 0.1

# (test, against the f64 truth?, rms-floored error, error under the
# reference's clamp) of every rel_err call in this session, summarised by
# conftest.py at the end.
RECORD = []


def ref_clamp_err(got, ref):
    """max |got - ref| / max(|ref|, 0.1): the reference's own measure."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    return float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), REF_CLAMP)))


def rel_err(got, ref, truth=True):
    """The bar's measure of `got` against `ref`. Against the f64 truth
    (truth=True) it is the larger of the rms-floored error and the
    reference's own measure, |got - ref| / |ref|.max(0.1) (quant.rs:552), so
    a test asserting rel_err <= 1e-2 holds both to 1e-2 (measured over the
    GPU suite: at most 4e-3 under the reference's measure). truth=False
    marks a comparison with another rounded route (the reference's
    dequantise-to-f16 route restated by the oracle, say), held to the
    rms-floored measure only: such a route's own rounding puts it up to
    ~0.4 from the truth under the 0.1 floor at K = 8192."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if ref.size == 0:
        return 0.0
    if not np.all(np.isfinite(got)):
        return float("inf")
    rms = float(np.sqrt(np.mean(ref * ref)))
    floor = max(0.1 * rms, 1e-30)
    err = float(np.max(np.abs(got - ref) / np.maximum(np.abs(ref), floor)))
    clamp = ref_clamp_err(got, ref)
    RECORD.append((os.environ.get("PYTEST_CURRENT_TEST", "?").split(" ")[0], truth, err, clamp))
    return max(err, clamp) if truth else err
