"""Dense oracles for the NF4 GEMMs (A7-A9) -- test infrastructure only.

Reference semantics:
  * forward  Y[T,N] = X[T,K] . W[N,K]^T (+ bias), fp16 operands, fp32
    accumulation, bias added to the fp32 accumulator, one fp16 rounding
    (solution/kernels/nf4_gemm.py:59-71; bnb fallback F.linear,
    solution/nf4_patch.py:4-7,108-120);
  * backward dX[T,K] = dY[T,N] . W[N,K] (solution/kernels/nf4_gemm.py:44-47,
    108-118; bnb MatMul4Bit.backward -> torch.matmul(dY, dequant(W))).
W is the bit-exact decoded fp16 weight (oracle.nf4).  The oracle computes the
products in float64 (a textbook matmul), so it is the "ideal" that any fp32
accumulation order approximates.  The acceptance gate is the reference's
preregistered one (experiments/reports/EXP-002.md:60-76):
assert_close(rtol=2e-3, atol=2e-3) on the fp16 output plus relative L2 <= 1e-3.

Beyond EXP-002's calibrated reductions (K <= 8960), ``no_worse_than_reference``
compares the errors of a result and of the reference's own decode-then-dense
path against the exact-weight product (the north star's "no worse than the
reference's own error").

Pins: the float64 product is numpy's matmul (a library routine); tests plant a
transposed operand and a dropped bias in the oracle on tiny shapes and check
that the gate rejects them, and compare against a brute-force triple loop.
"""

import numpy as np

RTOL = 2e-3
ATOL = 2e-3
REL_L2 = 1e-3
SLACK = 1.25     # no_worse_than_reference: allowed ratio to the reference's own error


def linear(x, w, bias=None):
    """float64 X . W^T (+ bias); x [T,K], w [N,K] (any float dtype)."""
    y = np.asarray(x, np.float64) @ np.asarray(w, np.float64).T
    if bias is not None:
        y = y + np.asarray(bias, np.float64)[None, :]
    return y


def linear_dx(dy, w):
    """float64 dY . W; dy [T,N], w [N,K]."""
    return np.asarray(dy, np.float64) @ np.asarray(w, np.float64)


def brute_force_linear(x, w, bias=None):
    """Triple loop, for tiny shapes only (pins ``linear``)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    t, k = x.shape
    n = w.shape[0]
    y = np.zeros((t, n))
    for i in range(t):
        for j in range(n):
            acc = 0.0
            for kk in range(k):
                acc += x[i, kk] * w[j, kk]
            y[i, j] = acc + (0.0 if bias is None else float(bias[j]))
    return y


def no_worse_than_reference(actual, exact, reference, slack=SLACK):
    """Return (ok, ratio_max, ratio_l2): is ``actual`` as close to the exact-weight
    product as the reference's own decode-then-dense result is?

    ``exact`` is the float64 product with the unrounded weight NF4 * scale
    (oracle.nf4.decode_exact); ``reference`` is what the reference computes: the
    product of the fp16-decoded weight with the output rounded to fp16.  Both the
    largest element error and the relative L2 error of ``actual`` against
    ``exact`` may exceed the reference's by at most the factor ``slack``.  This is
    the north star's "no worse than the reference's own error", for reductions
    longer than EXP-002 calibrated its fixed 2e-3 element tolerance on (K <= 8960):
    there the rounding of each decoded weight alone moves the decoded-weight
    product by more than 2e-3 (the deviation grows as sqrt(K)).
    """
    a = np.asarray(actual, np.float64)
    e = np.asarray(exact, np.float64)
    r = np.asarray(reference, np.float64)
    if a.shape != e.shape or not np.all(np.isfinite(a)):
        return False, float("inf"), float("inf")
    denom = max(np.linalg.norm(e), 1e-300)
    ra = np.abs(a - e).max(initial=0.0) / max(np.abs(r - e).max(initial=0.0), 1e-300)
    rl = (np.linalg.norm(a - e) / denom) / max(np.linalg.norm(r - e) / denom, 1e-300)
    return bool(ra <= slack and rl <= slack), float(ra), float(rl)


def gate(actual, expected, rtol=RTOL, atol=ATOL, rel_l2=REL_L2):
    """Return (ok, max_abs_err, rel_l2_err) for the EXP-002 correctness gate."""
    a = np.asarray(actual, np.float64)
    e = np.asarray(expected, np.float64)
    if a.shape != e.shape or not np.all(np.isfinite(a)):
        return False, float("inf"), float("inf")
    err = np.abs(a - e)
    ok_elem = bool(np.all(err <= atol + rtol * np.abs(e)))
    denom = np.linalg.norm(e)
    rel = float(np.linalg.norm(a - e) / denom) if denom > 0 else float(np.linalg.norm(a - e))
    return ok_elem and rel <= rel_l2, float(err.max(initial=0.0)), rel
