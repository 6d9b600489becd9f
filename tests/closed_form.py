"""Float64 closed forms that pin FP32 outputs independently of the oracle's own formula.

Row-scaled linears on INT8 activations (the INT8 and INT4 formats):
    y[m, r] = acc[m, r] * xs[m] * s[r] + bias[r],   acc = the exact integer product xq @ W^T.
The FP32 epilogue rounds (float)acc, the xs multiply, the s multiply and the bias add once each, so its error is
at most a few units of 2^-24 of |acc| * xs * s + |bias|; 1e-6 of that magnitude bounds it with room. A dropped
or doubled per-token xs, a scale indexed by token, or the bias added before the xs multiply are off by O(1) of it.
The reference tests normalise the same way (tests/test_int8_gemv.c:10-44, tests/test_q35_int4.c:24-33).
"""
import numpy as np

ROWSCALE_TOL = 1e-6


def exact_acc(xq, vals, chunk=16384):
    """xq [M, >=K] int8, vals [N, K] integer codes -> the exact integer product [M, N] as float64.

    float64 holds every partial sum exactly (|sum| < 2^53); rows are taken in chunks to bound memory."""
    K = vals.shape[1]
    a = xq[:, :K].astype(np.float64)
    out = np.empty((a.shape[0], vals.shape[0]))
    for r0 in range(0, vals.shape[0], chunk):
        out[:, r0:r0 + chunk] = a @ vals[r0:r0 + chunk].astype(np.float64).T
    return out


def rowscale_error(y, acc, xs, s, bias=None):
    """Largest |y - closed form| / (|acc| * xs * s + |bias|) over all outputs (float64)."""
    xs = xs.astype(np.float64)[:, None]
    s = (np.ones(acc.shape[1]) if s is None else s.astype(np.float64))[None, :]
    b = np.zeros(acc.shape[1]) if bias is None else bias.astype(np.float64)
    want = acc * xs * s + b[None, :]
    mag = np.abs(acc) * xs * s + np.abs(b)[None, :]
    return float(np.max(np.abs(y.astype(np.float64) - want) / (mag + 1e-300)))
