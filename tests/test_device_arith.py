"""The float-reciprocal division of engine.h (`rcp_u` / `divmod_u`), restated in numpy float32.

The kernels divide lane indices by a wave-uniform divisor (token row m by Tv in the QKV epilogue,
combine row R by NH * Tv and then Tv) as q = trunc(m * rcp(d)) followed by one correction step, with
rcp the hardware's v_rcp_f32 (within 1 ulp of 1 / d). The claim is that this equals integer division
for every m below 2^20. Here the reciprocal is taken as the correctly rounded 1 / d and as its two
neighbours one ulp away, which brackets v_rcp_f32's result, and the quotient and remainder are
compared with numpy's integer division over every m below 2^18 for the divisors the kernels see
(every d up to 256, the pi0.5 and MolmoAct2 token counts and their multiples by the head count) and
a spread of others up to 2^18. A planted mistake (the correction step left out) must fail.
"""
import numpy as np


def _divmod_float(m, d, rd, correct=True):
    q = (m.astype(np.float32) * np.float32(rd)).astype(np.int64)  # float32 product, truncated
    if correct:
        r = m - q * d
        q = np.where(r < 0, q - 1, np.where(r >= d, q + 1, q))
    return q, m - q * d


def _reciprocals(d):
    r0 = np.float32(1.0) / np.float32(d)
    return (np.nextafter(r0, np.float32(0)), r0, np.nextafter(r0, np.float32(np.inf)))


def _divisors():
    tok = [10, 30, 50, 200, 493, 968, 1018]
    ds = set(range(1, 257)) | set(tok) | {8 * t for t in tok} | {16 * t for t in tok}
    ds |= {int(x) for x in np.unique(np.geomspace(257, 1 << 18, 60).astype(np.int64))}
    return sorted(ds)


def test_divmod_u_matches_integer_division():
    m = np.arange(1 << 18, dtype=np.int64)
    for d in _divisors():
        for rd in _reciprocals(d):
            q, r = _divmod_float(m, d, rd)
            bad = np.flatnonzero((q != m // d) | (r != m % d))
            assert bad.size == 0, (d, float(rd), int(m[bad[0]]))


def test_divmod_u_needs_its_correction_step():
    m = np.arange(1 << 18, dtype=np.int64)
    wrong = 0
    for d in (3, 7, 10, 50, 968):
        for rd in _reciprocals(d):
            q, _ = _divmod_float(m, d, rd, correct=False)
            wrong += int((q != m // d).sum())
    assert wrong > 0
