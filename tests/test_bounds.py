"""Error bounds that the grouping kernel's bf16 dot-product pre-pass relies on, checked on the
CPU against exact arithmetic (no GPU, no library call).

The pre-pass (grp_assign_kernel in vcx_group.hip) forms |x - c|^2 as |x|^2 + |c|^2 - 2 x.c,
with each binary32 center entering the bf16 MFMA as two bf16 parts, and settles a token only
when its best distance is separated from every other by the bound E = kappa * S + 1e-30
(S = |x|^2 + |c|^2). A token it leaves open goes to the binary32 and fp64 chains, so the only
requirement is that the bound holds."""
import numpy as np

U = 2.0 ** -24


def rn_bf16(x):
    """binary32 -> bf16 (round to nearest, ties to even), returned as binary32."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    r = ((b + 0x7FFF + ((b >> 16) & 1)) >> 16) << 16
    return r.astype(np.uint32).view(np.float32)


def kappa(d):
    """The kernel's factor: ((D/4 + 9 + 2.016 (D + D/32)) u + 2^-17) * 1.02."""
    return ((d / 4 + 9 + 2.016 * (d + d // 32)) * U + 2.0 ** -17) * 1.02


def test_two_part_split_leaves_at_most_2_pow_minus_17():
    # hi = RN_bf16(c), lo = RN_bf16(c - hi): c - hi is exact in binary32 and the parts leave
    # at most 2^-17 |c|; the bound is attained to within 0.2 %, so 2^-18 would be wrong.
    rng = np.random.default_rng(0)
    c = (rng.standard_normal(4_000_000) * np.exp2(rng.integers(-30, 30, 4_000_000))).astype(np.float32)
    c = c[c != 0]
    hi = rn_bf16(c)
    diff = (c - hi).astype(np.float32)
    np.testing.assert_array_equal(diff.astype(np.float64), c.astype(np.float64) - hi.astype(np.float64))
    lo = rn_bf16(diff)
    rel = np.abs(c.astype(np.float64) - hi.astype(np.float64) - lo.astype(np.float64)) / np.abs(c.astype(np.float64))
    assert rel.max() <= 2.0 ** -17
    assert rel.max() > 0.998 * 2.0 ** -17


def _prepass_distance(x, c):
    """The pre-pass arithmetic with every accumulation rounded in sequence (one admissible
    order of the MFMA and dot2 roundings): x [n, D] bf16-valued binary32, c [D] binary32."""
    n, d = x.shape
    f32 = np.float32
    # |x|^2: lane group G holds channels 32k + 8G + [0, 8) of each 32-channel step; a dot2
    # step adds two exact squares with a rounding after each; then (g0 + g1) + (g2 + g3)
    groups = []
    for g in range(4):
        acc = np.zeros(n, f32)
        for k in range(d // 32):
            for e in range(4):
                for h in range(2):
                    ch = 32 * k + 8 * g + 2 * e + h
                    acc = (acc + (x[:, ch] * x[:, ch]).astype(f32)).astype(f32)
        groups.append(acc)
    x2 = (((groups[0] + groups[1]).astype(f32)) + ((groups[2] + groups[3]).astype(f32))).astype(f32)
    c2 = f32(np.sum(c.astype(np.float64) ** 2))
    hi = rn_bf16(c)
    lo = rn_bf16((c - hi).astype(f32))
    parts = []
    for part in (hi, lo):
        acc = np.zeros(n, f32)
        for ch in range(d):  # products of bf16 values are exact in binary32
            acc = (acc + (x[:, ch] * part[ch]).astype(f32)).astype(f32)
        parts.append(acc)
    p = (parts[0] + parts[1]).astype(f32)
    s = (x2 + c2).astype(f32)
    return (s - f32(2.0) * p).astype(f32)


def test_prepass_distance_within_the_kernel_bound():
    # Tokens near the center and far from it, at a large common offset (where |x|^2 + |c|^2
    # dwarfs |x - c|^2) and around zero: the rounded pre-pass distance stays within kappa * S
    # of the exact one. Exact reference: binary32 and bf16 values widen exactly to longdouble
    # (64-bit significand), whose sums of 128 squares of 33-bit differences are exact. The
    # bound is a worst case over every rounding order: these errors reach about 25 u * S
    # against kappa = 290-440 u, so this check catches a slip of a factor of ten or more (a
    # dropped D, u taken as 2^-53), and the split test above pins the 2^-17 term exactly.
    rng = np.random.default_rng(1)
    for d in (64, 128):
        for offset, spread in ((0.0, 1.0), (40.0, 1.0), (3.0e4, 1.0), (0.0, 1e-3)):
            c = (offset + rng.standard_normal(d)).astype(np.float32)
            x = rn_bf16(c + spread * rng.standard_normal((2000, d)).astype(np.float32))
            got = _prepass_distance(x, c).astype(np.longdouble)
            xl, cl = x.astype(np.longdouble), c.astype(np.longdouble)
            exact = ((xl - cl) ** 2).sum(axis=1)
            s = (xl ** 2).sum(axis=1) + (cl ** 2).sum()
            err = np.abs(got - exact)
            assert np.all(err <= np.longdouble(kappa(d)) * s + np.longdouble(1e-30)), (d, offset, spread)
