"""RMSNorm inputs whose mean square lies on a float rounding boundary.

The reference sums the squares as one serial chain of double adds
(sml/sml-run.c:147-152) and rounds ss/n to float. These vectors make that
chain end exactly on the midpoint between two floats while the sum of the
same squares in any tree order ends above it: x[0] = 1024 comes first, two
more elements bring the chain to M*n (M the midpoint), and every other
element squares to 2^-34, a quarter of the chain's last place from then on,
so the chain drops each of them while a tree sum keeps them. The two
orders' float(ss/n) then differ by one place, and a kernel that took the
tree sum without checking how close it lies to a boundary would be caught.
"""
import numpy as np

TINY = np.float32(2.0 ** -17)


def serial_ss(x):
    """The reference's chain: double adds of exact squares, in order."""
    x64 = np.asarray(x, np.float32).astype(np.float64)
    return float(np.cumsum(x64 * x64)[-1])


def tree_ss(x):
    """The same squares summed pairwise (numpy's order)."""
    x64 = np.asarray(x, np.float32).astype(np.float64)
    return float(np.sum(x64 * x64))


def mean_alike(s, n):
    """The kernels' window test: float(ss/n) for every ss within
    4*(n+4)*2^-53*s of s, or None when a rounding boundary lies inside."""
    d = s * (4 * (n + 4) * 2.0 ** -53)
    lo, hi = np.float32((s - d) / n), np.float32((s + d) / n)
    return lo if lo == hi else None


def _largest_root_below(r):
    """The largest float32 f >= 0 with f*f <= r (in double)."""
    f = np.float32(np.sqrt(r))
    while np.float64(f) * np.float64(f) > r:
        f = np.nextafter(f, np.float32(0))
    while np.float64(np.nextafter(f, np.float32(1e30))) ** 2 <= r:
        f = np.nextafter(f, np.float32(1e30))
    return f


def boundary_vector(n, rng):
    """x[n] (float32) whose serial sum of squares is exactly n times a float
    midpoint, with the tree sum above it; random signs, the rest tiny."""
    big = np.float32(1024.0)
    f = np.float32(2.0 ** 20 / n)
    if f.view(np.uint32) & 1:                          # a tie rounds to f only when f is even
        f = np.nextafter(f, np.float32(1e30))
    mid = (np.float64(f) + np.float64(np.nextafter(f, np.float32(1e30)))) / 2
    target = mid * n                                   # exact: 25 + 14 significant bits
    x1 = _largest_root_below(target - 2.0 ** 20)
    s2 = np.float64(2.0 ** 20) + np.float64(x1) ** 2  # the chain after two adds (rounded, <= target)
    x2 = _largest_root_below(target - s2)
    x = np.full(n, TINY, np.float32)
    x[0], x[1], x[2] = big, x1, x2
    x *= np.where(rng.random(n) < 0.5, np.float32(-1), np.float32(1))
    return x
