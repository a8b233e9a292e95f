"""An independent, exact-integer statement of the reference's window rule
(src/layers/seedvr2_dit_block.cpp:827-868), used by the tests to pin the
oracle's and the library's window plans.

The reference computes in double with truncating casts; here every quantity
is an exact integer or rational:
  * adaptive extents: the nearest integer to sqrt(3600 H / W) (ties to even)
    is found by comparing squares of half-integers exactly, instead of
    nearbyint(H * sqrt(3600 / (H W)));
  * a shifted axis (shift 1/2, only when the window is smaller than the
    extent) has ceil((2D - 1) / 2w) + 1 intervals with bounds
    trunc((2i - 1) w / 2) and trunc((2i + 1) w / 2), clamped to [0, D];
  * windows are kept in w -> h -> t loop order, empty ones dropped.
"""
from __future__ import annotations


def _trunc_div(a: int, b: int) -> int:
    q = abs(a) // b
    return q if a >= 0 else -q


def _round_sqrt_ratio(num: int, den: int) -> int:
    """round-half-even of sqrt(num / den) for positive integers, exactly."""
    n = 0
    # smallest n with (n + 1/2)^2 >= num/den  <=>  (2n + 1)^2 den >= 4 num
    while (2 * n + 1) ** 2 * den < 4 * num:
        n += 1
    if (2 * n + 1) ** 2 * den == 4 * num and n % 2 == 1:
        n += 1  # exact tie between n and n + 1: the even one
    return n


def adaptive(T: int, H: int, W: int) -> tuple[int, int, int]:
    rh = _round_sqrt_ratio(3600 * H, W)   # H * sqrt(3600 / (H W)) = sqrt(3600 H / W)
    rw = _round_sqrt_ratio(3600 * W, H)
    return (-(-min(T, 30) // 4), -(-rh // 3), -(-rw // 3))


def axis(D: int, w: int, shifted: bool) -> list[tuple[int, int]]:
    if shifted and w < D:
        count = -(-(2 * D - 1) // (2 * w)) + 1
        return [(max(_trunc_div((2 * i - 1) * w, 2), 0), min(_trunc_div((2 * i + 1) * w, 2), D))
                for i in range(count)]
    count = 1 if shifted else -(-D // w)
    return [(i * w, min((i + 1) * w, D)) for i in range(count)]


def plan(T: int, H: int, W: int, shifted: bool, wt: int = 0, wh: int = 0, ww: int = 0):
    at, ah, aw = adaptive(T, H, W)
    wt, wh, ww = wt or at, wh or ah, ww or aw
    out = []
    for (w0, w1) in axis(W, ww, shifted):
        for (h0, h1) in axis(H, wh, shifted):
            for (t0, t1) in axis(T, wt, shifted):
                if t1 > t0 and h1 > h0 and w1 > w0:
                    out.append((t0, t1, h0, h1, w0, w1))
    return out


def index_map(T: int, H: int, W: int, windows) -> list[int]:
    return [(t * H + y) * W + x for (t0, t1, h0, h1, w0, w1) in windows
            for t in range(t0, t1) for y in range(h0, h1) for x in range(w0, w1)]
