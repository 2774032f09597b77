"""The decode split's integer arithmetic, restated from the two kernels that
must agree on it, checked for consistency on random and edge-case batches.

decode_page_kernel (vllm-cpp_amd/csrc/decode.hip) gives range w the real
tiles [real_of(range_start(w, Tv, G)), real_of(range_start(w + 1, Tv, G))),
where the split axis puts X units before each non-empty sequence's tiles
(Tv = T + X K).  merge_split_kernel maps a sequence's first and last tiles to
ranges with range_of(t + X (k + 1), Tv, G).  If the two disagreed, a partial
would be written to one range's slot and read from another's; these checks
pin that they cannot."""
import numpy as np
import pytest


def range_start(w, T, G):
    return (w * T) // G


def range_of(t, T, G):
    return ((t + 1) * G - 1) // T


def range_live(w, T, G):
    return T >= G or range_start(w, T, G) < range_start(w + 1, T, G)


def axis(tiles, X):
    """Real prefix S, non-empty count before each sequence k, totals."""
    S = np.concatenate([[0], np.cumsum(tiles)])[:-1]
    k = np.concatenate([[0], np.cumsum(tiles > 0)])[:-1]
    return S, k, int(tiles.sum()), int((tiles > 0).sum())


def real_of(V, tiles, X):
    """decode_page_kernel's real_of: first real tile at or past virtual V."""
    S, k, T, K = axis(tiles, X)
    Tv = T + X * K
    if X == 0 or V <= 0:
        return max(V, 0)
    if V >= Tv:
        return T
    for s in range(len(tiles)):
        nt = int(tiles[s])
        vfirst = int(S[s]) + X * (int(k[s]) + 1)
        if nt > 0 and vfirst - X <= V < vfirst + nt:
            return max(int(S[s]), V - X * (int(k[s]) + 1))
    return T


def ranges(tiles, X, G):
    S, k, T, K = axis(tiles, X)
    Tv = T + X * K
    return [(real_of(range_start(w, Tv, G), tiles, X), real_of(range_start(w + 1, Tv, G), tiles, X))
            for w in range(G)], T, Tv


def check(tiles, X, G):
    tiles = np.asarray(tiles, dtype=np.int64)
    rs, T, Tv = ranges(tiles, X, G)
    # contiguous, in order, covering [0, T) (ranges may be empty when Tv < G)
    assert rs[0][0] == 0 and rs[-1][1] == T
    for (a0, b0), (a1, b1) in zip(rs, rs[1:]):
        assert a0 <= b0 == a1 <= b1
    owner = np.empty(T, dtype=np.int64)
    for w, (a, b) in enumerate(rs):
        owner[a:b] = w
    # the merge kernel's view of every sequence's first and last tiles
    S, k, _, _ = axis(tiles, X)
    for s, nt in enumerate(tiles):
        if nt == 0:
            continue
        shift = X * (int(k[s]) + 1)
        first, last = int(S[s]), int(S[s]) + int(nt) - 1
        assert range_of(first + shift, Tv, G) == owner[first]
        assert range_of(last + shift, Tv, G) == owner[last]
        # the merge reads the ranges between that range_live calls live: those
        # hold tiles of s, the others hold none
        for w in range(owner[first], owner[last] + 1):
            a, b = rs[w]
            if range_live(w, Tv, G):
                assert a < b and a <= last and b > first
            else:
                assert a == b


@pytest.mark.parametrize("X", [0, 1, 2, 4, 7])
def test_split_random_batches(X):
    rng = np.random.default_rng(1234 + X)
    for _ in range(60):
        n = int(rng.integers(1, 200))
        tiles = rng.integers(0, 300, n)
        tiles[rng.random(n) < 0.2] = 0  # empty sequences
        G = int(rng.choice([1, 3, 64, 256, 512]))
        if tiles.sum() == 0:
            tiles[0] = 1
        check(tiles, X, G)


@pytest.mark.parametrize("X", [0, 2])
def test_split_edge_cases(X):
    check([1], X, 256)                      # far fewer tiles than ranges
    check([0, 0, 5, 0], X, 7)               # empty sequences around one short one
    check([256] * 64, X, 256)               # BASELINE config 2's shape class
    check([2048] * 16, X, 256)              # config 4's shape class
    check([1] * 1000, X, 256)               # many one-tile sequences
    check([3000, 1, 1, 1, 4096], X, 512)    # long ones around short ones


def span_start(w, T, G, WG):
    """decode_page_kernel with fixed partitions: workgroup w of WG walks the
    ranges [range_start(w, G, WG), range_start(w + 1, G, WG)) of the G-range
    split of T tiles (no switch units)."""
    return range_start(range_start(w, G, WG), T, G)


def span_of(t, T, G, WG):
    """merge_split_kernel's Spans::span_of."""
    r = range_of(t, T, G)
    return r if WG == G else range_of(r, G, WG)


def span_live(w, T, G, WG):
    return T >= G or span_start(w, T, G, WG) < span_start(w + 1, T, G, WG)


@pytest.mark.parametrize("seed", range(8))
def test_partition_spans(seed):
    """Fixed partitions on the page kernel: every tile's workgroup as the
    merge computes it is the workgroup whose span holds the tile, and the
    spans the merge treats as live are exactly the non-empty ones."""
    rng = np.random.default_rng(99 + seed)
    for _ in range(40):
        T = int(rng.integers(1, 40000))
        G = int(rng.integers(1, 4096))
        WG = int(min(G, rng.choice([1, 7, 256, 512, G])))
        starts = [span_start(w, T, G, WG) for w in range(WG + 1)]
        assert starts[0] == 0 and starts[-1] == T
        assert all(a <= b for a, b in zip(starts, starts[1:]))
        for t in list(rng.integers(0, T, 50)) + [0, T - 1]:
            w = span_of(int(t), T, G, WG)
            assert starts[w] <= t < starts[w + 1]
        for w in range(WG):
            assert span_live(w, T, G, WG) == (starts[w] < starts[w + 1])


def test_partition_spans_config4():
    """Config 4 at 256-token partitions on 256 workgroups: 2048 partitions of
    16 tiles, 8 per workgroup, every workgroup span inside one sequence."""
    T, G, WG = 16 * 2048, 16 * 2048 // 16, 256
    for w in range(WG):
        a, b = span_start(w, T, G, WG), span_start(w + 1, T, G, WG)
        assert b - a == 128 and a // 2048 == (b - 1) // 2048


class Alternating:
    """Split in decode.hip with alternating range sizes (byte pages at two
    workgroups per CU): position 2k takes share / 256 of each pair's units,
    2k + 1 the rest; start(r) = Tv cum(r) / (128 G), cum(r) = 256 (r / 2) +
    share (r % 2).  rof is the kernel's inverse (an estimate, then steps)."""

    def __init__(self, Tv, G, share):
        self.Tv, self.G, self.share = Tv, G, share

    def rstart(self, r):
        cum = (r >> 1) * 256 + (r & 1) * self.share
        return (self.Tv * cum) // (self.G * 128)

    def rof(self, t):
        u = (t * self.G * 128) // self.Tv
        r = (u >> 8) * 2 + (1 if (u & 255) >= self.share else 0)
        while r + 1 < self.G and self.rstart(r + 1) <= t:
            r += 1
        while r > 0 and self.rstart(r) > t:
            r -= 1
        return r

    def all_live(self):
        return self.Tv * min(self.share, 256 - self.share) >= self.G * 128


def position(bx, WG):
    """The axis position of workgroup bx: the first dispatch round (ids
    below WG / 2) takes the even positions, the second the odd ones."""
    return 2 * bx if bx < WG // 2 else 2 * (bx - WG // 2) + 1


@pytest.mark.parametrize("share", [100, 128, 152, 164, 176, 220])
def test_alternating_split(share):
    """rof(t) is the range whose [start, next start) holds t, for every unit
    of random and edge-case axes; all_live implies no empty range; the
    workgroup-to-position map is a bijection that gives the last position to
    the last workgroup (the owner of trailing empty sequences)."""
    rng = np.random.default_rng(share)
    cases = [(1, 2), (7, 512), (511, 512), (512, 512), (40000, 512), (16, 8)]
    cases += [(int(rng.integers(1, 60000)), int(rng.choice([2, 8, 256, 512, 1024]))) for _ in range(30)]
    for Tv, G in cases:
        sp = Alternating(Tv, G, share)
        starts = [sp.rstart(r) for r in range(G + 1)]
        assert starts[0] == 0 and starts[-1] == Tv
        assert all(a <= b for a, b in zip(starts, starts[1:]))
        ts = range(Tv) if Tv <= 3000 else list(rng.integers(0, Tv, 3000)) + [0, Tv - 1]
        for t in ts:
            r = sp.rof(int(t))
            assert starts[r] <= t < starts[r + 1]
        if sp.all_live():
            assert all(a < b for a, b in zip(starts, starts[1:]))
        pos = [position(b, G) for b in range(G)]
        assert sorted(pos) == list(range(G)) and pos[G - 1] == G - 1 and pos[0] == 0
