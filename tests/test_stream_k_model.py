"""CPU model of conv2d_direct's split of (tile, k-tile) units over sharing
workgroups (lancius_amd/csrc/conv.hip, the stream-K loop of conv2d_direct
and the host's choice of sharers in launch()).  The kernel is correct only
if every sharing workgroup gets a nonempty range, a range holds at most two
partial tiles, its first and its last (it has two partial-sum slots; a
whole tile inside the range is stored directly), and the arrivals at each
partial tile's counter equal the number of workgroups that own a unit of
that tile (the last arrival finishes the tile).  Checked here for the small-grid split
(every workgroup shares) and the tail split ((n - 1) x CUs whole tiles, one
sharer per CU), at the shapes the GPU tests and the bench run."""
import pytest

CUS = 256


def split(tiles, ktiles, S):
    """(per-tile arrival counts, per-tile owner spans, most partial tiles in
    one range).  A partial tile anywhere but first or last fails here."""
    U = tiles * ktiles

    def owner(v):
        return ((v + 1) * S - 1) // U

    arrivals, widest = {}, 0
    for s in range(S):
        u, uend = s * U // S, (s + 1) * U // S
        assert uend > u, f"workgroup {s} has no units"
        t_rel = u // ktiles
        kbeg = u - t_rel * ktiles
        kend = min(ktiles, uend - t_rel * ktiles)
        u = t_rel * ktiles + kend
        partial, first = 0, True
        while True:
            if kbeg != 0 or kend != ktiles:
                assert first or u >= uend, f"workgroup {s}: a partial tile inside its range"
                partial += 1
                arrivals[t_rel] = arrivals.get(t_rel, 0) + 1
            if u >= uend:
                break
            first = False
            t_rel = u // ktiles
            kbeg, kend = 0, min(ktiles, uend - t_rel * ktiles)
            u = t_rel * ktiles + kend
        widest = max(widest, partial)
    spans = {t: owner((t + 1) * ktiles - 1) - owner(t * ktiles) + 1 for t in arrivals}
    return arrivals, spans, widest


def small_grid_sharers(tiles, ktiles):
    """The host's choice for grids under half the CUs, or None."""
    sk = min(CUS, tiles * min(8, max(1, ktiles // 18)))
    units = tiles * ktiles
    return sk if sk >= 2 * tiles and units >= 4 * sk else None


# (tiles, k-tiles): the variant tests' small grids, a long-K single tile,
# and shapes at the edges of the rule
SMALL = [(49, 36), (26, 72), (16, 144), (9, 45), (1, 1024), (10, 103), (98, 36), (127, 9), (64, 16)]


@pytest.mark.parametrize("tiles,ktiles", SMALL)
def test_small_grid_split(tiles, ktiles):
    S = small_grid_sharers(tiles, ktiles)
    if S is None:
        pytest.skip("the host keeps whole tiles for this grid")
    arrivals, spans, widest = split(tiles, ktiles, S)
    assert widest <= 2
    assert arrivals == spans
    assert max(arrivals.values()) <= 9  # a tile split at most 8 ways (9 with a boundary share)


@pytest.mark.parametrize("tiles,ktiles", [(1568, 36), (294, 9), (282, 18), (1568 + 64, 36)])
def test_tail_split(tiles, ktiles):
    per, rem = tiles // CUS, tiles % CUS
    if not (per >= 1 and rem != 0 and rem <= CUS // 4):
        pytest.skip("no tail split")
    rest = tiles - (per - 1) * CUS
    arrivals, spans, widest = split(rest, ktiles, CUS)
    assert widest <= 2
    assert arrivals == spans
