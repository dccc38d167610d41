"""Host-side model of the decode kernel's exchange protocol (CPU).

The decode kernel has no grid barrier: workgroups exchange values through a workspace of
tagged words, and a consumer accepts a word when its tag equals the one it expects. The
protocol is sound if a consumer can never accept a word that a producer has not yet
rewritten for this use: the stale content of every word it polls must carry a different
tag. This model restates, per workspace region, which launches and layers write (or
clear) it, which read it and with which tag, and checks that property for every read
against every stale content that a sequence of launches of any kinds can leave behind:

* launch kinds: the two kernel instances (contexts up to 256 positions / longer), each
  with any attention split count, as full-model launches (28 layers) or single-block
  launches (1 layer), in any order and number;
* 16-bit tags: 1 + ((32 epoch + layer) mod 65535), in the high half of a bf16 word;
  32-bit tags: 32 epoch + layer + 1, beside an fp32 value;
* epochs are distinct per launch and increase (one counter per device).

The word-level coverage (each region's words written at each layer by the workgroups'
lanes) is checked from the kernel's index formulas, restated here.
"""

import itertools

import pytest

NWG, NXCD, WGX = 256, 8, 32
ROWS, UNITS, XUNITS = 32, 12, 384
L_FULL = 28
MAX_LAYERS = 32


def tag16(epoch, layer):
    return 1 + ((32 * epoch + layer) % 65535)


def tag32(epoch, layer_plus_one):
    return (32 * epoch + layer_plus_one) % (1 << 32)


# Region -> (tag kind, who writes it). "every": every launch writes it at every layer;
# "unsplit"/"split": only launches of that instance write it at every layer, the others
# clear it (tag 0) at their start; "chunks": chunk j is written at every layer by split
# launches with j < nsplit, and cleared at the start of every launch that does not write it.
REGIONS = {
    "LX_H": ("16", "every"), "LX_H1": ("16", "every"), "LX_QKV": ("16", "every"), "LX_M": ("16", "every"),
    "LX_ATT": ("16", "unsplit"),
    "LX_HSS": ("32", "every"), "LX_H1SS": ("32", "every"),
    "X_OPART": ("32", "every"), "X_DPART": ("32", "every"),
    "LX_PART": ("32", "chunks"),
}


def expected_tag(region, epoch, layer, L):
    """Tag a consumer polls for at `layer` (layer == L: the final-norm gather)."""
    kind = REGIONS[region][0]
    if region == "LX_H":  # gathered at layer l (> 0) from layer l - 1, and after the last layer
        return tag16(epoch, layer - 1)
    if region == "LX_HSS":
        return tag32(epoch, layer)
    return tag16(epoch, layer) if kind == "16" else tag32(epoch, layer + 1)


def written_tag(region, epoch, layer):
    kind = REGIONS[region][0]
    return tag16(epoch, layer) if kind == "16" else tag32(epoch, layer + 1)


def fresh_write_layer(region, layer):
    """The layer whose write a poll at `layer` waits for."""
    return layer - 1 if region in ("LX_H", "LX_HSS") else layer


def reads(region, L):
    """Layers at which a launch of L layers polls the region (L: the final-norm gather)."""
    if region in ("LX_H", "LX_HSS"):
        return range(1, L + 1)
    return range(L)


EPOCHS = (1, 2, 5, 2047, 2048, 2049, 65534, 65535, 65536, 55296 + 7, (1 << 27) - 1, 1 << 27, (1 << 27) + 3)


@pytest.mark.parametrize("region", sorted(REGIONS))
def test_no_stale_word_carries_the_polled_tag(region):
    """For every poll (epoch E, layer l) the content just before the awaited write never
    carries the polled tag. That content is the same launch's previous-layer write, or, for
    the launch's first write of the region, whatever the previous launch left: its last
    layer's write (it had 1..32 layers) or 0, since every launch writes or clears every
    region (epoch distance 1)."""
    for E in EPOCHS:
        for L in (1, L_FULL, MAX_LAYERS):
            for layer in reads(region, L):
                want = expected_tag(region, E, layer, L)
                assert want == written_tag(region, E, fresh_write_layer(region, layer))
                fl = fresh_write_layer(region, layer)
                if fl >= 1:
                    stale = {written_tag(region, E, fl - 1)}
                else:
                    stale = {0} | {written_tag(region, E - 1, Lp - 1) for Lp in range(1, MAX_LAYERS + 1)}
                assert want not in stale, (region, E, L, layer)


def _alias_distance_if_not_cleared(region, l_read, l_prev):
    """Smallest epoch distance d >= 1 at which a word last written at layer l_prev of an
    earlier launch would carry the tag polled at layer l_read: the distance the clears
    rule out (without them, a run of d - 1 launches that skip the region would expose it)."""
    kind = REGIONS[region][0]
    if kind == "16":
        # 32 E' + l_prev == 32 E + l_read (mod 65535): 32 d == l_prev - l_read, and
        # 32^-1 = 2048 (mod 65535)
        return ((l_prev - l_read) * 2048) % 65535 or 65535
    if l_read != l_prev:
        return None
    return 1 << 27


def test_clears_are_needed_for_the_regions_only_some_launches_write():
    """Without the clears, LX_ATT (written by unsplit launches only) would alias after
    55296 launches that skip it, and LX_PART after 2^27: the model shows why a launch that
    does not write those regions clears them."""
    assert _alias_distance_if_not_cleared("LX_ATT", 0, 27) == 55296
    assert tag16(100, 27) == tag16(100 + 55296, 0)
    assert _alias_distance_if_not_cleared("LX_PART", 5, 5) == 1 << 27
    assert tag32(100, 6) == tag32(100 + (1 << 27), 6)


# ---------------------------------------------------------------- word coverage

def _qkv_words():
    return {16 * j + lane for j in range(WGX) for lane in range(16)}


def _rows_words():  # LX_H / LX_H1: reduce wave of workgroup j, lanes with hx == 0 -> row lane >> 1
    return {ROWS * j + (lane >> 1) for j in range(WGX) for lane in range(64) if (lane & 1) == 0}


def _m_words():
    return {UNITS * j + lane for j in range(WGX) for lane in range(UNITS)}


def _att_words():  # store wave: lane -> 4 words at hh * 128 + 4 (lane & 31)
    return {(lane >> 5) * 128 + 4 * (lane & 31) + e for lane in range(64) for e in range(4)}


def _ss_words():  # one (sum, tag) pair per workgroup j
    return {2 * j for j in range(WGX)}


def _part_words(nsplit):
    """Per chunk j < nsplit and head: (m, l) pair and 128 accumulator pairs, 2 words each."""
    words = set()
    for j in range(nsplit):
        for hh in range(2):
            base = 2 * ((j * 2 + hh) * 130)
            words |= {base + w for w in range(4)}  # m, tag, l, tag
            for lane in range(64):
                if lane >> 5 != hh:
                    continue
                dim = 4 * (lane & 31)
                words |= {base + 2 * (2 + dim) + w for w in range(8)}  # pairs dim, dim + 1, dim + 2, dim + 3
    return words


def test_every_polled_word_is_written_at_every_layer():
    assert _qkv_words() == set(range(512))
    assert _rows_words() == set(range(1024))
    assert _m_words() == set(range(XUNITS))
    assert _att_words() == set(range(256))
    assert _ss_words() == {2 * j for j in range(WGX)}
    for nsplit in (1, 2, 9, 32):
        words = _part_words(nsplit)
        # the merge polls, for each chunk j < nsplit and head, (m, l) and accumulator pairs
        # of dims d0, d0 + 1 for every d0 = 2 t, t < 64
        for j, hh in itertools.product(range(nsplit), range(2)):
            base = 2 * ((j * 2 + hh) * 130)
            assert {base, base + 1, base + 2, base + 3} <= words
            for t in range(64):
                d0 = 2 * t
                assert {base + 4 + 2 * d0 + w for w in range(4)} <= words


def test_cross_xcd_partials_cover_every_row():
    """X_OPART / X_DPART: workgroup (g, j) stores lane < 32 at [j][row lane][xcd g]; the reduce
    wave of (g', j) polls [j][row rr][xcd 4 hx .. 4 hx + 3] for rr < 32, hx < 2."""
    written = {(j, r, g) for g in range(NXCD) for j in range(WGX) for r in range(ROWS)}
    polled = {(j, lane >> 1, 4 * (lane & 1) + x) for j in range(WGX) for lane in range(64) for x in range(4)}
    assert polled == written
