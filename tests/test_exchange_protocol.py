"""Host-side model of the decode kernel's exchange protocol (CPU).

The decode kernel has no grid barrier: workgroups exchange values through a workspace of
tagged words, and a consumer accepts a word when its tag equals the one it expects. The
protocol is sound if a consumer can never accept a word that a producer has not yet
rewritten for this use: the stale content of every word it polls must carry a different
tag. This model restates, per workspace region, which launches and layers write (or
clear) it, which read it and with which tag, and checks that property for every read
against every stale content that a sequence of launches of any kinds can leave behind:

* launch kinds: the two kernel instances (contexts up to 256 positions / longer; the
  longer one's variant with pipelined LDS passes exchanges the same words), each with
  any attention split count, as full-model launches (28 layers) or single-block
  launches (1 layer), in any order and number;
* 16-bit tags: 1 + ((32 epoch + layer) mod 65535), in the high half of a bf16 word;
  32-bit tags: 32 epoch + layer + 1, beside an fp32 value;
* epochs: a launch takes the epoch its workspace holds plus one, and its last workgroup
  stores that epoch back (launches on one stream run one after another), so consecutive
  launches on one workspace differ by exactly one epoch. Two workspaces exist: the
  allocated one (host-driven and device-resident launches) and the no-allocation entry
  point's; launches on the two interleave in any order.

The word-level coverage (each region's words written at each layer by the workgroups'
lanes) is checked from the kernel's index formulas, restated here.
"""

import itertools

import pytest

NWG, NXCD, WGX = 256, 8, 32
NGA = NGB = 16          # group-A and group-B workgroups per XCD
ROWS, QROWS = 64, 32    # residual rows a workgroup reduces; q/k/v rows of an A workgroup
UNITS, XUNITS = 24, 384  # MLP units of a B workgroup; of an XCD
MAX_CHUNKS = 16
L_FULL = 28
MAX_LAYERS = 32


def tag16(epoch, layer):
    return 1 + ((32 * epoch + layer) % 65535)


def tag32(epoch, layer_plus_one):
    return (32 * epoch + layer_plus_one) % (1 << 32)


# Region -> (tag kind, who writes it). "every": every launch writes it at every layer;
# "split1": only split launches with one attention chunk write it at every layer (the other
# group-A workgroups read it there), every other launch clears it (tag 0) at its start; "chunks": chunk j is written at every layer by split
# launches with j < nsplit, and cleared at the start of every launch that does not write it.
# LX_H and LX_CUE_B are written by group B (h and its cue), LX_QKV, LX_ATT, LX_PART and
# LX_CUE_A by group A, LX_M by group B; LX_H1 by the reduce waves of group A, or of group B
# in unsplit launches of 129 or more positions (the same rows, member m's 64, either way);
# the cross-XCD arrays by both.
REGIONS = {
    "LX_H": ("16", "every"), "LX_H1": ("16", "every"), "LX_QKV": ("16", "every"), "LX_M": ("16", "every"),
    "LX_CUE_A": ("16", "every"), "LX_CUE_B": ("16", "every"),
    "LX_ATT": ("16", "split1"),
    "X_OPART": ("32", "every"), "X_DPART": ("32", "every"),
    "LX_PART": ("32", "chunks"),
}
# regions gathered at layer l from the previous layer's write (and after the last layer)
FROM_PREVIOUS_LAYER = ("LX_H", "LX_CUE_B")


def expected_tag(region, epoch, layer, L):
    """Tag a consumer polls for at `layer` (layer == L: the final-norm gather)."""
    kind = REGIONS[region][0]
    if region in FROM_PREVIOUS_LAYER:
        return tag16(epoch, layer - 1)
    return tag16(epoch, layer) if kind == "16" else tag32(epoch, layer + 1)


def written_tag(region, epoch, layer):
    kind = REGIONS[region][0]
    return tag16(epoch, layer) if kind == "16" else tag32(epoch, layer + 1)


def fresh_write_layer(region, layer):
    """The layer whose write a poll at `layer` waits for."""
    return layer - 1 if region in FROM_PREVIOUS_LAYER else layer


def reads(region, L):
    """Layers at which a launch of L layers polls the region (L: the final-norm gather)."""
    if region in FROM_PREVIOUS_LAYER:
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
    """Without the clears, LX_ATT (written by one-chunk split launches only) would alias after
    55296 launches that skip it, and LX_PART after 2^27: the model shows why a launch that
    does not write those regions clears them."""
    assert _alias_distance_if_not_cleared("LX_ATT", 0, 27) == 55296
    assert tag16(100, 27) == tag16(100 + 55296, 0)
    assert _alias_distance_if_not_cleared("LX_PART", 5, 5) == 1 << 27
    assert tag32(100, 6) == tag32(100 + (1 << 27), 6)


# ---------------------------------------------------------------- word coverage

def _qkv_words():
    """Stream wave s of A workgroup a: lanes 16 q (q < 4) hold rows 2 q, 2 q + 1 of the wave's
    8 and store them as one pair at word 32 a + 8 s + 2 q."""
    return {QROWS * a + 8 * s + 2 * q + e for a in range(NGA) for s in range(4) for q in range(4) for e in range(2)}


def _rows_words():  # LX_H (B) / LX_H1 (A): reduce wave of member m, lane -> row 64 m + lane
    return {ROWS * m + lane for m in range(NGA) for lane in range(64)}


def _m_words():
    """Stream wave s of B workgroup b: lanes < 6 store the wave's 6 units at word 24 b + 6 s + lane."""
    return {UNITS * b + 6 * s + lane for b in range(NGB) for s in range(4) for lane in range(6)}


def _att_words():  # store wave: lane -> 4 words at hh * 128 + 4 (lane & 31)
    return {(lane >> 5) * 128 + 4 * (lane & 31) + e for lane in range(64) for e in range(4)}


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


def _gather_half_words(c):
    """Poll wave c of the residual-stream gather: chunks lane + 128 c and lane + 128 c + 64
    (4 tagged words each)."""
    return {4 * (ch) + e for lane in range(64) for ch in (lane + 128 * c, lane + 128 * c + 64) for e in range(4)}


def test_every_polled_word_is_written_at_every_layer():
    assert _qkv_words() == set(range(512))
    assert _rows_words() == set(range(1024))
    assert _m_words() == set(range(XUNITS))
    assert _att_words() == set(range(256))
    # the two poll waves' halves of a gather are disjoint and cover the 1024 rows
    assert _gather_half_words(0) | _gather_half_words(1) == set(range(1024))
    assert not _gather_half_words(0) & _gather_half_words(1)
    # the m gather: poll thread q < 96 loads words 4q .. 4q + 3
    assert {4 * q + e for q in range(XUNITS // 4) for e in range(4)} == _m_words()
    for nsplit in (1, 2, 9, MAX_CHUNKS):
        words = _part_words(nsplit)
        # the merge polls, for each chunk j < nsplit and head, (m, l) and accumulator pairs
        # of dims d0, d0 + 1 for every d0 = 2 t, t < 64
        for j, hh in itertools.product(range(nsplit), range(2)):
            base = 2 * ((j * 2 + hh) * 130)
            assert {base, base + 1, base + 2, base + 3} <= words
            for t in range(64):
                d0 = 2 * t
                assert {base + 4 + 2 * d0 + w for w in range(4)} <= words
    # the chunk records fit the XCD's region: LX_PART (4096) + 16 chunks x 2 heads x 130 pairs
    assert 4096 + 2 * MAX_CHUNKS * 2 * 130 <= 32768


def test_cross_xcd_partials_cover_every_row():
    """X_OPART / X_DPART ([member][xcd][row] pairs): stream wave s of workgroup (g, m) stores
    lane < 16 at [m][g][16 s + lane] (one contiguous 128-byte run per wave); the reduce wave
    of (g', m) polls [m][x][lane] for every XCD x, lane < 64, one 8-byte pair per load."""
    written = {(m, g, 16 * s + lane) for g in range(NXCD) for m in range(NGA) for s in range(4) for lane in range(16)}
    assert len(written) == NXCD * NGA * ROWS
    polled = {(m, x, lane) for m in range(NGA) for x in range(NXCD) for lane in range(64)}
    assert polled == written
    # word offsets: producer 2 ((m 8 + g) 64 + lane), consumer 2 (m 8 64 + lane) + 2 64 x
    for m, g, lane in itertools.product(range(NGA), range(NXCD), range(64)):
        assert 2 * ((m * NXCD + g) * ROWS + lane) == 2 * (m * NXCD * ROWS + lane) + 2 * ROWS * g
    # both arrays fit between the per-XCD regions and the LM-head partials
    assert 2 * NGA * ROWS * NXCD + 2 * NGB * ROWS * NXCD == 32768


# ---------------------------------------------------------------- epochs across workspaces

def _launch_polls_ok(region, E, L, prev):
    """Every poll of a launch (epoch E, L layers) finds no stale word with the polled tag;
    `prev` = (epoch, layers) of the previous launch on the same workspace, or None (the
    workspace is zero)."""
    for layer in reads(region, L):
        want = expected_tag(region, E, layer, L)
        fl = fresh_write_layer(region, layer)
        if fl >= 1:
            stale = {written_tag(region, E, fl - 1)}
        else:
            stale = {0}
            if prev is not None:
                stale.add(written_tag(region, prev[0], prev[1] - 1))
        if want in stale:
            return False
    return True


def _run(sequence, epoch_of, only=None):
    """Simulate launches [(workspace, layers)]: epoch_of(state, ws) gives a launch's epoch and
    advances the state. Returns the first (index, region) whose poll could accept a stale
    word, or None (only: check the launches on that workspace alone)."""
    state = {"ws": {}, "counter": 0}
    last = {}
    for i, (ws, L) in enumerate(sequence):
        E = epoch_of(state, ws)
        for region in REGIONS if only in (None, ws) else ():
            if not _launch_polls_ok(region, E, L, last.get(ws)):
                return i, region
        last[ws] = (E, L)
    return None


def _per_workspace_epoch(state, ws):  # the kernel's rule: the workspace's stored epoch + 1
    E = state["ws"].get(ws, 0) + 1
    state["ws"][ws] = E
    return E


def _shared_host_counter(state, ws):  # the earlier rule: one host counter per device
    state["counter"] += 1
    return state["counter"]


def test_interleaved_workspaces_never_alias():
    """Launches on the allocated and the no-allocation workspace in any interleaving, of 1, 2,
    28 or 32 layers: with per-workspace epochs no poll can accept a stale word, including
    after runs of 2047 and 55295 launches on the other workspace (the distances at which
    a shared counter aliases, below)."""
    import random

    rng = random.Random(7)
    for trial in range(40):
        seq = [(rng.choice("an"), rng.choice((1, 2, 28, 32))) for _ in range(rng.randint(2, 60))]
        assert _run(seq, _per_workspace_epoch) is None, seq
    for gap in (2047, 55295):
        for Lp in (2, 28):
            seq = [("n", Lp)] + [("a", 28)] * gap + [("n", 28)]
            assert _run(seq, _per_workspace_epoch, only="n") is None


def test_a_shared_epoch_counter_would_alias():
    """Why epochs are per workspace: with one counter for both workspaces, a no-allocation
    launch d epochs after the previous one on its workspace polls its first layer for the
    tag that launch's last layer (L' layers) left when 32 d == L' - 1 (mod 65535), i.e.
    d == 2048 (L' - 1): 2048 after a 2-layer launch, 55296 after a 28-layer one."""
    for Lp in (2, 28):
        d = (2048 * (Lp - 1)) % 65535
        assert tag16(100, Lp - 1) == tag16(100 + d, 0)
        seq = [("n", Lp)] + [("a", 28)] * (d - 1) + [("n", 28)]
        hit = _run(seq, _shared_host_counter, only="n")
        assert hit is not None and hit[0] == len(seq) - 1, hit
        assert _run(seq, _per_workspace_epoch, only="n") is None
