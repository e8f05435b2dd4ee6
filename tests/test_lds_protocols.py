"""CPU checks of the attention kernel's LDS layouts and barrier protocol
(wan2-ti2v-5b_amd/csrc/flash_fwd.hip), as properties of its index maps:

* the 1 KB row-staging copies (`stage_rows32`) and the output staging write every LDS
  position of their region exactly once, and each reader finds the chunk it wants
  there; every address stays inside the region;
* the 8-wave ring of four K and four V tiles with a barrier after every second step:
  for every tile count, each operand read sees its tile landed and published by an
  earlier barrier, no copy overwrites a buffer that a slower wave may still read, the
  output staging (which reuses K buffers 0 and 1) starts only after every K read, and
  a planted mistake in the protocol is caught.

No kernel runs here; the GPU tests check the numbers the kernel produces.
"""
import pytest


# ---------------------------------------------------------------------------
# layouts
# ---------------------------------------------------------------------------

def test_row_staging_layout():
    """stage_rows32: copy i, lane l -> row 4i + l/16, position l%16 holding chunk
    (l%16) ^ (row & 15); reader of chunk c of row r looks at position c ^ (r & 15)."""
    written = {}
    for i in range(8):
        for lane in range(64):
            rr = 4 * i + (lane >> 4)
            c = (lane & 15) ^ (rr & 15)
            off = i * 1024 + lane * 16
            assert off not in written
            written[off] = (rr, c)
    assert sorted(written) == list(range(0, 8192, 16))
    for r in range(32):
        for c in range(16):
            assert written[r * 256 + ((c ^ (r & 15)) << 4)] == (r, c)
    # the 16 rows a half-wave reads for one chunk fall on 16 distinct 16-byte slots mod 256 B
    for c in range(16):
        assert len({(r * 256 + ((c ^ (r & 15)) << 4)) % 256 for r in range(16)}) == 16


def test_output_staging_layout():
    """Output staging: lane (n32, hh) writes 8 B of row n32 at channel 32 mm + 8 g + 4 hh of
    each 64-channel half; readers take 16 B (row 8j + l/8, chunk l%8) for the store."""
    for half in range(2):
        lds = {}
        for lane in range(64):
            n32, hh = lane & 31, lane >> 5
            for mm in range(2):
                for g in range(4):
                    for e in range(4):
                        ch = 32 * (2 * half + mm) + 8 * g + 4 * hh + e
                        c = 4 * mm + g
                        addr = n32 * 64 + ((c ^ (n32 & 7)) << 3) + 4 * hh + e
                        assert 0 <= addr < 2048 and addr not in lds
                        lds[addr] = (n32, ch)
        assert len(lds) == 2048
        for j in range(4):
            for lane in range(64):
                r, c = 8 * j + (lane >> 3), lane & 7
                for e in range(8):
                    assert lds[r * 64 + ((c ^ (r & 7)) << 3) + e] == (r, 64 * half + 8 * c + e)
    for wave in range(8):   # waves 0-3 use K buffer 0, 4-7 buffer 1, 4 KB each
        assert (wave & 3) * 2048 + 2047 < 8192


def test_rope_staging_regions_disjoint():
    """8 waves with RoPE: cos rows in K buffers 1-3 and the extra 32 KB, sin rows in V
    buffers 1-3 and the extra 32 KB, 8 KB per wave, none touching K0 / V0 (copied
    meanwhile)."""
    tile = 16384   # bytes per K or V tile
    regions = []
    for wave in range(8):
        if wave < 6:
            cos = ("k", (1 + wave // 2) * tile + (wave & 1) * 8192)
            sin = ("v", (1 + wave // 2) * tile + (wave & 1) * 8192)
        else:
            cos = ("x", (wave - 6) * 8192)
            sin = ("x", 16384 + (wave - 6) * 8192)
        regions += [cos, sin]
    spans = {}
    for buf, start in regions:
        for b in range(start, start + 8192, 1024):
            assert (buf, b) not in spans
            spans[(buf, b)] = True
        if buf in "kv":
            assert start >= tile and start + 8192 <= 4 * tile   # not tile 0, inside the ring
        else:
            assert start + 8192 <= 32768                        # inside the extra 32 KB


# ---------------------------------------------------------------------------
# the ring-of-four protocol
# ---------------------------------------------------------------------------

def _ring4_ops(n, *, drop_epilogue_barrier=False, v_ring_of_two=False, no_wait_on_odd=False):
    """The per-wave sequence of the 8-wave kernel for n tiles: tile copies, waits, operand
    reads, barriers (every wave runs the same sequence; any may run ahead to the next
    barrier)."""
    ops = []
    K = lambda t: ("k", t % 4)
    V = lambda t: ("v", t % (2 if v_ring_of_two else 4))
    # prologue (RoPE path): K0, V0; staging; barrier; K1, V1, K2; S(0); wait; barrier
    ops += [("issue", K(0), ("K", 0)), ("issue", V(0), ("V", 0)), ("wait",), ("bar",)]
    if n > 1:
        ops += [("issue", K(1), ("K", 1)), ("issue", V(1), ("V", 1))]
    if n > 2:
        ops += [("issue", K(2), ("K", 2))]
    ops += [("read", K(0), ("K", 0)), ("wait",), ("bar",)]

    def step(t):
        ops.append(("read", K(t + 1), ("K", t + 1)))     # S(t+1) and the softmax of tile t
        if t % 2 == 0:
            for tile in (t + 3, t + 4):
                if tile < n:
                    ops.append(("issue", K(tile), ("K", tile)))
            for tile in (t + 2, t + 3):
                if tile < n:
                    ops.append(("issue", V(tile), ("V", tile)))
        ops.append(("read", V(t), ("V", t)))             # PV of tile t
        if t % 2 == 1:
            ops.extend(([] if no_wait_on_odd else [("wait",)]) + [("bar",)])

    t = 0
    while t + 4 < n:
        for i in range(4):
            step(t + i)
        t += 4
    while t + 1 < n:
        step(t)
        t += 1
    ops.append(("read", V(t), ("V", n - 1)))
    if not drop_epilogue_barrier:
        ops.append(("bar",))
    ops.append(("epilogue",))
    return ops


def _check_protocol(n, **mistakes):
    phase, pending, issues, reads, epi = 0, [], [], [], None
    for op in _ring4_ops(n, **mistakes):
        if op[0] == "bar":
            phase += 1
        elif op[0] == "issue":
            pending.append(len(issues))
            issues.append({"buf": op[1], "tile": op[2], "phase": phase, "visible": None})
        elif op[0] == "wait":
            for i in pending:
                issues[i]["visible"] = phase + 1   # published by the next barrier
            pending = []
        elif op[0] == "read":
            reads.append((op[1], op[2], phase))
        else:
            epi = phase
    assert not pending, "a copy is never waited for"
    for buf, tile, ph in reads:
        src = [i for i in issues if i["buf"] == buf and i["tile"] == tile]
        assert len(src) == 1, f"{tile} is not copied into {buf} exactly once"
        assert src[0]["visible"] is not None and src[0]["visible"] <= ph, f"{tile} read before published"
        for other in issues:   # a later copy into the same buffer comes after the barrier
            if other["buf"] == buf and other["tile"] != tile and other["phase"] >= src[0]["phase"]:
                assert other["phase"] > ph, f"{other['tile']} may overwrite {tile} while it is read"
    for buf, tile, ph in reads:
        if buf[0] == "k" and buf[1] in (0, 1):
            assert ph < epi, "the output staging may overwrite a K tile still being read"
    return sum(1 for op in _ring4_ops(n, **mistakes) if op[0] == "bar")


@pytest.mark.parametrize("n", list(range(1, 40)) + [123])
def test_ring4_protocol(n):
    assert _check_protocol(n) == 3 + (n - 1) // 2   # prologue 2, one per tile pair, epilogue 1


@pytest.mark.parametrize("mistake", ["drop_epilogue_barrier", "v_ring_of_two", "no_wait_on_odd"])
def test_ring4_planted_mistakes_are_caught(mistake):
    with pytest.raises(AssertionError):
        for n in range(1, 20):
            _check_protocol(n, **{mistake: True})
