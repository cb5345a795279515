"""Independent checks that pin a SWTCF to the canonical form.

Written from the format rules (src/swtcf_convert.cu, SWTCF appendix of the
build notes restated in the oracle header) with numpy set operations, not from
the oracle's code.  `check_canonical` passes for exactly one SWTCF per input:

* per column window, the multiset of rows {(degree, bitmap, dst)} equals the
  one computed from the COO, the rows appear in (degree desc, dst asc) order,
  8 per tile, with the padding rows of the last tile empty;
* per super-window, the slots are its distinct destinations in ascending
  order, and tile rows point at the slot of their destination;
* the repeat cache holds the min(32, #repeated) rows first in
  (occurrence desc, slot asc) order, with matching forward/reverse maps.
"""
from __future__ import annotations

import numpy as np

INVALID = 0xFFFFFFFF


def _rows_from_coo(dst, src, S):
    """{window: sorted list of (-deg, dst, bits)} and {sw: {dst: occurrence}}."""
    dst = np.asarray(dst, np.int64)
    src = np.asarray(src, np.int64)
    w = src >> 3
    key = w * (1 << 32) + dst
    order = np.argsort(key, kind="stable")
    key_s, lc_s = key[order], (src & 7)[order]
    uk, start, cnt = np.unique(key_s, return_index=True, return_counts=True)
    bits = np.bitwise_or.reduceat(np.left_shift(1, lc_s), start) if len(start) else np.array([], np.int64)
    per_window = {}
    occ = {}
    for k, c, b in zip(uk.tolist(), cnt.tolist(), bits.tolist()):
        win, d = k >> 32, k & 0xFFFFFFFF
        per_window.setdefault(win, []).append((-c, d, b))
        occ.setdefault(win // S, {}).setdefault(d, 0)
        occ[win // S][d] += 1
    for win in per_window:
        per_window[win].sort()
    return per_window, occ


def check_canonical(dst, src, cols: int, S: int, m: dict) -> None:
    """Raise AssertionError unless `m` is the canonical SWTCF of the COO."""
    CW = (cols + 7) // 8
    SW = (CW + S - 1) // S
    per_window, occ = _rows_from_coo(dst, src, S)
    cwo = np.asarray(m["colWindowOffset"], np.int64)
    swo = np.asarray(m["superWindowRowOffset"], np.int64)
    assert cwo.shape == (CW + 1,) and swo.shape == (SW + 1,)
    # tiles per window and super-window row lists (closed forms)
    expected_tiles = [(len(per_window.get(w, [])) + 7) // 8 for w in range(CW)]
    assert cwo[0] == 0 and np.array_equal(np.diff(cwo), expected_tiles), "colWindowOffset"
    sw_rows = [np.array(sorted(occ.get(s, {}).keys()), np.int64) for s in range(SW)]
    assert swo[0] == 0 and np.array_equal(np.diff(swo), [len(r) for r in sw_rows]), "superWindowRowOffset"
    U = int(swo[-1])
    rows_arr = np.asarray(m["superWindowRows"][:U], np.int64)
    assert np.array_equal(rows_arr, np.concatenate(sw_rows) if SW else rows_arr[:0]), "superWindowRows"
    T = int(cwo[-1])
    tlb = np.asarray(m["tileLocalBit"][:T], np.uint64)
    trs = np.asarray(m["tileRowSlot"][:T * 8], np.int64)
    for w in range(CW):
        s = w // S
        want = per_window.get(w, [])
        got = []
        for t in range(int(cwo[w]), int(cwo[w + 1])):
            for r in range(8):
                b = int((int(tlb[t]) >> (8 * r)) & 0xFF)
                slot = int(trs[t * 8 + r])
                i = (t - int(cwo[w])) * 8 + r
                if i >= len(want):
                    assert b == 0 and slot == INVALID, f"padding row of window {w}"
                    continue
                assert slot != INVALID and slot < len(sw_rows[s]), f"slot of window {w}"
                got.append((-bin(b).count("1"), int(sw_rows[s][slot]), b))
        # rows in canonical order with the right (degree, dst, bitmap)
        want_bits = [(-bin(b).count("1"), d, b) for (_, d, b) in want]
        assert got == want_bits, f"rows of window {w}"
    # repeat cache
    rcs = np.asarray(m["superWindowRowCacheSlot"][:U], np.int64)
    crs = np.asarray(m["superWindowCachedRowSlot"], np.int64).reshape(SW, 32)
    cc = np.asarray(m["superWindowCachedCount"][:SW], np.int64)
    for s in range(SW):
        base = int(swo[s])
        o = occ.get(s, {})
        rep = sorted([(-o[d], slot) for slot, d in enumerate(sw_rows[s].tolist()) if o[d] > 1])
        n = min(32, len(rep))
        assert cc[s] == n, f"cachedCount of super-window {s}"
        for c in range(32):
            if c < n:
                slot = rep[c][1]
                assert crs[s, c] == slot, f"cache slot {c} of super-window {s}"
                assert rcs[base + slot] == c, f"reverse map of super-window {s}"
            else:
                assert crs[s, c] == INVALID, f"unused cache entry {c} of super-window {s}"
        cached = set(int(crs[s, c]) for c in range(n))
        for slot in range(len(sw_rows[s])):
            if slot not in cached:
                assert rcs[base + slot] == 0xFF, f"uncached row has a cache slot (sw {s})"


def coo_from_swtcf(m: dict, S: int):
    """Reconstruct the sorted (dst, src) list from a SWTCF (decode only)."""
    cwo, swo = m["colWindowOffset"], m["superWindowRowOffset"]
    out = []
    for w in range(len(cwo) - 1):
        base = int(swo[w // S])
        for t in range(int(cwo[w]), int(cwo[w + 1])):
            for r in range(8):
                b = (int(m["tileLocalBit"][t]) >> (8 * r)) & 0xFF
                if not b:
                    continue
                d = int(m["superWindowRows"][base + int(m["tileRowSlot"][t * 8 + r])])
                out.extend((d, w * 8 + c) for c in range(8) if b >> c & 1)
    return sorted(out)
