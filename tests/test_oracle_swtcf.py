"""CPU tests that pin the oracle's COO -> SWTCF restatement
(oracle/oracle.c: oracle_swtcf_convert, oracle_validate_swtcf,
oracle_validate_repeat_cache).

Pins used: a hand-worked example (tests/golden/hand_example.json), the
independent canonical-form checks of tests/swtcf_checks.py, the reference's
own validators restated in C (src/swtcf_convert_main.cu:36-310), COO
reconstruction, special cases, and mistakes planted in oracle outputs that
each check must catch.
"""
import json
import os

import numpy as np
import pytest

from swtcf_checks import check_canonical, coo_from_swtcf

HERE = os.path.dirname(os.path.abspath(__file__))


def hand():
    with open(os.path.join(HERE, "golden", "hand_example.json")) as f:
        return json.load(f)


def random_coo(n_dst, n_src, nnz, seed):
    rng = np.random.default_rng(seed)
    keys = rng.choice(n_dst * n_src, size=nnz, replace=False)
    return (keys // n_src).astype(np.uint32), (keys % n_src).astype(np.uint32)


def test_hand_example(oracle):
    h = hand()
    m = oracle.swtcf_convert(h["dst"], h["src"], h["rows"], h["cols"], h["S"])
    assert m["err"] == 0
    v = oracle.swtcf_valid_extents(m)
    assert v["colWindowOffset"].tolist() == h["colWindowOffset"]
    assert v["superWindowRowOffset"].tolist() == h["superWindowRowOffset"]
    assert v["superWindowRows"].tolist() == h["superWindowRows"]
    assert v["superWindowRowCacheSlot"].tolist() == h["superWindowRowCacheSlot"]
    assert v["superWindowCachedCount"].tolist() == h["superWindowCachedCount"]
    assert v["superWindowCachedRowSlot"][:3].tolist() == h["superWindowCachedRowSlot_sw0_head"]
    assert v["tileRowSlot"].tolist() == h["tileRowSlot"]
    assert [f"0x{int(x):016x}" for x in v["tileLocalBit"]] == [s.lower() for s in h["tileLocalBit"]]
    check_canonical(h["dst"], h["src"], h["cols"], h["S"], m)


@pytest.mark.parametrize("S", [1, 2, 3, 7, 16, 32])
@pytest.mark.parametrize("seed", [0, 1, 2])
def test_random_graphs_canonical_and_valid(oracle, S, seed):
    n_dst, n_src = 97 + 31 * seed, 203 + 17 * seed  # cols not a multiple of 8 or 128
    dst, src = random_coo(n_dst, n_src, 900 + 200 * seed, seed)
    m = oracle.swtcf_convert(dst, src, n_dst, n_src, S)
    assert m["err"] == 0
    assert oracle.validate_swtcf(dst, src, n_src, m) == 0
    assert oracle.validate_repeat_cache(m) == 0
    check_canonical(dst, src, n_src, S, m)
    assert coo_from_swtcf(m, S) == sorted(zip(dst.tolist(), src.tolist()))


def test_uniform_config1_canonical(oracle):
    from tcc_amd.graphs import uniform_graph

    rows, cols = uniform_graph(4096, 16, 1)
    dst, src = rows.numpy().astype(np.uint32), cols.numpy().astype(np.uint32)
    m = oracle.swtcf_convert(dst, src, 4096, 4096, 16)
    assert m["err"] == 0 and m["numGroups"] > 60000
    assert oracle.validate_swtcf(dst, src, 4096, m) == 0
    assert oracle.validate_repeat_cache(m) == 0
    check_canonical(dst, src, 4096, 16, m)


def test_more_than_32_repeated_rows(oracle):
    # one super-window (S=4, 32 sources); 40 destinations in all 4 windows,
    # 10 in 3 windows, 20 in 2: the cache keeps the 32 most frequent, lowest
    # slot first.
    dst, src = [], []
    for d in range(70):
        nwin = 4 if d < 40 else (3 if d < 50 else 2)
        for w in range(nwin):
            dst.append(d)
            src.append(w * 8 + (d % 8))
    dst = np.array(dst, np.uint32)
    src = np.array(src, np.uint32)
    m = oracle.swtcf_convert(dst, src, 70, 32, 4)
    assert m["err"] == 0
    assert int(m["superWindowCachedCount"][0]) == 32
    assert m["superWindowCachedRowSlot"][:32].tolist() == list(range(32))
    assert oracle.validate_repeat_cache(m) == 0
    check_canonical(dst, src, 32, 4, m)


def test_special_cases(oracle):
    # single edge
    m = oracle.swtcf_convert([3], [5], 4, 6, 16)
    assert m["err"] == 0 and m["numTiles"] == 1 and m["numRows"] == 1
    assert int(m["tileLocalBit"][0]) == 1 << 5
    assert m["tileRowSlot"][:8].tolist() == [0] + [0xFFFFFFFF] * 7
    # an empty window has 0 tiles; a window with 9 rows has 2 tiles, 7 padding slots
    dst = np.arange(9, dtype=np.uint32)
    src = np.full(9, 17, np.uint32)  # window 2 only
    m = oracle.swtcf_convert(dst, src, 9, 24, 16)
    assert m["colWindowOffset"].tolist() == [0, 0, 0, 2]
    assert m["tileRowSlot"][8:16].tolist() == [8] + [0xFFFFFFFF] * 7
    check_canonical(dst, src, 24, 16, m)


def test_device_error_codes(oracle):
    # 9 copies of one edge: degree 9 > 8 -> error 1 (src/swtcf_convert.cu:186-196)
    assert oracle.swtcf_convert([1] * 9, [2] * 9, 4, 8, 16)["err"] == 1
    # src >= cols -> 5, dst >= rows -> 6 (range checks the reference does not make)
    assert oracle.swtcf_convert([1], [8], 4, 8, 16)["err"] == 5
    assert oracle.swtcf_convert([4], [1], 4, 8, 16)["err"] == 6


def test_planted_mistakes_are_caught(oracle):
    dst, src = random_coo(60, 120, 700, 7)
    good = oracle.swtcf_convert(dst, src, 60, 120, 16)
    assert oracle.validate_swtcf(dst, src, 120, good) == 0

    def mutated(fn):
        m = {k: (v.copy() if isinstance(v, np.ndarray) else v) for k, v in good.items()}
        fn(m)
        return m

    # a flipped bitmap bit breaks COO reconstruction
    m = mutated(lambda m: m["tileLocalBit"].__setitem__(0, m["tileLocalBit"][0] ^ np.uint64(1 << 63)))
    assert oracle.validate_swtcf(dst, src, 120, m) != 0
    # a padding slot that is not INVALID
    T = good["numTiles"]
    pad = [i for i in range(T * 8) if ((int(good["tileLocalBit"][i // 8]) >> (8 * (i % 8))) & 0xFF) == 0]
    assert pad, "the sample needs a padding row"
    m = mutated(lambda m: m["tileRowSlot"].__setitem__(pad[0], 0))
    assert oracle.validate_swtcf(dst, src, 120, m) != 0
    # swapping two equal-degree rows keeps the matrix legal but not canonical
    tlb = good["tileLocalBit"]
    t = next(t for t in range(T) if all(((int(tlb[t]) >> (8 * r)) & 0xFF) for r in range(2))
             and bin((int(tlb[t]) >> 0) & 0xFF).count("1") == bin((int(tlb[t]) >> 8) & 0xFF).count("1"))

    def swap_rows(m):
        b = int(m["tileLocalBit"][t])
        r0, r1 = b & 0xFF, (b >> 8) & 0xFF
        m["tileLocalBit"][t] = np.uint64((b & ~0xFFFF) | (r0 << 8) | r1)
        s = m["tileRowSlot"]
        s[t * 8], s[t * 8 + 1] = s[t * 8 + 1], s[t * 8]

    m = mutated(swap_rows)
    assert oracle.validate_swtcf(dst, src, 120, m) == 0
    with pytest.raises(AssertionError):
        check_canonical(dst, src, 120, 16, m)
    # a cache entry pointing at the wrong row
    if good["superWindowCachedCount"][0] >= 2:
        def swap_cache(m):
            c = m["superWindowCachedRowSlot"]
            c[0], c[1] = c[1], c[0]
        m = mutated(swap_cache)
        assert oracle.validate_repeat_cache(m) != 0
    # a wrong cached count
    m = mutated(lambda m: m["superWindowCachedCount"].__setitem__(0, m["superWindowCachedCount"][0] + 1))
    assert oracle.validate_repeat_cache(m) != 0


def test_golden_fixtures_unchanged(oracle):
    """The committed fixtures (tests/golden/*.npz, made by make_fixtures.py)
    still match the oracle bit for bit."""
    import glob

    files = sorted(glob.glob(os.path.join(HERE, "golden", "swtcf_*.npz")))
    assert files, "run tests/golden/make_fixtures.py"
    for path in files:
        z = np.load(path)
        S, rows, cols = int(z["S"]), int(z["rows"]), int(z["cols"])
        m = oracle.swtcf_convert(z["dst"], z["src"], rows, cols, S)
        v = oracle.swtcf_valid_extents(m)
        for k in v:
            assert np.array_equal(v[k], z[k]), f"{os.path.basename(path)}: {k}"
