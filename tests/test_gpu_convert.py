"""GPU parity: HIP COO -> SWTCF conversion, bit-exact against the oracle's
canonical form (src/swtcf_convert.cu semantics), through the C-ABI."""
import json
import os

import numpy as np
import pytest
import torch

from swtcf_checks import check_canonical

pytestmark = pytest.mark.gpu
HERE = os.path.dirname(os.path.abspath(__file__))


def convert_gpu(dst, src, rows, cols, S, cap=None):
    from tcc_amd import swtcf

    dst = np.asarray(dst, np.uint32)
    src = np.asarray(src, np.uint32)
    E = dst.size
    cap = cap or E
    d = torch.from_numpy(dst.view(np.int32)).cuda()
    s = torch.from_numpy(src.view(np.int32)).cuda()
    m = swtcf.DeviceSWTCFMatrix(rows, cols, cap, S)
    ws = swtcf.SWTCFConvertWorkspace(cap, cols, S)
    swtcf.convertCOOToSWTCF(d, s, E, m, ws)
    err = ws.device_error()
    ng = ws.num_groups()
    host = m.to_host()
    return host, err, ng


def assert_same(oracle, gpu_m, ref):
    v = oracle.swtcf_valid_extents(ref)
    for k, want in v.items():
        got = gpu_m[k]
        assert got.shape == want.shape, k
        assert np.array_equal(got, want), k


def test_hand_example(gpu, oracle):
    with open(os.path.join(HERE, "golden", "hand_example.json")) as f:
        h = json.load(f)
    m, err, _ = convert_gpu(h["dst"], h["src"], h["rows"], h["cols"], h["S"])
    assert err == 0
    assert m["tileRowSlot"].tolist() == h["tileRowSlot"]
    assert [f"0x{int(x):016x}" for x in m["tileLocalBit"]] == [s.lower() for s in h["tileLocalBit"]]
    assert m["superWindowRowCacheSlot"].tolist() == h["superWindowRowCacheSlot"]


@pytest.mark.parametrize("S", [1, 2, 3, 7, 16, 32])
@pytest.mark.parametrize("seed", [0, 1])
def test_random_bit_exact(gpu, oracle, S, seed):
    rng = np.random.default_rng(100 + seed)
    nd, ns = 300 + 37 * seed, 517 + 11 * seed
    keys = rng.choice(nd * ns, size=6000, replace=False)
    dst, src = (keys // ns).astype(np.uint32), (keys % ns).astype(np.uint32)
    m, err, ng = convert_gpu(dst, src, nd, ns, S)
    ref = oracle.swtcf_convert(dst, src, nd, ns, S)
    assert err == 0 and ng == ref["numGroups"]
    assert_same(oracle, m, ref)
    check_canonical(dst, src, ns, S, m)


def test_golden_fixtures(gpu, oracle):
    import glob

    for path in sorted(glob.glob(os.path.join(HERE, "golden", "swtcf_*.npz"))):
        z = np.load(path)
        m, err, _ = convert_gpu(z["dst"], z["src"], int(z["rows"]), int(z["cols"]), int(z["S"]))
        assert err == 0
        for k in ("colWindowOffset", "superWindowRowOffset", "tileLocalBit", "tileRowSlot", "superWindowRows",
                  "superWindowRowCacheSlot", "superWindowCachedRowSlot", "superWindowCachedCount"):
            assert np.array_equal(m[k], z[k]), f"{os.path.basename(path)}: {k}"


def test_config1_uniform_bit_exact(gpu, oracle):
    from tcc_amd.graphs import uniform_graph

    rows, cols = uniform_graph(4096, 16, 1)
    dst, src = rows.numpy().astype(np.uint32), cols.numpy().astype(np.uint32)
    # shuffled input order must not change the result
    perm = np.random.default_rng(3).permutation(dst.size)
    m, err, _ = convert_gpu(dst[perm], src[perm], 4096, 4096, 16)
    assert err == 0
    assert_same(oracle, m, oracle.swtcf_convert(dst, src, 4096, 4096, 16))


def test_rmat_config2_size_bit_exact(gpu, oracle):
    from tcc_amd.graphs import rmat_graph

    rows, cols = rmat_graph(169_000, 1_170_000, 2)
    dst, src = rows.numpy().astype(np.uint32), cols.numpy().astype(np.uint32)
    m, err, _ = convert_gpu(dst, src, 169_000, 169_000, 16)
    assert err == 0
    ref = oracle.swtcf_convert(dst, src, 169_000, 169_000, 16)
    assert_same(oracle, m, ref)
    assert oracle.validate_swtcf(dst, src, 169_000, ref) == 0


def test_repeat_cache_top32(gpu, oracle):
    dst, src = [], []
    for d in range(70):
        for w in range(4 if d < 40 else (3 if d < 50 else 2)):
            dst.append(d)
            src.append(w * 8 + (d % 8))
    m, err, _ = convert_gpu(dst, src, 70, 32, 4)
    assert err == 0
    assert int(m["superWindowCachedCount"][0]) == 32
    assert_same(oracle, m, oracle.swtcf_convert(np.array(dst, np.uint32), np.array(src, np.uint32), 70, 32, 4))


def test_capacity_larger_than_edges(gpu, oracle):
    rng = np.random.default_rng(5)
    keys = rng.choice(200 * 300, size=900, replace=False)
    dst, src = (keys // 300).astype(np.uint32), (keys % 300).astype(np.uint32)
    m, err, _ = convert_gpu(dst, src, 200, 300, 16, cap=5000)
    assert err == 0
    assert_same(oracle, m, oracle.swtcf_convert(dst, src, 200, 300, 16))


def test_device_errors(gpu):
    _, err, _ = convert_gpu([1] * 9, [2] * 9, 4, 8, 16)
    assert err == 1  # degree > 8 (src/swtcf_convert.cu:186-196)
    _, err, _ = convert_gpu([1, 2], [3, 8], 4, 8, 16)
    assert err == 5  # src >= cols
    _, err, _ = convert_gpu([1, 9], [3, 2], 4, 8, 16)
    assert err == 6  # dst >= rows


def test_reference_api_errors(gpu):
    from tcc_amd import swtcf
    from tcc_amd._lib import TccError

    with pytest.raises(TccError, match="invalid SWTCF allocation size"):
        swtcf.DeviceSWTCFMatrix(4, 8, 0, 16)
    m = swtcf.DeviceSWTCFMatrix(4, 8, 4, 16)
    ws = swtcf.SWTCFConvertWorkspace(4, 8, 16)
    d = torch.zeros(8, dtype=torch.int32, device="cuda")
    with pytest.raises(TccError, match="invalid COO"):
        swtcf.convertCOOToSWTCF(d, d, 5, m, ws)  # more edges than the capacity


def _hub_graph(rows, cols, seed):
    """Every 97th row is a hub touching about 60% of the columns, the rest
    hold about 6 edges each; returned in (dst, src) order."""
    rng = np.random.default_rng(seed)
    dense = rng.random((rows, cols)) < np.where(np.arange(rows)[:, None] % 97 == 0, 0.6, 6.0 / cols)
    dst, src = np.nonzero(dense)
    return dst.astype(np.uint32), src.astype(np.uint32)


@pytest.mark.parametrize("S", [16, 3])
def test_multi_tile_segments_sorted_and_shuffled(gpu, oracle, S):
    """Super-windows of many 4096-element tiles, hub rows of up to 8S elements
    across tile ends: a COO in (dst, src) order (the sort's one-digit path)
    and the same COO shuffled (every digit) give the oracle's arrays."""
    rows, cols = 40_000, 256
    dst, src = _hub_graph(rows, cols, 7 + S)
    ref = oracle.swtcf_convert(dst, src, rows, cols, S)
    per_sw = np.bincount(src // (8 * S))
    assert per_sw.max() > 6 * 4096  # many tiles per super-window
    m, err, ng = convert_gpu(dst, src, rows, cols, S)
    assert err == 0 and ng == ref["numGroups"]
    assert_same(oracle, m, ref)
    perm = np.random.default_rng(S).permutation(dst.size)
    m2, err2, ng2 = convert_gpu(dst[perm], src[perm], rows, cols, S)
    assert err2 == 0 and ng2 == ref["numGroups"]
    assert_same(oracle, m2, ref)


@pytest.mark.parametrize("pos", [1, 63, 64, 1023, 1024, 4095, 4096, 8191])
def test_one_pair_out_of_order(gpu, oracle, pos):
    """A (dst, src)-ordered COO with one adjacent pair swapped, at lane, wave
    and tile boundaries: the input pass must see it, or the one-digit sort
    would leave that pair out of order."""
    rows, cols = 3_000, 1_000
    rng = np.random.default_rng(pos)
    keys = np.sort(rng.choice(rows * cols, size=12_000, replace=False))
    dst, src = (keys // cols).astype(np.uint32), (keys % cols).astype(np.uint32)
    dst[[pos - 1, pos]] = dst[[pos, pos - 1]]
    src[[pos - 1, pos]] = src[[pos, pos - 1]]
    m, err, _ = convert_gpu(dst, src, rows, cols, 16)
    assert err == 0
    assert_same(oracle, m, oracle.swtcf_convert(dst, src, rows, cols, 16))


def test_rows_unknown_wide_keys(gpu, oracle):
    """rows = 0 (no destination bound): 32 destination bits, so the element
    keys pass 32 bits and take five low-digit passes."""
    rows, cols = 5_000, 2_000
    rng = np.random.default_rng(11)
    keys = rng.choice(rows * cols, size=30_000, replace=False)
    dst, src = (keys // cols).astype(np.uint32), (keys % cols).astype(np.uint32)
    dst = (dst * 811_371).astype(np.uint32)  # destinations far above 2**24
    m, err, _ = convert_gpu(dst, src, 0, cols, 16)
    assert err == 0
    assert_same(oracle, m, oracle.swtcf_convert(dst, src, 0, cols, 16))


@pytest.mark.parametrize("rows", [5_000, 0])
@pytest.mark.parametrize("S", [1, 16])
def test_two_sw_passes_sorted_and_shuffled(gpu, oracle, S, rows):
    """Enough super-windows for two sw passes, in order and shuffled.  With
    rows = 5000 the keys fit 32 bits: the second sw pass rebuilds each
    element's low sw bits from its position in the first's output, and the
    shuffled COO takes the per-super-window low-digit passes.  With rows = 0
    (32 destination bits) the 64-bit elements take every digit."""
    n_dst, cols = 5_000, 300_000
    rng = np.random.default_rng(40 + S)
    keys = np.sort(rng.choice(n_dst * cols, size=200_000, replace=False))
    dst, src = (keys // cols).astype(np.uint32), (keys % cols).astype(np.uint32)
    ref = oracle.swtcf_convert(dst, src, rows, cols, S)
    for order in (np.arange(dst.size), np.random.default_rng(S).permutation(dst.size)):
        m, err, ng = convert_gpu(dst[order], src[order], rows, cols, S)
        assert err == 0 and ng == ref["numGroups"]
        assert_same(oracle, m, ref)
