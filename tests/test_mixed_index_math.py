"""Host replay of the first layer's feature-row lookups (no GPU).

The kernels resolve column j as (bcsr_spmm.hip, mixed_row; reference rule
spmm_kernel.cu:129-153): g = cache_search_map[j]; g >= 0 reads row g % cap
of cache entry g / cap, else row id_map[j] of the host table (zeros when
id_map[j] < 0).  A lookup outside its table is refused (zeros and
TCC_DEVERR_FEATURE_INDEX) instead of read.  This replays that arithmetic on
the inputs of the GPU tests of the first-layer product and of the GCN
feature table, and checks that every lookup lands inside its table, so that
those tests never depend on the refusal path (the GPU test of refused
lookups plants bad entries on purpose)."""
import numpy as np


def lookups(csm, id_map, cap, cache_entries, cache_rows, host_rows):
    """(cache entry, row) or ('host', row) of every column, and whether it is
    inside its table, by the kernels' rule."""
    out = []
    for j in range(csm.size):
        g = int(csm[j])
        if g >= 0:
            d, r = divmod(g, cap)
            out.append(("cache", d, r, d < cache_entries and r < cache_rows))
        elif id_map[j] >= 0:
            out.append(("host", 0, int(id_map[j]), int(id_map[j]) < host_rows))
        else:
            out.append(("zero", 0, 0, True))
    return out


def forms_test_inputs():
    """tests/test_spmm_cnic_ext.py::test_forward_tensorcore_mixed_forms."""
    nc = 800
    rng = np.random.default_rng(4)
    rng.standard_normal((nc, 100))
    hot_ids = np.sort(rng.choice(nc, size=nc // 5, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    return csm, np.arange(nc, dtype=np.int32), hot_ids.size, nc


def feature_source_test_inputs():
    """tests/test_gpu_spmm.py::test_mixed_hot_cold_feature_source."""
    nc = 1000
    rng = np.random.default_rng(21)
    rng.standard_normal((nc, 100))
    hot_ids = np.sort(rng.choice(nc, size=nc // 5, replace=False))
    csm = np.full(nc, -1, np.int32)
    csm[hot_ids] = np.arange(hot_ids.size, dtype=np.int32)
    id_map = np.arange(nc, dtype=np.int32)
    id_map[7] = -1
    csm[7] = -1
    return csm, id_map, hot_ids.size, nc


def feature_table_inputs(n=5000, seed=3):
    """tcc_amd.gcn.FeatureTable: hot = top 20% of columns by degree, rank
    order; id_map = identity; one cache entry of n_hot rows."""
    rng = np.random.default_rng(seed)
    deg = rng.integers(0, 50, n)
    n_hot = max(1, int(round(n * 0.2)))
    order = np.lexsort((np.arange(n), -deg))
    hot_ids = np.sort(order[:n_hot])
    csm = np.full(n, -1, np.int32)
    csm[hot_ids] = np.arange(n_hot, dtype=np.int32)
    return csm, np.arange(n, dtype=np.int32), n_hot, n


def test_every_lookup_of_the_gpu_tests_is_inside_its_table():
    for csm, id_map, cap, n in (forms_test_inputs(), feature_source_test_inputs(), feature_table_inputs()):
        res = lookups(csm, id_map, cap, cache_entries=1, cache_rows=cap, host_rows=n)
        assert all(ok for *_, ok in res)
        kinds = {k for k, *_ in res}
        assert "cache" in kinds and "host" in kinds


def test_replay_flags_planted_bad_entries():
    """The replay itself catches the two bad entries the refusal test plants
    (a mistake planted in the inputs, on the CPU)."""
    csm, id_map, cap, n = forms_test_inputs()
    csm = csm.copy()
    id_map = id_map.copy()
    hot = np.nonzero(csm >= 0)[0]
    cold = np.nonzero(csm < 0)[0]
    csm[hot[0]] = cap + 3
    id_map[cold[0]] = n
    res = lookups(csm, id_map, cap, cache_entries=1, cache_rows=cap, host_rows=n)
    bad = [j for j, (*_, ok) in enumerate(res) if not ok]
    assert bad == sorted([int(hot[0]), int(cold[0])])
