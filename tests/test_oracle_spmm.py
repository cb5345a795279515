"""CPU tests that pin the oracle's numerics: TF32 rounding
(include/mma_tf32.cuh:17-22), the CSR / SWTCF / BCSR / BCSC SpMM oracles and
the canonical block builders.

Pins: definition-based TF32 vectors and an independent float64 formulation
of round-to-nearest-ties-away; the reference's closed-form known-answer test
(src/swtcf_spmm_main.cu:33-112); numpy dense matmul on the same rounded
inputs; identity / all-ones-tile / linearity invariants; exact COO
reconstruction of the block formats.
"""
import numpy as np
import pytest


# ------------------------------------------------------------------ TF32
def tf32_reference_f64(x: np.ndarray) -> np.ndarray:
    """Round fp32 to 10 explicit mantissa bits, ties away from zero, computed
    in float64 from |x| = q * ulp (a different route from the bit trick)."""
    x = x.astype(np.float32)
    out = x.astype(np.float64).copy()
    fin = np.isfinite(x) & (x != 0)
    a = np.abs(x[fin].astype(np.float64))
    _, e = np.frexp(a)  # a = m * 2**e, m in [0.5, 1)
    ulp = np.maximum(np.ldexp(1.0, e - 11), np.ldexp(1.0, -136))
    q = np.floor(a / ulp + 0.5)
    r = np.sign(x[fin]) * q * ulp
    r = np.where(np.abs(r) >= 2.0 ** 128, np.sign(r) * np.inf, r)
    out[fin] = r
    return out.astype(np.float32)


def test_tf32_known_vectors(oracle):
    cases = {
        0x3F801000: 0x3F802000,  # tie -> away from zero
        0x3F800FFF: 0x3F800000,  # below half -> down
        0x3F801001: 0x3F802000,  # above half -> up
        0xBF801000: 0xBF802000,  # negative tie -> away from zero
        0x3F7FF000: 0x3F800000,  # carries into the exponent
        0x7F7FF000: 0x7F800000,  # rounds up to +inf
        0x7F800000: 0x7F800000,  # inf unchanged
        0x7FC00001: 0x7FC00001,  # NaN payload unchanged
        0x00000000: 0x00000000,
        0x80000000: 0x80000000,
        0x00001000: 0x00002000,  # subnormal tie
        0x00000FFF: 0x00000000,
    }
    for b, want in cases.items():
        assert oracle.tf32_bits(b) == want, hex(b)


def test_tf32_matches_independent_formulation(oracle):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2 ** 32, size=200_000, dtype=np.uint64).astype(np.uint32)
    # add every rounding boundary pattern around a few exponents
    edge = np.array([(e << 23) | m for e in (1, 100, 127, 200, 254) for m in
                     (0x0FFF, 0x1000, 0x1001, 0x2FFF, 0x3000, 0x7FEFFF, 0x7FF000, 0x7FFFFF)], np.uint32)
    bits = np.concatenate([bits, edge, edge | np.uint32(0x80000000)])
    x = bits.view(np.float32)
    x = x[np.isfinite(x)]
    got = oracle.tf32(x)
    want = tf32_reference_f64(x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# ------------------------------------------------------------------ SpMM
def random_csr(n_rows, n_cols, nnz, seed, values=True):
    rng = np.random.default_rng(seed)
    keys = np.sort(rng.choice(n_rows * n_cols, size=nnz, replace=False))
    r, c = keys // n_cols, keys % n_cols
    rowptr = np.zeros(n_rows + 1, np.int64)
    np.cumsum(np.bincount(r, minlength=n_rows), out=rowptr[1:])
    vals = rng.uniform(-2, 2, nnz).astype(np.float32) if values else None
    return r, c, rowptr, c.astype(np.uint32), vals


def dense_of(r, c, vals, n_rows, n_cols):
    A = np.zeros((n_rows, n_cols), np.float64)
    A[r, c] = 1.0 if vals is None else vals
    return A


@pytest.mark.parametrize("values", [False, True])
def test_csr_spmm_matches_numpy_dense(oracle, values):
    r, c, rowptr, colind, vals = random_csr(70, 90, 800, 1, values)
    X = np.random.default_rng(2).standard_normal((90, 13)).astype(np.float32)
    for use_tf32 in (False, True):
        Y = oracle.csr_spmm(rowptr, colind, vals, X, use_tf32=use_tf32)
        tv = None if vals is None else (oracle.tf32(vals) if use_tf32 else vals)
        Xr = oracle.tf32(X) if use_tf32 else X
        want = dense_of(r, c, tv, 70, 90) @ Xr.astype(np.float64)
        np.testing.assert_allclose(Y, want, rtol=1e-12, atol=1e-12)


def test_kat_closed_form(oracle):
    # X[s][f] = a(s) + b(s) f (src/swtcf_spmm_main.cu:33-56); Y = sum a + f sum b
    assert oracle.kat_source_a(0) == np.float32(13 * 0.001)
    assert oracle.kat_source_b(1) == np.float32(36 * 0.00001)
    r, c, rowptr, colind, _ = random_csr(40, 64, 300, 3, values=False)
    X = oracle.kat_fill_x(64, 128)
    Y = oracle.csr_spmm(rowptr, colind, None, X, use_tf32=False)
    K = oracle.kat_expected(r.astype(np.uint32), c.astype(np.uint32), 40, 128)
    # only the fp32 rounding of a + b f separates the two
    np.testing.assert_allclose(Y, K, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("tc,use_tf32", [(0, True), (65, False)])
def test_swtcf_spmm_oracle_matches_csr(oracle, tc, use_tf32):
    r, c, rowptr, colind, _ = random_csr(60, 100, 700, 4, values=False)
    X = np.random.default_rng(5).standard_normal((100, 9)).astype(np.float32)
    m = oracle.swtcf_convert(r.astype(np.uint32), c.astype(np.uint32), 60, 100, 16)
    Y = oracle.swtcf_spmm(m, X, tc=tc, rows=60)
    want = oracle.csr_spmm(rowptr, colind, None, X, use_tf32=use_tf32)
    np.testing.assert_allclose(Y, want, rtol=1e-12, atol=1e-12)


def test_swtcf_spmm_threshold_splits_tiles(oracle):
    # one full 8x8 tile (popcount 64) and one single-entry tile: at tc=12 the
    # dense tile uses TF32 X, the sparse one fp32 X (src/swtcf_spmm.cu:188-241)
    dst = [r for r in range(8) for _ in range(8)] + [9]
    src = [cc for _ in range(8) for cc in range(8)] + [8]
    m = oracle.swtcf_convert(np.array(dst, np.uint32), np.array(src, np.uint32), 10, 16, 16)
    X = np.full((16, 1), 1.0 + 2.0 ** -20, np.float32)  # TF32 rounds this to 1.0
    Y = oracle.swtcf_spmm(m, X, tc=12, rows=10)
    assert np.all(Y[:8, 0] == 8.0)  # all-ones tile: sum of 8 rounded rows
    assert Y[9, 0] == np.float64(np.float32(1.0 + 2.0 ** -20))


def test_identity_and_linearity(oracle):
    n = 50
    idx = np.arange(n, dtype=np.uint32)
    m = oracle.swtcf_convert(idx, idx, n, n, 16)
    X = np.random.default_rng(6).standard_normal((n, 7)).astype(np.float32)
    np.testing.assert_array_equal(oracle.swtcf_spmm(m, X, tc=65, rows=n), X.astype(np.float64))
    r, c, rowptr, colind, vals = random_csr(30, 40, 200, 7)
    X1 = np.random.default_rng(8).standard_normal((40, 5)).astype(np.float32)
    X2 = np.random.default_rng(9).standard_normal((40, 5)).astype(np.float32)
    y = oracle.csr_spmm(rowptr, colind, vals, X1 + X2, use_tf32=False)
    y12 = oracle.csr_spmm(rowptr, colind, vals, X1, use_tf32=False) + oracle.csr_spmm(rowptr, colind, vals, X2,
                                                                                      use_tf32=False)
    np.testing.assert_allclose(y, y12, rtol=1e-5, atol=1e-5)


# ------------------------------------------------------------------ blocks
def decode_bcsr(d):
    out = []
    for w in range(d["num_rowWindows"]):
        for b in range(int(d["rowWindowOffset"][w]), int(d["rowWindowOffset"][w + 1])):
            bm = int(d["tcLocalBit"][b])
            k = int(d["tcOffset"][b])
            for bit in range(64):
                if bm >> bit & 1:
                    out.append((w * 8 + bit // 8, int(d["sparseA2B"][b * 8 + bit % 8]), float(d["data"][k])))
                    k += 1
    return sorted(out)


def decode_bcsc(d):
    out = []
    for w in range(d["num_colWindows"]):
        for b in range(int(d["colWindowOffset"][w]), int(d["colWindowOffset"][w + 1])):
            bm = int(d["tcLocalBit"][b])
            k = int(d["tcOffset"][b])
            for bit in range(64):
                if bm >> bit & 1:
                    out.append((int(d["sparseA2C"][b * 8 + bit // 8]), w * 8 + bit % 8, float(d["data"][k])))
                    k += 1
    return sorted(out)


def test_bcsr_builder_roundtrip_and_layout(oracle):
    r, c, rowptr, colind, vals = random_csr(45, 77, 500, 10)
    d = oracle.bcsr_build(45, 77, rowptr, colind, vals)
    assert decode_bcsr(d) == sorted(zip(r.tolist(), c.tolist(), vals.astype(float).tolist()))
    for w in range(d["num_rowWindows"]):
        b0, b1 = int(d["rowWindowOffset"][w]), int(d["rowWindowOffset"][w + 1])
        cols = d["sparseA2B"][b0 * 8:b1 * 8]
        real = cols[cols != 0xFFFFFFFF]
        want = np.unique(c[(r >= 8 * w) & (r < 8 * w + 8)])
        assert np.array_equal(real, want)  # distinct columns ascending, 8 per block
        assert np.all(cols[len(real):] == 0xFFFFFFFF)  # padding only at the end
    assert int(d["tcOffset"][-1]) == 500


def test_bcsc_builder_roundtrip_and_order(oracle):
    r, c, rowptr, colind, vals = random_csr(45, 77, 500, 11)
    order = np.lexsort((r, c))
    colptr = np.zeros(78, np.int64)
    np.cumsum(np.bincount(c, minlength=77), out=colptr[1:])
    d = oracle.bcsc_build(45, 77, colptr, r[order].astype(np.uint32), vals[order])
    assert decode_bcsc(d) == sorted(zip(r.tolist(), c.tolist(), vals.astype(float).tolist()))
    # same row order as the SWTCF with one window per super-window
    m = oracle.swtcf_convert(r.astype(np.uint32), c.astype(np.uint32), 45, 77, 1)
    v = oracle.swtcf_valid_extents(m)
    assert np.array_equal(d["colWindowOffset"], v["colWindowOffset"])
    assert np.array_equal(d["tcLocalBit"][:d["num_TCBlocks"]], v["tileLocalBit"])


@pytest.mark.parametrize("values", [False, True])
def test_block_spmm_oracles_match_csr(oracle, values):
    r, c, rowptr, colind, vals = random_csr(45, 77, 500, 12, values)
    X = np.random.default_rng(13).standard_normal((77, 6)).astype(np.float32)
    want = oracle.csr_spmm(rowptr, colind, vals, X, use_tf32=True)
    d = oracle.bcsr_build(45, 77, rowptr, colind, vals)
    np.testing.assert_allclose(oracle.bcsr_spmm(d, X, use_data=values)[:45], want, rtol=1e-12, atol=1e-12)
    order = np.lexsort((r, c))
    colptr = np.zeros(78, np.int64)
    np.cumsum(np.bincount(c, minlength=77), out=colptr[1:])
    e = oracle.bcsc_build(45, 77, colptr, r[order].astype(np.uint32), None if vals is None else vals[order])
    np.testing.assert_allclose(oracle.bcsc_spmm(e, X, use_data=values), want, rtol=1e-12, atol=1e-12)
    # A^T dY through the BCSC equals the dense transpose product in plain fp32
    # operands (torch.sparse.mm of train/tcgnn_conv_release.py:152 rounds nothing)
    dY = np.random.default_rng(14).standard_normal((45, 4)).astype(np.float32)
    At = dense_of(r, c, vals, 45, 77).T
    got = oracle.bcsc_transpose_spmm(e, dY, use_data=values)[:77]
    np.testing.assert_allclose(got, At @ dY.astype(np.float64), rtol=1e-12, atol=1e-12)
    # and differs from the TF32-rounded product (the planted-mistake check)
    if values:
        assert not np.allclose(got, dense_of(r, c, oracle.tf32(vals), 45, 77).T @ oracle.tf32(dY).astype(np.float64),
                               rtol=1e-9, atol=1e-9)


def test_resolve_features(oracle):
    F = 4
    hot = np.arange(3 * F, dtype=np.float32).reshape(3, F)
    cpu = -np.arange(5 * F, dtype=np.float32).reshape(5, F) - 1
    csm = np.array([2, -1, 0, -1], np.int32)
    idm = np.array([0, 4, 0, -1], np.int32)
    X = oracle.resolve_features(idm, csm, hot, 3, cpu, F)
    assert np.array_equal(X[0], hot[2]) and np.array_equal(X[1], cpu[4])
    assert np.array_equal(X[2], hot[0]) and np.all(X[3] == 0)
