"""Binary hub tiles (tcc_coo_to_hybrid_scaled, TCC_TILES_BINARY).

The reference multiplies each block's bitmap as a {0, 1} operand
(src/swtcf_spmm.cu:193-200); the binary hybrid stores the 16x16 tiles of the
degree-ordered matrix as patterns and takes a matrix's values as row and
column scales, A = diag(r) P diag(c).

Checked through the C-ABI:
- the arrays, exactly, against an independent numpy construction of the
  layout include/tcc_spmm_cnic.h states: steps = (group of G row blocks,
  pair of 16-column blocks) whose tiles hold at least min_step_nnz entries
  together, every entry of such a step stored in sub-step records of the
  2:4 sparse MFMA's operands (per lane and 32-row tile a value-mask byte
  and 16 bits of positions, two value slots per group of four columns, a
  second layer where a group holds more than two entries); units, their
  launch order, the partial-sum slots of shared groups and the shared-group
  list; the scales in rowOrder's order and in row order; the remainder
  equal to the oracle's BCSR of exactly the other entries, without values;
- the products, against the fp64 CSR oracle over the pattern and the
  column-scaled, TF32-rounded X, times the row scales (rel-L2 <= 1e-5: the
  tiles' bf16 halves of TF32(c x) are exact, the sums fp32), and against the
  north star's bound, rel-L2 <= 1e-3 of the TF32 CSR oracle over the values
  fp32(r_i c_j) (sym-norm scales, F >= 16); without scales the product is the oracle's own (1e-5);
  in a workspace of NaN bytes, Y = AX and Y += AX, G = 8 and 16, step
  thresholds from 1 to 256, units of 1 to 3000 steps (the kernel reads
  a unit's step list 256 steps at a time), phased remainders, F from 1 to
  700, hubs or uniform, a fully dense corner;
- an Inf in a hub column's feature row: rows with that column get Inf (or
  NaN), the rows a zero value slot pointing at it reaches get NaN (0 * Inf
  in the tiles' products), every other row stays finite;
- half records: fp16 values of 2^e x where exact for a whole (column-block
  pair, 32-feature slice), the bf16 halves elsewhere, both in one product (a
  feature below the fp16 grid and one above its range), through the hybrid
  and through tcc_hub_tiles_spmm alone;
- argument errors.
"""
import numpy as np
import pytest
import torch

from test_gpu_hybrid import dev_u32, oracle_product, random_coo, rel_l2, tf32

pytestmark = pytest.mark.gpu

REL = 1e-5
NORTH_STAR = 1e-3
DEFAULT_MIN_STEP, DEFAULT_G, DEFAULT_UNIT_STEPS = 40, 16, 1024


def _nibble_tables():
    """(values, positions)[layer][nibble]: the two value slots a nibble's
    entries take in a layer (layer 0: its lowest two set bits, layer 1: the
    rest), as the sparse MFMA reads them: value bits (slot 0 low) and 2-bit
    positions (slot 0 low), increasing, a slot without an entry on an unused
    position."""
    vals = np.zeros((2, 16), np.uint32)
    pos = np.zeros((2, 16), np.uint32)
    for nib in range(16):
        bits = [p for p in range(4) if nib >> p & 1]
        for layer, sel in enumerate((bits[:2], bits[2:])):
            if len(sel) == 2:
                v, (p0, p1) = 3, sel
            elif len(sel) == 1:
                v, (p0, p1) = (1, (sel[0], 3)) if sel[0] < 3 else (2, (2, 3))
            else:
                v, (p0, p1) = 0, (0, 1)
            vals[layer, nib], pos[layer, nib] = v, p0 | p1 << 2
    return vals, pos


NIB_VALS, NIB_POS = _nibble_tables()


def reference_binary_layout(dst, src, nr, nc, min_step, G, unit_steps, r=None, c=None):
    """The layout include/tcc_spmm_cnic.h states for binary tiles: steps of
    G row blocks by a pair of 16-column blocks, the pattern in sub-step
    records of value masks and positions (a second layer where a group of
    four columns holds more than two entries)."""
    dst = dst.astype(np.int64)
    src = src.astype(np.int64)
    rorder = np.lexsort((np.arange(nr), -np.bincount(dst, minlength=nr)))
    corder = np.lexsort((np.arange(nc), -np.bincount(src, minlength=nc)))
    rrank = np.empty(nr, np.int64)
    rrank[rorder] = np.arange(nr)
    crank = np.empty(nc, np.int64)
    crank[corder] = np.arange(nc)
    RB, CB = (nr + 15) // 16, (nc + 15) // 16
    CB += CB % 2
    CP = CB // 2
    NG = (RB + G - 1) // G
    T = G // 2
    row_order = np.full(16 * G * NG, 0xFFFFFFFF, np.uint32)
    row_order[:nr] = rorder
    rr, cr = rrank[dst], crank[src]
    rb, cb = rr // 16, cr // 16
    tile = rb * CB + cb
    tkeys, tcounts = np.unique(tile, return_counts=True)
    tstep = (tkeys // CB) // G * CP + (tkeys % CB) // 2
    skeys, sinv = np.unique(tstep, return_inverse=True)
    snnz = np.bincount(sinv, weights=tcounts).astype(np.int64) if tkeys.size else np.zeros(0, np.int64)
    dense_tile = snnz[sinv] >= min_step if tkeys.size else np.zeros(0, bool)
    dense_keys = tkeys[dense_tile]
    in_dense = np.isin(tile, dense_keys)
    step_keys = np.unique((dense_keys // CB) // G * CP + (dense_keys % CB) // 2)
    S = step_keys.size
    raw = np.zeros((S, 2, 32 * G), np.uint8)
    sid = np.searchsorted(step_keys, (rb[in_dense] // G) * CP + cb[in_dense] // 2)
    j, i, k = rb[in_dense] % G, rr[in_dense] % 16, cr[in_dense] % 16
    byte = (16 * (j % 2) + i + 32 * (k // 8)) * (G // 2) + j // 2
    np.bitwise_or.at(raw, (sid, cb[in_dense] % 2, byte), (1 << (k % 8)).astype(np.uint8))
    lanes = raw.reshape(S, 2, 64, T).astype(np.uint32)  # [step, half, lane, tile]
    nib = np.stack([lanes[:, 0] & 15, lanes[:, 0] >> 4, lanes[:, 1] & 15, lanes[:, 1] >> 4], -1)  # [S, lane, tile, 4]
    crowded = (np.array([bin(x).count("1") for x in range(16)])[nib] > 2).reshape(S, 64 * T * 4).any(1)
    layers = np.where(crowded, 2, 1)
    sub_step = np.repeat(np.arange(S), layers)
    sub_layer = np.concatenate([np.arange(n) for n in layers]) if S else np.zeros(0, np.int64)
    SS = sub_step.size
    recs = np.zeros((SS + 1, 96 * G), np.uint8)
    for q in range(SS):
        n4 = nib[sub_step[q]]
        L = sub_layer[q]
        m = (NIB_VALS[L][n4] << (2 * np.arange(4))).sum(-1)        # [lane, tile] value masks
        ix = (NIB_POS[L][n4] << (4 * np.arange(4))).sum(-1)        # [lane, tile] 16-bit positions
        recs[q, :32 * G] = m.astype(np.uint8).reshape(-1)
        recs[q, 32 * G:] = ix.astype("<u2").reshape(-1).view(np.uint8)
    sg, sp = step_keys // CP, step_keys % CP
    gso_steps = np.searchsorted(sg, np.arange(NG + 1))
    sub_pos = np.concatenate([[0], np.cumsum(layers)]).astype(np.int64)
    gso = sub_pos[gso_steps].astype(np.uint32)
    sc = sp[sub_step]
    units, partial, shared = [], [], []
    slots = 0  # partial-sum slots handed out so far (units of shared groups, in unit order)
    for g in range(NG):
        p0, p1 = int(gso[g]), int(gso[g + 1])
        nu = -(-(p1 - p0) // unit_steps)
        if nu > 1:
            shared.append((g, slots, nu))
        for q in range(nu):
            units.append((g, p0 + q * unit_steps, min(p0 + (q + 1) * unit_steps, p1)))
            partial.append(slots if nu > 1 else 0xFFFFFFFF)
            slots += 1 if nu > 1 else 0
    units = np.array(units, np.uint32).reshape(-1, 3)
    # launch order: buckets of 128 sub-steps, the largest first, then the column pair of the first sub-step
    size = units[:, 2].astype(np.int64) - units[:, 1]
    unit_order = (np.lexsort((sc[units[:, 1]], -np.minimum(size // 128, 65535))) if len(units)
                  else np.zeros(0, np.int64)).astype(np.uint32)
    hub_cols = min(32 * (int(sp.max()) + 1), nc) if S else 0
    d = dict(rowOrder=row_order, hubColOrder=corder[:hub_cols].astype(np.uint32), groupStepOffset=gso,
             stepCol=sc.astype(np.uint32), tileMasks=recs, units=units, unitOrder=unit_order,
             unitPartial=np.array(partial, np.uint32), sharedGroups=np.array(shared, np.uint32).reshape(-1, 3),
             hub_cols=hub_cols, num_tiles=int(dense_keys.size), rest=~in_dense, layers=layers)
    if r is not None:
        rs = np.zeros(16 * G * NG, np.float32)
        rs[:nr] = r[rorder]
        d["rowScale"] = rs
        rr8 = np.zeros((nr + 7) // 8 * 8, np.float32)
        rr8[:nr] = r
        d["restRowScale"] = rr8
    return d


def scaled_product(oracle, dst, src, nr, X, r, c):
    """r_i * sum_j P_ij TF32(fp32(c_j X_j)) in fp64: the oracle's CSR SpMM of
    the pattern over the column-scaled, TF32-rounded rows, times r."""
    Xs = X if c is None else (X * c[:, None]).astype(np.float32)
    Y = oracle_product(oracle, dst, src, None, nr, tf32(Xs))
    return Y if r is None else Y * r[:, None].astype(np.float64)


def scales(nr, nc, dst, src, kind, seed):
    if kind == "none":
        return None, None
    if kind == "symnorm":  # config 3's values: 1/sqrt(rowdeg * coldeg)
        rd = np.bincount(dst.astype(np.int64), minlength=nr).astype(np.float64)
        cd = np.bincount(src.astype(np.int64), minlength=nc).astype(np.float64)
        r = np.where(rd > 0, 1.0 / np.sqrt(np.maximum(rd, 1)), 0.0).astype(np.float32)
        c = np.where(cd > 0, 1.0 / np.sqrt(np.maximum(cd, 1)), 0.0).astype(np.float32)
        return r, c
    rng = np.random.default_rng(seed)
    return rng.uniform(-2, 2, nr).astype(np.float32), rng.uniform(-2, 2, nc).astype(np.float32)


def build(swtcf, dst, src, nr, nc, r, c, **kw):
    return swtcf.coo_to_hybrid_scaled(dev_u32(dst), dev_u32(src), nr, nc,
                                      None if r is None else torch.from_numpy(r).cuda(),
                                      None if c is None else torch.from_numpy(c).cuda(), **kw)


@pytest.mark.parametrize("nr, nc, nnz, hubs, min_step, G, unit_steps, scale", [
    (500, 700, 30000, True, 32, 16, 0, "symnorm"),
    (500, 700, 30000, True, 8, 8, 3, "random"),
    (129, 33, 2000, False, 1, 16, 1, "none"),       # every occupied step stored; a partly empty last group
    (300, 300, 5000, True, 256, 16, 0, "random"),   # steps need 256 entries
    (300, 300, 5000, True, 100000, 8, 0, "random"),  # no step qualifies: all in the remainder
    (40, 900, 9000, True, 6, 16, 7, "symnorm"),     # fewer rows than one group
    (300, 4000, 60000, True, 4, 8, 300, "random"),  # units past 256 steps (step list in two reads)
    (600, 5000, 150000, True, 16, 16, 3000, "symnorm"),
    (60, 60, 0, False, 32, 16, 0, "random"),
    (64, 64, 4096, False, 64, 16, 0, "none"),        # a fully dense corner: every step in two layers
])
def test_binary_arrays_match_numpy_layout(gpu, oracle, nr, nc, nnz, hubs, min_step, G, unit_steps, scale):
    from tcc_amd import swtcf

    dst, src = random_coo(nr, nc, nnz, nr * 7 + nc + nnz, hubs)
    r, c = scales(nr, nc, dst, src, scale, nnz + 3)
    H = build(swtcf, dst, src, nr, nc, r, c, min_step_nnz=min_step, group_blocks=G, unit_steps=unit_steps)
    h = H.to_host()
    want = reference_binary_layout(dst, src, nr, nc, min_step, G, unit_steps or DEFAULT_UNIT_STEPS, r, c)
    print(f"binary layout nr={nr} nc={nc} nnz={nnz} step>={min_step} G={G}: {h['num_steps']} sub-steps "
          f"({int((want['layers'] == 2).sum())} second layers), "
          f"{h['num_tiles']} tiles, {h['tile_nnz']} tile entries, {h['num_shared_groups']} shared groups", flush=True)
    assert h["tile_format"] == swtcf.TILES_BINARY
    if nnz == nr * nc:
        assert np.all(want["layers"] == 2)
    assert h["group_blocks"] == G and h["unit_steps"] == (unit_steps or DEFAULT_UNIT_STEPS)
    assert h["hub_cols"] == want["hub_cols"] and h["num_tiles"] == want["num_tiles"]
    for k in ("rowOrder", "hubColOrder", "groupStepOffset", "stepCol", "units", "unitOrder", "unitPartial",
              "sharedGroups", "tileMasks"):
        assert np.array_equal(h[k], want[k]), k
    assert h["num_partial_units"] == int((want["unitPartial"] != 0xFFFFFFFF).sum())
    assert h["tile_nnz"] == int((~want["rest"]).sum())
    if r is None:
        assert h["rowScale"] is None and h["colScale"] is None and h["restRowScale"] is None
    else:
        assert np.array_equal(h["rowScale"], want["rowScale"])
        assert np.array_equal(h["restRowScale"], want["restRowScale"])
        assert np.array_equal(h["colScale"], c)
    rest = want["rest"]
    rd, rs = dst[rest].astype(np.int64), src[rest]
    order = np.lexsort((rs, rd))
    rowptr = np.zeros(nr + 1, np.int64)
    np.cumsum(np.bincount(rd, minlength=nr), out=rowptr[1:])
    ob = oracle.bcsr_build(nr, nc, rowptr, rs[order], None)
    got = h["rest"]
    B = ob["num_TCBlocks"]
    assert got["num_TCBlocks"] == B and got["nnz"] == int(rest.sum())
    assert got["data"] is None
    assert np.array_equal(got["rowWindowOffset"], ob["rowWindowOffset"])
    assert np.array_equal(got["sparseA2B"], ob["sparseA2B"][: 8 * B])
    assert np.array_equal(got["tcLocalBit"], ob["tcLocalBit"][:B])


BIN_CASES = [
    # nr, nc, nnz, hubs, min_step, G, unit_steps, phases, scale, F
    (500, 700, 30000, True, 32, 16, 0, 1, "symnorm", 602),
    (500, 700, 30000, True, 32, 16, 1, 4, "random", 602),
    (500, 700, 30000, True, 8, 8, 3, 1, "none", 90),
    (1000, 900, 60000, True, 24, 16, 0, 4, "symnorm", 256),
    (1000, 900, 60000, True, 24, 8, 2, 1, "random", 257),
    (129, 33, 2000, False, 1, 16, 3, 1, "random", 64),
    (300, 300, 5000, True, 256, 16, 0, 1, "symnorm", 100),
    (64, 64, 4096, False, 64, 16, 0, 1, "random", 1),    # a fully dense corner
    (64, 64, 4096, False, 1, 8, 1, 1, "none", 3),
    (777, 1500, 40000, True, 16, 16, 5, 2, "symnorm", 700),
    (400, 4000, 120000, True, 4, 16, 300, 1, "random", 130),   # units past 256 steps
    (600, 5000, 150000, True, 16, 16, 3000, 1, "symnorm", 96),  # a unit of every step of a group
    (400, 8000, 200000, True, 8, 8, 0, 1, "symnorm", 33),
    (40, 900, 9000, True, 6, 16, 7, 1, "random", 48),
    (60, 60, 0, False, 32, 16, 0, 1, "random", 64),
]


@pytest.mark.parametrize("nr, nc, nnz, hubs, min_step, G, unit_steps, phases, scale, F", BIN_CASES)
def test_binary_hybrid_spmm_vs_oracle(gpu, oracle, nr, nc, nnz, hubs, min_step, G, unit_steps, phases, scale, F):
    from tcc_amd import swtcf

    print(f"binary hybrid nr={nr} nc={nc} nnz={nnz} step>={min_step} G={G} unit_steps={unit_steps} "
          f"phases={phases} scale={scale} F={F}", flush=True)
    dst, src = random_coo(nr, nc, nnz, 11 * nr + nc + F, hubs)
    r, c = scales(nr, nc, dst, src, scale, F + nnz)
    rng = np.random.default_rng(F + nnz + min_step)
    X = rng.standard_normal((nc, F)).astype(np.float32)
    H = build(swtcf, dst, src, nr, nc, r, c, min_step_nnz=min_step, group_blocks=G, unit_steps=unit_steps,
              phases=phases)
    Xd = torch.from_numpy(X).cuda()
    ws = torch.full((H.workspace_bytes(F) + 16,), 255, dtype=torch.uint8, device="cuda")
    Y = swtcf.hybrid_spmm(H, Xd, workspace=ws)
    want = scaled_product(oracle, dst, src, nr, X, r, c)
    got = Y.cpu().numpy()
    assert got.shape[0] >= nr
    e = rel_l2(got[:nr], want)
    assert e <= REL, f"rel-L2 {e}"
    assert not np.any(got[nr:])
    # the north star's bound against the TF32 CSR oracle over the values
    # fp32(r_i c_j), for the configurations' own values (sym-norm) over
    # enough features: the two rounding orders differ per term by a few
    # 1e-4, which averages out over a row's terms and the features, but not
    # on a dense rank-one block with signed scales and one feature (every
    # row then scales one cancelling sum: 1.3e-3 measured at 64 x 64, F = 1)
    if scale == "symnorm" and F >= 16:
        v = (r[dst.astype(np.int64)] * c[src.astype(np.int64)]).astype(np.float32)
        e_ns = rel_l2(got[:nr], oracle_product(oracle, dst, src, v, nr, X))
        assert e_ns <= NORTH_STAR, f"rel-L2 {e_ns} against the TF32 CSR oracle"
    Y0 = rng.standard_normal(got.shape).astype(np.float32)
    Yd = torch.from_numpy(Y0).cuda()
    swtcf.hybrid_spmm(H, Xd, Yd, accumulate=True, workspace=ws)
    e = rel_l2(Yd.cpu().numpy()[:nr], want + Y0[:nr])
    assert e <= REL, f"accumulate rel-L2 {e}"
    swtcf.hybrid_spmm(H, Xd, Y, workspace=ws)
    assert rel_l2(Y.cpu().numpy()[:nr], want) <= REL


def test_binary_symnorm_error_against_tf32_values(gpu, oracle):
    """How far the scaled form sits from the reference's numerics on a
    config-3-like graph: rounding TF32(c x) once instead of TF32(v) and
    TF32(x) moves the result by a few 1e-4, inside the north star's 1e-3,
    and far more than the fp32 summation order does."""
    from tcc_amd import swtcf

    nr = nc = 3000
    dst, src = random_coo(nr, nc, 300000, 17, True)
    r, c = scales(nr, nc, dst, src, "symnorm", 0)
    X = np.random.default_rng(3).standard_normal((nc, 128)).astype(np.float32)
    H = build(swtcf, dst, src, nr, nc, r, c, min_step_nnz=16)
    got = swtcf.hybrid_spmm(H, torch.from_numpy(X).cuda()).cpu().numpy()[:nr]
    v = (r[dst.astype(np.int64)] * c[src.astype(np.int64)]).astype(np.float32)
    e_values = rel_l2(got, oracle_product(oracle, dst, src, v, nr, X))
    e_scaled = rel_l2(got, scaled_product(oracle, dst, src, nr, X, r, c))
    print(f"symnorm: rel-L2 {e_values:.3e} vs TF32(v) TF32(x), {e_scaled:.3e} vs r TF32(c x)", flush=True)
    assert e_scaled <= REL
    assert 1e-5 < e_values <= NORTH_STAR


def zero_slot_rows(h, G, pair, half, col):
    """Rows that a value slot of 0 pointing at column `col` of block `half`
    of column pair `pair` reaches in some sub-step: 0 * X[col] enters their
    sums (lane l < 32 holds columns 0..7 of each block, l >= 32 columns
    8..15; slots 4*half + 2*(c%8 // 4) .. +1 cover column c)."""
    T = G // 2
    recs, gso, steps = h["tileMasks"], h["groupStepOffset"], h["stepCol"]
    lanes = np.arange(32) + 32 * (col // 8)
    k = 2 * half + (col % 8) // 4  # nibble of the lane
    rows = set()
    for g in range(h["num_groups"]):
        for q in range(int(gso[g]), int(gso[g + 1])):
            if steps[q] != pair:
                continue
            m = recs[q, :32 * G].reshape(64, T).astype(np.uint32)[lanes]
            ix = recs[q, 32 * G:].view("<u2").reshape(64, T).astype(np.uint32)[lanes]
            hit = np.zeros(m.shape, bool)
            for slot in (2 * k, 2 * k + 1):
                hit |= ((m >> slot) & 1 == 0) & ((ix >> (2 * slot)) & 3 == col % 4)
            for lane, t in zip(*np.nonzero(hit)):
                r = int(h["rowOrder"][16 * G * g + 32 * t + lane % 32])
                if r != 0xFFFFFFFF:
                    rows.add(r)
    return np.array(sorted(rows), np.int64)


@pytest.mark.parametrize("G", [8, 16])
def test_binary_inf_in_hub_column(gpu, oracle, G):
    """An Inf in a hub column's feature row: rows with an entry in that
    column get Inf (or NaN, where a second layer's empty slot also points
    at it); the other rows that a zero value slot pointing at that column
    reaches get NaN (0 * Inf inside the tiles' products, as inside the
    reference's 8x8 mma blocks); every other row stays finite and exact."""
    from tcc_amd import swtcf

    nr, nc, F = 400, 500, 8
    dst, src = random_coo(nr, nc, 20000, 23, True)
    H = build(swtcf, dst, src, nr, nc, None, None, min_step_nnz=8, group_blocks=G)
    h = H.to_host()
    c0 = int(h["hubColOrder"][0])  # the highest-degree column: rank 0, column 0 of block 0 of pair 0
    X = np.random.default_rng(5).standard_normal((nc, F)).astype(np.float32)
    X[c0, 0] = np.inf
    Y = swtcf.hybrid_spmm(H, torch.from_numpy(X).cuda()).cpu().numpy()[:nr]
    has = np.zeros(nr, bool)
    has[dst[src == c0].astype(np.int64)] = True
    exposed = np.zeros(nr, bool)
    exposed[zero_slot_rows(h, G, 0, 0, 0)] = True
    assert has.any() and (exposed & ~has).any() and (~(has | exposed)).any()
    assert not np.any(np.isfinite(Y[has, 0])) and not np.any(np.isneginf(Y[has, 0]))
    assert np.all(np.isnan(Y[exposed & ~has, 0]))
    assert np.all(np.isfinite(Y[~(has | exposed), 0]))
    X[c0, 0] = 0.0
    want = scaled_product(oracle, dst, src, nr, X, None, None)
    assert rel_l2(Y[:, 1:], want[:, 1:]) <= REL
    keep = ~(has | exposed)
    assert rel_l2(Y[keep, 0], want[keep, 0]) <= REL


def mixed_range_features(nc, F, seed):
    """N(0, 1) features with feature 0 at 1e-20 of that and feature 40 at
    1e30: with one power-of-two scale per 32-feature slice, the fp16 form of
    2^e x is inexact in every record of the slices holding them (feature 0
    falls below the fp16 grid, feature 40 above its range), so those slices
    take the bf16 halves and the others fp16."""
    X = np.random.default_rng(seed).standard_normal((nc, F)).astype(np.float32)
    X[:, 0] *= np.float32(1e-20)
    if F > 40:
        X[:, 40] *= np.float32(1e30)
    return X


def column_rel(Y, want, cols):
    return max(rel_l2(Y[:, j], want[:, j]) for j in cols)


@pytest.mark.parametrize("G, scale", [(16, "symnorm"), (8, "random"), (16, "none")])
def test_binary_half_and_bf16_records(gpu, oracle, G, scale):
    """The tiles multiply fp16 records where 2^e x is exact in fp16 and
    the bf16 halves elsewhere, in one product: the tiny feature 0, the huge
    feature 40 and every other feature each within 1e-5 of the scaled
    oracle, column by column."""
    from tcc_amd import swtcf

    nr, nc, F = 700, 900, 100
    dst, src = random_coo(nr, nc, 60000, 31, True)
    r, c = scales(nr, nc, dst, src, scale, 7)
    H = build(swtcf, dst, src, nr, nc, r, c, min_step_nnz=16, group_blocks=G)
    assert H.view.tiles.num_steps > 0
    X = mixed_range_features(nc, F, 3)
    want = scaled_product(oracle, dst, src, nr, X, r, c)
    # a workspace of NaN bytes: the bf16 steps' ring tail reads the zero pair in its bf16 form
    ws = torch.full((H.workspace_bytes(F) + 16,), 255, dtype=torch.uint8, device="cuda")
    Y = swtcf.hybrid_spmm(H, torch.from_numpy(X).cuda(), workspace=ws).cpu().numpy()[:nr].astype(np.float64)
    assert column_rel(Y, want, [0]) <= REL and column_rel(Y, want, [40]) <= REL
    assert column_rel(Y, want, [j for j in range(F) if j not in (0, 40)]) <= REL


@pytest.mark.parametrize("G", [8, 16])
def test_binary_tiles_alone(gpu, oracle, G):
    """tcc_hub_tiles_spmm on its own (its slice scales from its own pass
    over the hub rows, not the remainder's pack): Y += the product of the
    tile entries only, against the scaled oracle of exactly those entries,
    with the mixed-range features above."""
    from tcc_amd import swtcf

    nr, nc, F = 500, 700, 72
    dst, src = random_coo(nr, nc, 40000, 37, True)
    r, c = scales(nr, nc, dst, src, "symnorm", 1)
    H = build(swtcf, dst, src, nr, nc, r, c, min_step_nnz=16, group_blocks=G)
    lay = reference_binary_layout(dst, src, nr, nc, 16, G, DEFAULT_UNIT_STEPS, r, c)
    tile = ~lay["rest"]
    assert tile.any() and (~tile).any()
    X = mixed_range_features(nc, F, 4)
    Y0 = np.random.default_rng(9).standard_normal((H.out_rows, F)).astype(np.float32)
    ws = torch.full((H.workspace_bytes(F) + 16,), 255, dtype=torch.uint8, device="cuda")
    Y = swtcf.hub_tiles_spmm(H, torch.from_numpy(X).cuda(), torch.from_numpy(Y0).cuda(), workspace=ws).cpu().numpy()
    want = scaled_product(oracle, dst[tile], src[tile], nr, X, r, c) + Y0[:nr].astype(np.float64)
    got = Y[:nr].astype(np.float64)
    assert column_rel(got, want, [0]) <= REL and column_rel(got, want, [40]) <= REL
    assert column_rel(got, want, [j for j in range(F) if j not in (0, 40)]) <= REL


def test_binary_errors(gpu):
    from tcc_amd import _lib, swtcf

    one = dev_u32(np.array([0], np.uint32))
    with pytest.raises(_lib.TccError, match="groupBlocks 8 or 16"):
        swtcf.coo_to_hybrid_scaled(one, dev_u32(np.array([1], np.uint32)), 4, 4, group_blocks=4)
    with pytest.raises(_lib.TccError, match="duplicate"):
        swtcf.coo_to_hybrid_scaled(dev_u32(np.array([0, 1, 1], np.uint32)), dev_u32(np.array([2, 3, 3], np.uint32)),
                                   4, 4)
    with pytest.raises(_lib.TccError, match="out of range"):
        swtcf.coo_to_hybrid_scaled(dev_u32(np.array([0, 9], np.uint32)), dev_u32(np.array([0, 1], np.uint32)), 4, 4)
    with pytest.raises(ValueError, match="row_scale"):
        swtcf.coo_to_hybrid_scaled(one, one, 4, 4, row_scale=torch.ones(3, device="cuda"))
    H = swtcf.coo_to_hybrid_scaled(one, dev_u32(np.array([1], np.uint32)), 4, 4)
    small = torch.empty(8, dtype=torch.uint8, device="cuda")
    with pytest.raises(_lib.TccError, match="workspace"):
        swtcf.hybrid_spmm(H, torch.ones(4, 8, device="cuda"), workspace=small)
