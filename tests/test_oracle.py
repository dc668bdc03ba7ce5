"""Pins the CPU oracle (oracle/vbsr_oracle.c) without running the reference.

Each check is chosen so that a plausible mistake in the restatement fails it:
a wrong engine constant fails the standard's known answers; a wrong draw
order, size table, locality formula or value-draw count fails the reference
CSV fingerprints; a transposed block, wrong leading dimension, dropped block
or wrong accumulation precision fails brute force / closed forms.
"""

import json
import os

import numpy as np
import pytest

import oracle_ffi as o

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "fingerprints.json")


def engine64(seed):
    e = o.MT64()
    o.lib().orc_mt64_seed(e, seed)
    return e


def engine32(seed):
    e = o.MT32()
    o.lib().orc_mt32_seed(e, seed)
    return e


# ---- engines: C++ standard [rand.predef] known answers --------------------------------------------


def test_mt19937_64_known_answer():
    e = engine64(5489)
    for _ in range(9999):
        o.lib().orc_mt64_next(e)
    assert o.lib().orc_mt64_next(e) == 9981545732273789042


def test_mt19937_known_answer():
    e = engine32(5489)
    for _ in range(9999):
        o.lib().orc_mt32_next(e)
    assert o.lib().orc_mt32_next(e) == 4123659995


def test_uniform_float_closed_forms():
    f64 = o.lib().orc_uniform_pm1_from_u64
    f32 = o.lib().orc_uniform_pm1_from_u32
    assert f64(0) == -1.0
    assert f64(1 << 63) == 0.0
    assert f64(3 << 62) == 0.5
    # float(2^64 - 1) rounds to 2^64, so u == 1 maps to nextafter(1, 0) = 1 - 2^-24.
    assert f64((1 << 64) - 1) == np.float32(1.0 - 2.0 ** -23)
    assert f32(0) == -1.0
    assert f32(1 << 31) == 0.0
    assert f32((1 << 32) - 1) == np.float32(1.0 - 2.0 ** -23)
    # Below the rounding boundary u stays < 1: 2^64 - 2^40 is exact in float.
    assert f64((1 << 64) - (1 << 40)) == np.float32(2.0 * (1.0 - 2.0 ** -24) - 1.0)


# ---- generator: draw order pinned from the engine alone -------------------------------------------


def test_generator_draw_order_closed_form():
    """Uniform sizes draw nothing; one random column draw per row, then h*w values per block."""
    m = o.generate(1, 1, 1, "uniform", "random", seed=123)
    e = engine64(123)
    o.lib().orc_mt64_next(e)  # the column draw
    expected = [o.lib().orc_uniform_pm1_from_u64(o.lib().orc_mt64_next(e)) for _ in range(32 * 32)]
    np.testing.assert_array_equal(m.values, np.array(expected, dtype=np.float32))
    assert m.row_size.tolist() == [32] and m.col_size.tolist() == [32]


def test_generator_high_sizes_closed_form():
    """HighVariance: rows then columns, each {8..64}[e() % 8]."""
    m = o.generate(5, 7, 2, "high", "random", seed=9)
    e = engine64(9)
    sizes = [8 * (1 + o.lib().orc_mt64_next(e) % 8) for _ in range(12)]
    assert m.row_size.tolist() == sizes[:5]
    assert m.col_size.tolist() == sizes[5:]


@pytest.mark.parametrize("distribution,allowed", [
    ("uniform", {32}), ("low", {24, 32, 40}), ("high", set(range(8, 65, 8))), ("bimodal", {8, 16, 48, 64}),
    ("bimodal8or64", {8, 64}), ("tied8to64", set(range(8, 65, 8)))])
@pytest.mark.parametrize("locality", ["random", "local", "clamped"])
def test_generator_invariants(distribution, allowed, locality):
    R, C, d = 40, 37, 5
    m = o.generate(R, C, d, distribution, locality, seed=77)
    assert o.validate(m) == 0
    assert set(m.row_size.tolist()) <= allowed and set(m.col_size.tolist()) <= allowed
    if distribution == "tied8to64":
        assert m.col_size[:R].tolist() == m.row_size[:C].tolist()[:min(R, C)]
    assert np.all(np.diff(m.row_ptr) == d)
    for i in range(R):
        cols = m.block_col[m.row_ptr[i]:m.row_ptr[i + 1]]
        assert np.all(np.diff(cols) > 0)  # distinct and sorted
        if locality == "local":
            assert all(((c - i) % C) <= d or ((i - c) % C) <= d for c in cols)
        if locality == "clamped":
            centre = min(i, C - 1)
            assert np.all(cols >= max(0, centre - d)) and np.all(cols <= min(C - 1, centre + d))
    assert np.all(m.values >= -1.0) and np.all(m.values < 1.0)


def test_generator_rejects_bad_options():
    for args in [(0, 4, 1), (4, 0, 1), (4, 4, 0), (4, 4, 17), (4, 3, 4)]:
        with pytest.raises(ValueError):
            o.generate(*args)


def test_generator_deterministic():
    a = o.generate(50, 50, 4, "bimodal", "local", seed=5)
    b = o.generate(50, 50, 4, "bimodal", "local", seed=5)
    c = o.generate(50, 50, 4, "bimodal", "local", seed=6)
    for name in o.HostMatrix.FIELDS:
        np.testing.assert_array_equal(getattr(a, name), getattr(b, name))
    assert not np.array_equal(a.values, c.values)


def test_structure_only_path_matches_full_generator():
    for args in [(64, 64, 4, "high", "random", 3), (30, 41, 16, "bimodal", "local", 8),
                 (20, 20, 1, "low", "clamped", 2)]:
        full = o.generate(*args)
        structure = _structure(*args)
        for name in ("row_ptr", "block_col", "row_size", "col_size", "row_scalar_off", "col_scalar_off",
                     "value_off"):
            np.testing.assert_array_equal(getattr(full, name), structure[name])


def _structure(R, C, d, distribution, locality, seed):
    L = o.lib()
    L.orc_generate_structure.argtypes = L.orc_generate.argtypes
    m = o.OrcMatrix()
    assert L.orc_generate_structure(R, C, d, o.DISTRIBUTIONS[distribution], o.LOCALITIES[locality], seed,
                                    m) == 0
    try:
        nnzb = m.nnzb
        take = lambda p, n: np.ctypeslib.as_array(p, shape=(n,)).copy()  # noqa: E731
        out = {"row_ptr": take(m.row_ptr, R + 1), "block_col": take(m.block_col, nnzb),
               "row_size": take(m.row_size, R), "col_size": take(m.col_size, C),
               "row_scalar_off": take(m.row_scalar_off, R + 1), "col_scalar_off": take(m.col_scalar_off, C + 1),
               "value_off": take(m.value_off, nnzb + 1)}
        out["sum_hw"] = int(m.value_count)
        return out
    finally:
        L.orc_matrix_free(m)


# ---- generator: the reference's own published fingerprints ----------------------------------------


def _instances(block_rows=None):
    with open(GOLDEN) as handle:
        items = json.load(handle)["instances"]
    return [x for x in items if block_rows is None or x["block_rows"] == block_rows]


def test_fingerprint_fixture_covers_the_grid():
    items = _instances()
    assert len(items) == 192
    assert {x["distribution"] for x in items} == {"uniform", "low", "high", "bimodal"}
    assert {x["locality"] for x in items} == {"local", "random"}
    # Uniform blocks are 32x32 with no draw: S = rows * degree * 1024 exactly.
    for x in items:
        if x["distribution"] == "uniform":
            exact = x["block_rows"] * x["degree"] * 1024
            assert x["sum_hw_low"] <= exact <= x["sum_hw_high"]


@pytest.mark.parametrize("instance", _instances(1024), ids=lambda x: "{block_rows}-{degree}-{distribution}-"
                         "{locality}-s{seed}".format(**x))
def test_fingerprints_1024(instance):
    x = instance
    m = o.generate(x["block_rows"], x["block_cols"], x["degree"], x["distribution"], x["locality"], x["seed"])
    assert x["sum_hw_low"] <= m.sum_hw() <= x["sum_hw_high"]


@pytest.mark.slow
@pytest.mark.parametrize("instance", _instances(4096), ids=lambda x: "{block_rows}-{degree}-{distribution}-"
                         "{locality}-s{seed}".format(**x))
def test_fingerprints_4096(instance):
    x = instance
    s = _structure(x["block_rows"], x["block_cols"], x["degree"], x["distribution"], x["locality"], x["seed"])
    assert x["sum_hw_low"] <= s["sum_hw"] <= x["sum_hw_high"]


# ---- validation: reference negative tests + one case per rule ---------------------------------------


def _valid():
    return o.generate(4, 4, 2, "high", "local", seed=1)


def mutations():
    """(description, mutate(matrix), expected rule code)."""
    def setf(name, index, value):
        def f(m):
            getattr(m, name)[index] = value
        return f

    def extend(name, value):
        def f(m):
            setattr(m, name, np.append(getattr(m, name), value).astype(getattr(m, name).dtype))
        return f

    def shrink(name):
        def f(m):
            setattr(m, name, getattr(m, name)[:-1].copy())
        return f

    def both(*fs):
        def f(m):
            for g in fs:
                g(m)
        return f

    return [
        ("row_ptr.back()++ (test_main.cpp:124)", lambda m: m.row_ptr.__setitem__(-1, m.row_ptr[-1] + 1), 4),
        ("row_size[0]=7 (test_main.cpp:129)", setf("row_size", 0, 7), 6),
        ("block_rows 0", lambda m: setattr(m, "block_rows", 0), 1),
        ("block_cols -1", lambda m: setattr(m, "block_cols", -1), 1),
        ("row_ptr too long", extend("row_ptr", 8), 2),
        ("row_size too short", shrink("row_size"), 2),
        ("col_size too long", extend("col_size", 8), 2),
        ("row_scalar_off too short", shrink("row_scalar_off"), 3),
        ("col_scalar_off too long", extend("col_scalar_off", 999), 3),
        ("row_ptr[0] != 0", setf("row_ptr", 0, 1), 4),
        ("value_off too short", shrink("value_off"), 5),
        ("value_off[0] != 0", setf("value_off", 0, 1), 5),
        ("values too short", shrink("values"), 5),
        ("row_ptr not monotone", setf("row_ptr", 2, 0), 6),
        ("row_size 72", setf("row_size", 1, 72), 6),
        ("row_size 0", setf("row_size", 1, 0), 6),
        ("row offsets inconsistent", setf("row_scalar_off", 2, 7), 6),
        ("col_size 12", setf("col_size", 2, 12), 7),
        ("col offsets inconsistent", setf("col_scalar_off", 1, 3), 7),
        ("block column -1", setf("block_col", 0, -1), 8),
        ("block column == block_cols", setf("block_col", 3, 4), 8),
        ("payload mismatch", both(setf("value_off", 1, 5)), 9),
    ]


@pytest.mark.parametrize("case", mutations(), ids=lambda c: c[0])
def test_validate_rejects(case):
    _, mutate, rule = case
    m = _valid()
    assert o.validate(m) == 0
    mutate(m)
    assert o.validate(m) == rule


def test_validate_accepts_what_the_reference_does_not_check():
    """vbsr.cpp:29-82 checks neither scalar offset bases, column order, duplicates nor empty rows."""
    m = _valid()
    m.row_scalar_off = m.row_scalar_off + 5
    m.col_scalar_off = m.col_scalar_off + 3
    assert o.validate(m) == 0
    m = _valid()
    m.block_col[0], m.block_col[1] = m.block_col[1], m.block_col[0]  # unsorted (payload sizes may differ)
    h = int(m.row_size[0])
    m.value_off[1] = h * int(m.col_size[m.block_col[0]])
    assert o.validate(m) == 0
    m = _rows_with_empty()
    assert o.validate(m) == 0


def _rows_with_empty():
    """Three block rows (h = 8, 16, 8), the middle one empty; block column 1 twice in row 0."""
    row_size = np.array([8, 16, 8])
    col_size = np.array([8, 24, 16])
    block_col = np.array([1, 1, 0, 2])
    row_ptr = np.array([0, 2, 2, 4])
    owners = [0, 0, 2, 2]
    counts = [row_size[r] * col_size[c] for r, c in zip(owners, block_col)]
    value_off = np.concatenate([[0], np.cumsum(counts)])
    rng = np.random.default_rng(4)
    return o.HostMatrix(3, 3, row_ptr=row_ptr, block_col=block_col, row_size=row_size, col_size=col_size,
                        row_scalar_off=np.concatenate([[0], np.cumsum(row_size)]),
                        col_scalar_off=np.concatenate([[0], np.cumsum(col_size)]), value_off=value_off,
                        values=rng.uniform(-1, 1, value_off[-1]).astype(np.float32))


# ---- products: brute force and closed forms -------------------------------------------------------


def _dense_product(m, b, rhs):
    return (m.dense() @ b.reshape(rhs, m.scalar_cols).T.astype(np.float64)).T.reshape(-1)


@pytest.mark.parametrize("rhs", [8, 16, 32, 64])
@pytest.mark.parametrize("args", [(9, 17, 4, "high", "local", 11), (6, 5, 3, "bimodal", "random", 12),
                                  (7, 7, 1, "low", "clamped", 13), (3, 11, 8, "tied8to64", "random", 14)])
def test_cpu_reference_brute_force(args, rhs):
    m = o.generate(*args)
    b = o.make_random_input(m.scalar_cols * rhs, args[-1])
    got = o.cpu_reference(m, b, rhs)
    want = _dense_product(m, b, rhs)
    bound = o.abs_product_sum(m, b, rhs)
    # Each block's dot is rounded once to float and blocks are summed in float.
    assert np.all(np.abs(got - want) <= 4 * np.finfo(np.float32).eps * np.maximum(bound, 1e-30) + 1e-30)
    fm = o.fmaf_order(m, b, rhs)
    assert np.all(np.abs(fm - want) <= 1e-5 * np.max(bound))
    # The bound is the dense product of |A| and |B|.
    np.testing.assert_allclose(bound, (np.abs(m.dense()) @ np.abs(b.reshape(rhs, -1)).T.astype(np.float64)).T
                               .reshape(-1), rtol=1e-12)


def test_cpu_reference_empty_and_duplicate_blocks():
    m = _rows_with_empty()
    rhs = 8
    b = o.make_random_input(m.scalar_cols * rhs, 3)
    got = o.cpu_reference(m, b, rhs).reshape(rhs, m.scalar_rows)
    want = _dense_product(m, b, rhs).reshape(rhs, m.scalar_rows)
    assert np.all(got[:, 8:24] == 0.0)  # the empty row stays zero
    np.testing.assert_allclose(got, want, rtol=1e-6, atol=1e-6)
    np.testing.assert_allclose(o.fmaf_order(m, b, rhs).reshape(rhs, -1), want, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("threads", [1, 3, 8])
def test_threaded_cpu_reference_is_bit_identical(threads):
    """The multi-core baseline keeps each row's arithmetic, so its bits equal the serial oracle's."""
    for args, rhs in (((300, 300, 8, "high", "random", 5), 32), ((9, 17, 4, "bimodal", "local", 6), 8)):
        m = o.generate(*args)
        b = o.make_random_input(m.scalar_cols * rhs, args[-1])
        np.testing.assert_array_equal(o.cpu_reference_threads(m, b, rhs, threads), o.cpu_reference(m, b, rhs))
        np.testing.assert_array_equal(o.abs_product_sum_threads(m, b, rhs, threads), o.abs_product_sum(m, b, rhs))
    m = _rows_with_empty()
    b = o.make_random_input(m.scalar_cols * 8, 3)
    np.testing.assert_array_equal(o.cpu_reference_threads(m, b, 8, threads), o.cpu_reference(m, b, 8))
    np.testing.assert_array_equal(o.abs_product_sum_threads(m, b, 8, threads), o.abs_product_sum(m, b, 8))
    with pytest.raises(ValueError):
        o.cpu_reference_threads(m, b[:-1], 8, threads)
    with pytest.raises(ValueError):
        o.cpu_reference_threads(m, b, 8, 0)


def test_identity_blocks_copy_b():
    """Degree 1, block column i for row i, A_i = I: C equals B exactly."""
    sizes = np.array([8, 24, 64, 16])
    values = np.concatenate([np.eye(s, dtype=np.float32).reshape(-1) for s in sizes])
    value_off = np.concatenate([[0], np.cumsum(sizes * sizes)])
    offs = np.concatenate([[0], np.cumsum(sizes)])
    m = o.HostMatrix(4, 4, row_ptr=np.arange(5), block_col=np.arange(4), row_size=sizes, col_size=sizes,
                     row_scalar_off=offs, col_scalar_off=offs, value_off=value_off, values=values)
    assert o.validate(m) == 0
    b = o.make_random_input(m.scalar_cols * 16, 21)
    np.testing.assert_array_equal(o.cpu_reference(m, b, 16), b)
    np.testing.assert_array_equal(o.fmaf_order(m, b, 16), b)


def test_unit_vector_b_extracts_columns():
    m = o.generate(6, 9, 3, "high", "random", seed=31)
    K, M = m.scalar_cols, m.scalar_rows
    rhs = 8
    cols = [0, 5, K // 2, K - 1, 17, 100 % K, 3, K - 8]
    b = np.zeros(K * rhs, dtype=np.float32)
    for n, j in enumerate(cols):
        b[n * K + j] = 1.0
    dense = m.dense()
    got = o.cpu_reference(m, b, rhs).reshape(rhs, M)
    for n, j in enumerate(cols):
        np.testing.assert_array_equal(got[n], dense[:, j].astype(np.float32))
    got = o.fmaf_order(m, b, rhs).reshape(rhs, M)
    for n, j in enumerate(cols):
        np.testing.assert_array_equal(got[n], dense[:, j].astype(np.float32))


def test_degree_one_is_a_batched_gemm_and_linear():
    m = o.generate(12, 12, 1, "bimodal", "random", seed=41)
    rhs = 32
    b1 = o.make_random_input(m.scalar_cols * rhs, 1)
    b2 = o.make_random_input(m.scalar_cols * rhs, 2)
    c1, c2 = o.cpu_reference(m, b1, rhs), o.cpu_reference(m, b2, rhs)
    c12 = o.cpu_reference(m, b1 + b2, rhs)
    bound = o.abs_product_sum(m, np.abs(b1) + np.abs(b2), rhs)
    assert np.all(np.abs(c12 - (c1.astype(np.float64) + c2)) <= 4e-7 * bound + 1e-30)
    B = b1.reshape(rhs, m.scalar_cols).T.astype(np.float64)
    C = c1.reshape(rhs, m.scalar_rows).T
    for i in range(m.block_rows):
        blk = m.row_ptr[i]
        h, w = int(m.row_size[i]), int(m.col_size[m.block_col[blk]])
        A = m.values[m.value_off[blk]:m.value_off[blk + 1]].reshape(w, h).T.astype(np.float64)
        c0 = int(m.col_scalar_off[m.block_col[blk]])
        r0 = int(m.row_scalar_off[i])
        want = (A @ B[c0:c0 + w]).astype(np.float32)
        np.testing.assert_allclose(C[r0:r0 + h], want, rtol=0, atol=2 * np.finfo(np.float32).eps * 64)


def test_integer_inputs_are_exact_in_both_orders():
    """Small integers make every product and sum exact: both orders equal the dense product bit for bit."""
    m = o.generate(8, 8, 4, "high", "random", seed=51)
    m.values = np.round(m.values * 4).astype(np.float32)
    rhs = 16
    b = np.round(o.make_random_input(m.scalar_cols * rhs, 5) * 4).astype(np.float32)
    want = _dense_product(m, b, rhs).astype(np.float32)
    np.testing.assert_array_equal(o.cpu_reference(m, b, rhs), want)
    np.testing.assert_array_equal(o.fmaf_order(m, b, rhs), want)


def test_b_size_is_checked():
    m = _valid()
    with pytest.raises(ValueError):
        o.cpu_reference(m, np.zeros(m.scalar_cols * 8 - 1, np.float32), 8)


# ---- the reference test's B generator ---------------------------------------------------------------


def test_make_random_input_stream():
    b = o.make_random_input(700, 1234)
    e = engine32(1234)
    expected = [o.lib().orc_uniform_pm1_from_u32(o.lib().orc_mt32_next(e)) for _ in range(700)]
    np.testing.assert_array_equal(b, np.array(expected, dtype=np.float32))
    # std::mt19937{unsigned(seed)} truncates the seed to 32 bits.
    np.testing.assert_array_equal(o.make_random_input(10, (1 << 32) + 1234), b[:10])


def test_useful_flops():
    m = o.generate(10, 10, 3, "high", "random", seed=2)
    assert o.useful_flops(m, 32) == 2 * 32 * m.sum_hw()


# ---- the fmaf order itself: inputs whose bits depend on the order and on fusion ----------------------------

BIG = np.float32(2.0 ** 24)


def _one_row(blocks, col_widths, h=8):
    """One block row of height h whose blocks (h x w value arrays, column-major) sit in block columns 0, 1, ...
    of widths col_widths."""
    values = np.concatenate([np.asarray(v, np.float32).reshape(-1, order="F") for v in blocks])
    sizes = [np.asarray(v).size for v in blocks]
    col_widths = np.asarray(col_widths)
    return o.HostMatrix(1, len(col_widths), row_ptr=[0, len(blocks)], block_col=np.arange(len(blocks)),
                        row_size=[h], col_size=col_widths, row_scalar_off=[0, h],
                        col_scalar_off=np.concatenate([[0], np.cumsum(col_widths)]),
                        value_off=np.concatenate([[0], np.cumsum(sizes)]), values=values)


def order_probes():
    """(name, matrix, B, rhs, fmaf-order C, cpu_reference C): closed forms whose bits differ by summation
    order or by fusion, so that an emulation (or kernel) with k reversed, blocks reversed or multiply and
    add rounded separately gives other bits.  2^24 + 1 rounds to 2^24 (tie to even) while 1 - 2^24 is exact;
    (1 + 2^-12)^2 = 1 + 2^-11 + 2^-24 is exact only inside a fused multiply-add."""
    probes = []
    rhs = 8
    # k order within a block: rows 0-2 of one 8 x 8 block, B = 1.
    a = np.zeros((8, 8), np.float32)
    a[0, :3] = [BIG, 1, -BIG]
    a[1, :3] = [-BIG, 1, BIG]
    a[2, :3] = [1, BIG, -BIG]
    m = _one_row([a], [8])
    b = np.ones(8 * rhs, np.float32)
    fm = np.zeros((rhs, 8), np.float32)
    fm[:, 1] = 1  # in k order: 0, 1, 0; reversed: 1, 0, 1
    ref = np.zeros((rhs, 8), np.float32)
    ref[:, :3] = 1  # each block's sum is exact in double
    probes.append(("k-order", m, b, rhs, fm.reshape(-1), ref.reshape(-1)))
    # Block order: three 8 x 8 blocks, the values in column 0 of each.
    blocks = [np.zeros((8, 8), np.float32) for _ in range(3)]
    for row, vals in ((0, (BIG, 1, -BIG)), (1, (-BIG, 1, BIG))):
        for blk, v in zip(blocks, vals):
            blk[row, 0] = v
    m = _one_row(blocks, [8, 8, 8])
    b = np.ones(24 * rhs, np.float32)
    fm = np.zeros((rhs, 8), np.float32)
    fm[:, 1] = 1  # blocks in row_ptr order: 0, 1; reversed: 1, 0
    probes.append(("block-order", m, b, rhs, fm.reshape(-1), fm.reshape(-1).copy()))
    # Fusion: A row 0 = [-(1 + 2^-11), 1 + 2^-12], B column = [1, 1 + 2^-12, 0, ...].
    a = np.zeros((8, 8), np.float32)
    a[0, :2] = [-(1 + 2.0 ** -11), 1 + 2.0 ** -12]
    m = _one_row([a], [8])
    col = np.zeros(8, np.float32)
    col[:2] = [1, 1 + 2.0 ** -12]
    b = np.tile(col, rhs)
    fm = np.zeros((rhs, 8), np.float32)
    fm[:, 0] = 2.0 ** -24  # fused, in order; unfused or reversed: 0
    probes.append(("fusion", m, b, rhs, fm.reshape(-1), fm.reshape(-1).copy()))
    return probes


@pytest.mark.parametrize("probe", order_probes(), ids=lambda p: p[0])
def test_fmaf_order_is_pinned_by_order_and_fusion_sensitive_closed_forms(probe):
    _, m, b, rhs, want_fmaf, want_reference = probe
    assert o.validate(m) == 0
    np.testing.assert_array_equal(o.fmaf_order(m, b, rhs), want_fmaf)
    np.testing.assert_array_equal(o.cpu_reference(m, b, rhs), want_reference)


def test_order_probes_tell_the_alternatives_apart():
    """The probes' expected values are not what the plausible mistakes give: computed here in numpy with k
    reversed, blocks reversed, and the multiply rounded before the add."""
    f32 = np.float32

    def chain(terms, fused=True):
        acc = f32(0)
        for x, y in terms:
            acc = f32(np.float64(x) * np.float64(y) + np.float64(acc)) if fused else f32(f32(x * y) + acc)
        return acc

    row0 = [(BIG, 1), (f32(1), 1), (-BIG, 1)]
    assert chain(row0) == 0 and chain(row0[::-1]) == 1
    fuse = [(f32(-(1 + 2.0 ** -11)), f32(1)), (f32(1 + 2.0 ** -12), f32(1 + 2.0 ** -12))]
    assert chain(fuse) == f32(2.0 ** -24)
    assert chain(fuse, fused=False) == 0 and chain(fuse[::-1]) == 0
