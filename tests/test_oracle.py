"""Pins the CPU oracle (oracle/rns8_oracle.c) before it is trusted as the
parity checker for the GPU path.

Three kinds of evidence, none of which retypes the oracle's formulas:
  * the reference's own known-answer tests (tests/golden/reference_kats.json,
    transcribed from the reference test sources named there);
  * the reference's header-only reducers compiled in place into
    oracle/_ref/libref.so (build container only; those tests skip elsewhere);
  * mathematics: Python big-integer products, brute-force sums and the Chinese
    remainder property.
"""
from __future__ import annotations

import ctypes as C
import json
import math
from pathlib import Path

import numpy as np
import pytest

import oracle

KATS = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kats.json").read_text())
LADDER = KATS["ladder"]["moduli"]
SUCCESS, INVALID_ARGUMENT, RANGE_ERROR = 0, 1, 5


def centered(x: int, m: int) -> int:
    """((x + floor(m/2)) mod m) - floor(m/2): the reference centering rule
    (cpu_reference.cpp:26-32), used here only to build residue inputs."""
    h = m // 2
    return (x + h) % m - h


def product(prefix: int) -> int:
    return math.prod(LADDER[:prefix])


def residues_for(x: int, prefix: int) -> np.ndarray:
    return np.array([centered(x, LADDER[p]) for p in range(prefix)], dtype=np.int8)


def _p(a):
    return a.ctypes.data_as(C.c_void_p)


def parse_value(text: str, prefix: int) -> int:
    P = product(prefix)
    table = {"P-1": P - 1, "P/2": P // 2, "P/2-1": P // 2 - 1, "P-2^63": P - (1 << 63)}
    if text in table:
        return table[text]
    if text.startswith("-(P") and text.endswith("/2)"):
        return -(product(int(text[3:-3])) // 2)
    return int(text)


# ---- ladder and prefix products -----------------------------------------------------


def test_ladder_matches_reference_kat():
    L = oracle.lib()
    assert [L.orc_modulus(i) for i in range(28)] == LADDER
    assert oracle.LADDER == LADDER
    assert L.orc_ladder_pairwise_coprime() == 1
    assert all(math.gcd(a, b) == 1 for i, a in enumerate(LADDER) for b in LADDER[i + 1:])


def _range_words(x: int) -> np.ndarray:
    return np.array([(x >> (64 * i)) & ((1 << 64) - 1) for i in range(4)], dtype=np.uint64)


def test_prefix_products_and_required_prefix():
    """test_moduli.cpp:21-39: product(prefix) and required_prefix(P-1) == prefix,
    required_prefix(P) == prefix + 1 (0 past the maximum prefix)."""
    L = oracle.lib()
    for prefix in range(1, 21):
        P = product(prefix)
        assert oracle.modulus_product(prefix) == P
        assert L.orc_required_prefix_for_range(_p(_range_words(P - 1))) == prefix
        assert L.orc_required_prefix_for_range(_p(_range_words(P))) == (prefix + 1 if prefix < 20 else 0)


def test_prefix9_contract():
    """test_moduli.cpp:41-55: P_9 > 2^64 > P_8; range 2^64 - 1 and 2^64 need prefix 9."""
    L = oracle.lib()
    assert product(9) > 1 << 64 > product(8)
    assert L.orc_required_prefix_for_range(_p(_range_words((1 << 64) - 1))) == 9
    assert L.orc_required_prefix_for_range(_p(_range_words(1 << 64))) == 9


def test_prefix_range_bits():
    L = oracle.lib()
    kat = KATS["prefix_range_bits"]
    for prefix, bits in kat["table"]:
        got = L.orc_prefix_range_bits(prefix)
        assert abs(got - bits) <= kat["margin"]
        assert abs(got - math.log2(product(prefix))) < 1e-9
    for prefix in kat["zero_for"]:
        assert L.orc_prefix_range_bits(prefix) == 0.0


# ---- residues and reducers ------------------------------------------------------------


def test_centered_residue_kats():
    L = oracle.lib()
    for x, m, want in KATS["centered_residues"]["cases"]:
        assert L.orc_centered_i64(x, m) == want
    for r, m, want in KATS["centered_residues"]["canonical_from_centered"]:
        assert L.orc_canonical_from_centered(r, m) == want
    # int64 min reduces into the centered range (test_residues.cpp:33-38)
    r = L.orc_centered_i64(-(1 << 63), 251)
    assert -125 <= r <= 125 and r == centered(-(1 << 63), 251)


def test_centered_residues_closed_form_all_moduli():
    L = oracle.lib()
    rng = np.random.default_rng(5)
    values = [0, 1, -1, (1 << 63) - 1, -(1 << 63), 127, 128, -128, -129] + \
        [int(v) for v in rng.integers(-(1 << 63), (1 << 63) - 1, size=300, dtype=np.int64)]
    uvalues = [0, 1, (1 << 64) - 1, 1 << 63, 255, 256] + \
        [int(v) for v in rng.integers(0, (1 << 64) - 1, size=300, dtype=np.uint64)]
    for m in range(2, 257):
        for x in values:
            assert L.orc_centered_i64(x, m) == centered(x, m)
        for x in uvalues:
            assert L.orc_centered_u64(x, m) == centered(x, m)


def test_reducer_kat_values_all_ladder_moduli():
    """test_residues.cpp:40-78: the int32 reducer on the boundary values."""
    L = oracle.lib()
    R = oracle.ref()
    for m in LADDER:
        for v in KATS["reducer_values"]["values"]:
            assert L.orc_reduce_to_centered(v, m) == centered(v, m)
            if R is not None:
                assert R.ref_reduce_to_centered_i32(v, m) == centered(v, m)
                assert R.ref_reduce_to_centered_accelerator_i32(v, m) == centered(v, m)


def _ref_or_skip():
    """The reference's compiled reducers, loaded when a test runs (never at
    collection, so a run that selects no such test never maps them)."""
    R = oracle.ref()
    if R is None:
        pytest.skip("oracle/_ref is built only where the reference sources exist")
    return R


def test_reducer_matches_reference_header_sampled():
    """Oracle int32 reduction against the reference's finite_u8_reducer.hpp on
    every ladder modulus: 2^18 values around zero plus 2^18 random int32."""
    L = oracle.lib()
    R = _ref_or_skip()
    rng = np.random.default_rng(11)
    vals = np.concatenate([np.arange(-(1 << 17), 1 << 17, dtype=np.int32),
                           rng.integers(-(1 << 31), (1 << 31) - 1, size=1 << 18, dtype=np.int64).astype(np.int32),
                           np.array([-(1 << 31), (1 << 31) - 1], dtype=np.int32)])
    want = np.empty(vals.size, dtype=np.int8)
    for m in LADDER:
        R.ref_reduce_many(_p(vals), vals.size, m, _p(want))
        got = np.array([L.orc_reduce_to_centered(int(v), m) for v in vals[::97]], dtype=np.int8)
        assert np.array_equal(got, want[::97])
        # closed form on the full sample (vectorized)
        h = m // 2
        assert np.array_equal(((vals.astype(np.int64) + h) % m - h).astype(np.int8), want)


def test_finite_byte_maps_match_reference_header():
    L = oracle.lib()
    R = _ref_or_skip()
    for m in list(range(2, 257)):
        for b in range(256):
            if b < m:
                assert R.ref_center_u8(b, m) == centered(b, m)
        for r in range(-128, 128):
            if -(m // 2) <= r <= m - 1 - m // 2:
                assert L.orc_canonical_from_centered(r, m) == R.ref_canonical_from_centered(r, m) == r % m


# ---- ring GEMM and residue dot -------------------------------------------------------


def test_ring_gemm_kat():
    """test_ring_gemm.cpp:27-45 against a brute-force big-integer sum."""
    g = KATS["ring_gemm"]
    A = np.array(g["A"], dtype=np.int8).reshape(g["m"], g["k"])
    B = np.array(g["B"], dtype=np.int8).reshape(g["k"], g["n"])
    exact = A.astype(np.int64) @ B.astype(np.int64)
    for m in g["moduli"]:
        got = oracle.ring_gemm(A, B, m)
        assert np.array_equal(got, np.vectorize(lambda x: centered(int(x), m))(exact).astype(np.int8))


def test_ring_gemm_safe_k_block():
    """test_ring_gemm.cpp:47-53: K = 65537 of 127*127 splits the int32 block."""
    c = KATS["ring_gemm"]["safe_block_case"]
    A = np.full((1, c["k"]), c["value"], dtype=np.int8)
    B = np.full((c["k"], 1), c["value"], dtype=np.int8)
    got = oracle.ring_gemm(A, B, c["modulus"])
    assert got[0, 0] == centered(c["value"] * c["value"] * c["k"], c["modulus"])


def test_residue_dot_k_edges():
    """test_residue_dot.cpp:9-31: every safe K block boundary, 20 moduli,
    constant and alternating operands; oracle and (where built) the reference
    header against the exact int64 sum."""
    L = oracle.lib()
    R = oracle.ref()
    d = KATS["residue_dot"]
    for k in d["k"]:
        for m in LADDER[:20]:
            lo = -(m // 2)
            for alternating in (False, True):
                a = np.full(k, lo, dtype=np.int8)
                b = np.full(k * d["b_stride"], d["fill"], dtype=np.int8)
                col = np.full(k, lo, dtype=np.int8)
                if alternating:
                    col[1::2] = d["alternating_value"]
                b[::d["b_stride"]] = col
                exact = int(np.dot(a.astype(np.int64), col.astype(np.int64)))
                want = centered(exact, m)
                assert L.orc_centered_residue_dot(_p(a), _p(b), k, d["b_stride"], m) == want
                if R is not None:
                    assert R.ref_centered_residue_dot(_p(a), _p(b), k, d["b_stride"], m) == want


# ---- CRT reconstruction ----------------------------------------------------------------


def _rec_signed(res, prefix, bound, sentinel=123):
    out = C.c_int64(sentinel)
    st = oracle.lib().orc_reconstruct_signed(_p(res), prefix, bound, C.byref(out))
    return st, out.value


def _rec_unsigned(res, prefix, bound, sentinel=456):
    out = C.c_uint64(sentinel)
    st = oracle.lib().orc_reconstruct_unsigned(_p(res), prefix, bound, C.byref(out))
    return st, out.value


def _rec_canonical(res, prefix):
    out = np.zeros(4, dtype=np.uint64)
    oracle.lib().orc_reconstruct_canonical(_p(res), prefix, _p(out))
    return sum(int(w) << (64 * i) for i, w in enumerate(out))


def test_crt_signed_kats():
    for c in KATS["crt"]["signed"]:
        prefix = c["prefix"]
        res = residues_for(parse_value(c["value"], prefix), prefix)
        st, out = _rec_signed(res, prefix, int(c["bound"]))
        assert st == c["status"], c
        assert out == (int(c["out"]) if st == SUCCESS else 123), c  # output untouched on error


def test_crt_unsigned_kats():
    for c in KATS["crt"]["unsigned"]:
        prefix = c["prefix"]
        res = residues_for(parse_value(c["value"], prefix), prefix)
        st, out = _rec_unsigned(res, prefix, int(c["bound"]))
        assert st == c["status"], c
        assert out == (int(c["out"]) if st == SUCCESS else 456), c


def test_crt_prefix2_threshold_constants():
    assert product(2) == KATS["crt"]["prefix2_product"]
    assert (product(2) + 1) // 2 == KATS["crt"]["prefix2_threshold"]


def test_crt_canonical_across_prefixes():
    """test_crt.cpp:44-59 and test_hip_arithmetic_host.cpp:30-54: canonical
    reconstruction returns the unique representative in [0, P)."""
    for prefix in range(1, 21):
        P = product(prefix)
        vals = [0, 1, 2, P // 2 - 1, P // 2, P - 1]
        if prefix >= 9:
            vals += [(1 << 64) - 1, P - (1 << 63)]
        for x in vals:
            assert _rec_canonical(residues_for(x, prefix), prefix) == x


def test_crt_random_chinese_remainder_property():
    rng = np.random.default_rng(3)
    for prefix in range(1, 21):
        P = product(prefix)
        for _ in range(40):
            x = int(rng.integers(0, 1 << 62)) * int(rng.integers(0, 1 << 62)) * int(rng.integers(1, 1 << 40)) % P
            assert _rec_canonical(residues_for(x, prefix), prefix) == x


def test_crt_malformed_prefix():
    res = np.zeros(21, dtype=np.int8)
    assert _rec_signed(res, 0, 1)[0] == INVALID_ARGUMENT
    assert _rec_signed(res, 21, 1)[0] == INVALID_ARGUMENT
    assert _rec_unsigned(res, 0, 1)[0] == INVALID_ARGUMENT


def test_audit_f01_prefix8_value_two():
    """docs/audit-2026-10-06.md: x = 2 at prefix 8 must reconstruct to 2 (a
    wrapped weighted-CRT gave 4558134011519499778)."""
    a = KATS["audit_f01"]
    res = residues_for(a["value"], a["prefix"])
    # bounds the prefix admits (2 * bound < P_8 for signed, bound < P_8 unsigned)
    assert _rec_signed(res, a["prefix"], 1 << 62) == (SUCCESS, 2)
    assert _rec_unsigned(res, a["prefix"], 1 << 63) == (SUCCESS, 2)
    assert _rec_canonical(res, a["prefix"]) == 2 != a["wrapped_wrong_answer"]


def _limbs_of(x: int, limbs: int) -> list[int]:
    x %= 1 << (64 * limbs)
    return [(x >> (64 * i)) & ((1 << 64) - 1) for i in range(limbs)]


def test_exact_wide_limb_kats():
    """test_exact_wide_limb_boundary_cases.inc: fixed-width two's complement /
    unsigned limbs, RANGE_ERROR leaves the output untouched."""
    L = oracle.lib()
    sentinel = 0xA5A5A5A5A5A5A5A5
    for signed in (True, False):
        fn = L.orc_exact_wide_signed_limbs if signed else L.orc_exact_wide_unsigned_limbs
        for c in KATS["exact_wide_limbs"]["signed" if signed else "unsigned"]:
            prefix, limbs = c["prefix"], c["limbs"]
            x = parse_value(c["value"], prefix)
            out = np.full(32, sentinel, dtype=np.uint64)
            st = fn(_p(residues_for(x, prefix)), prefix, _p(out), limbs)
            assert st == c["status"], c
            if st == SUCCESS:
                assert [int(w) for w in out[:limbs]] == _limbs_of(x, limbs), c
            else:
                assert all(int(w) == sentinel for w in out), c


# ---- pack ---------------------------------------------------------------------------------


def test_pack_tails_all_boundaries():
    """test_hip_arithmetic_host.cpp:56-78: boundary values over row lengths
    255..259 / 4095 / 4096 and prefixes 1, 8, 9, 20."""
    t = KATS["pack_tails"]
    pattern = [int(v) for v in t["boundaries"]]
    for cells in t["cells"]:
        src = np.array([pattern[c % len(pattern)] for c in range(cells)], dtype=np.int64).reshape(1, cells)
        for prefix in t["prefixes"]:
            got = oracle.pack_i64(src, prefix)
            for p in range(prefix):
                want = np.array([centered(int(v), LADDER[p]) for v in src[0]], dtype=np.int8)
                assert np.array_equal(got[p, 0], want)


def test_pack_u64_and_finite_closed_form():
    rng = np.random.default_rng(9)
    U = rng.integers(0, (1 << 64) - 1, size=(7, 33), dtype=np.uint64)
    U[0, :3] = [0, (1 << 64) - 1, 1 << 63]
    got = oracle.pack_u64(U, 20)
    for p in range(20):
        want = np.vectorize(lambda v: centered(int(v), LADDER[p]))(U.astype(object)).astype(np.int8)
        assert np.array_equal(got[p], want)
    for m in (2, 3, 7, 251, 255, 256):
        X = rng.integers(0, m, size=(5, 40), dtype=np.uint8) if m < 256 else \
            rng.integers(0, 256, size=(5, 40), dtype=np.uint8)
        got = oracle.pack_finite_u8(X, m)
        assert np.array_equal(got, ((X.astype(np.int64) + m // 2) % m - m // 2).astype(np.int8))


# ---- end to end ---------------------------------------------------------------------------


def test_example_bounded_i64():
    e = KATS["example_bounded_i64"]
    A = np.array(e["A"], dtype=np.int64).reshape(e["m"], e["k"])
    B = np.array(e["B"], dtype=np.int64).reshape(e["k"], e["n"])
    prefix = C.c_uint32(0)
    st = oracle.lib().orc_select_prefix(1, 1, e["bound"], e["k"], 0, 0, 0, 0, C.byref(prefix))
    assert st == SUCCESS
    st, got = oracle.gemm_i64(A, B, prefix.value, e["bound"])
    assert st == SUCCESS and got.reshape(-1).tolist() == e["C"]


@pytest.mark.parametrize("m,n,k", [(1, 1, 1), (3, 5, 7), (17, 9, 31), (8, 8, 65537)])
def test_gemm_i64_brute_force(m, n, k):
    rng = np.random.default_rng(m * 1000 + n * 10 + k)
    bits = 20 if k < 1000 else 12
    A = rng.integers(-(1 << bits), 1 << bits, size=(m, k), dtype=np.int64)
    B = rng.integers(-(1 << bits), 1 << bits, size=(k, n), dtype=np.int64)
    exact = A.astype(object) @ B.astype(object)
    bound = max(1, max(abs(int(v)) for v in exact.reshape(-1)))
    prefix = next(p for p in range(1, 21) if product(p) > 2 * bound)
    st, got = oracle.gemm_i64(A, B, prefix, bound)
    assert st == SUCCESS
    assert got.astype(object).tolist() == exact.tolist()
    # a bound one below the true maximum must be rejected, output untouched
    if bound > 1:
        st, _ = oracle.gemm_i64(A, B, prefix, bound - 1)
        assert st == RANGE_ERROR


def test_gemm_u64_brute_force():
    rng = np.random.default_rng(21)
    A = rng.integers(0, 1 << 23, size=(9, 300), dtype=np.uint64)
    B = rng.integers(0, 1 << 23, size=(300, 11), dtype=np.uint64)
    exact = A.astype(object) @ B.astype(object)
    st, got = oracle.gemm_u64(A, B, 8, (1 << 62))
    assert st == SUCCESS and got.astype(object).tolist() == exact.tolist()


def test_exact_gemm_brute_force_256bit():
    rng = np.random.default_rng(4)
    A = rng.integers(-(1 << 63), (1 << 63) - 1, size=(4, 50), dtype=np.int64)
    B = rng.integers(-(1 << 63), (1 << 63) - 1, size=(50, 3), dtype=np.int64)
    got = oracle.exact_gemm_i64(A, B, limbs=4)
    exact = A.astype(object) @ B.astype(object)
    for i in range(4):
        for j in range(3):
            assert oracle.limbs_to_int(got[i, j * 4:(j + 1) * 4], True) == exact[i, j]


def test_select_prefix_closed_form():
    """Bounded plans: the smallest prefix with P > 2*bound (int64) or P > bound
    (uint64), within the budget; FORCE_FIXED_PREFIX takes the budget."""
    L = oracle.lib()
    out = C.c_uint32(0)
    for bound in [1, 100, (1 << 40) * 256, (1 << 62), (1 << 63) - 1, 1 << 63]:
        for budget in (0, 8, 9, 20):
            eff = budget or 9
            need = next((p for p in range(1, 21) if product(p) > 2 * bound), 0)
            st = L.orc_select_prefix(1, 1, bound, 4096, budget, 0, 0, 0, C.byref(out))
            if need and need <= eff:
                assert st == SUCCESS and out.value == need
                st = L.orc_select_prefix(1, 1, bound, 4096, budget, 1, 0, 0, C.byref(out))
                assert st == SUCCESS and out.value == eff
            else:
                assert st != SUCCESS
    for bound in [1, (1 << 62), (1 << 64) - 1]:
        need = next(p for p in range(1, 21) if product(p) > bound)
        st = L.orc_select_prefix(2, 2, bound, 77, 0, 0, 0, 0, C.byref(out))
        assert st == SUCCESS and out.value == need


def test_generator_matches_product_inputs_module():
    """The benchmark's vectorized SplitMix64 streams equal the oracle's."""
    from rns8_amd import inputs

    seed = inputs.operand_seed(2026, "A")
    got = inputs.int_range(seed, (16, 16), 25)
    want = oracle.fill(seed, 0, 25, 256, np.int64).reshape(16, 16)
    assert np.array_equal(got, want)
    assert got.min() >= -(1 << 25) and got.max() < (1 << 25)
