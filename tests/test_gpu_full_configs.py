"""The BASELINE configurations at their full sizes, through the C ABI.

Two independent checks per configuration:
  * Freivalds' identity C x = A (B x) for random vectors x, modulo three primes
    near 2^20 (every product and sum stays exact in int64 at these sizes), over
    the whole output: a wrong cell survives one prime with probability 1/p;
  * bit-exact comparison with the CPU oracle (the reference's CPU_REFERENCE
    pipeline, restated in oracle/) on sampled rows, first and last included.
Configurations: C2 finite field 251 at 4096^3, C3 bounded int64 at 4096^3
(prefix 9 forced), C4 exact-wide signed at 2048^3 (prefix 20 forced, 3 limbs),
C5 bounded uint64 at 128 x 128 x 65536 (split-K).
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r
from rns8_amd import inputs

pytestmark = pytest.mark.gpu

PRIMES = [1048573, 1048571, 1048559]


def _mod_p_signed(x: np.ndarray, p: int) -> np.ndarray:
    return np.mod(x.astype(np.int64), p) if x.dtype == np.int64 else _mod_p_u64(x, p)


def _mod_p_u64(x: np.ndarray, p: int) -> np.ndarray:
    x = x.astype(np.uint64)
    hi = (x >> np.uint64(32)).astype(np.int64) % p
    lo = (x & np.uint64(0xFFFFFFFF)).astype(np.int64) % p
    return (hi * (pow(2, 32, p)) + lo) % p


def freivalds(A_p, B_p, C_p, p, seed):
    """A_p, B_p, C_p already reduced to [0, p) int64."""
    rng = np.random.default_rng(seed)
    x = rng.integers(0, p, size=(B_p.shape[1],), dtype=np.int64)
    bx = (B_p @ x) % p
    lhs = (C_p @ x) % p
    rhs = (A_p @ bx) % p
    return np.array_equal(lhs, rhs)


def sample_rows(m):
    rng = np.random.default_rng(m)
    return sorted({0, m - 1, *rng.integers(0, m, size=6).tolist()})


def test_c3_bounded_i64_4096_prefix9(gpu_ctx):
    M = N = K = 4096
    A = inputs.int_range(inputs.operand_seed(11, "A"), (M, K), 25)
    B = inputs.int_range(inputs.operand_seed(11, "B"), (K, N), 25)
    desc = r.gemm_desc(r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, M, N, K, bound=1 << 62, max_prefix=9,
                       flags=r.PLAN_FORCE_FIXED_PREFIX)
    st, C = r.gemm_i64_oneshot(gpu_ctx, desc, A, B)
    assert st == r.SUCCESS
    for i, p in enumerate(PRIMES):
        assert freivalds(np.mod(A, p), np.mod(B, p), np.mod(C, p), p, seed=i)
    for row in sample_rows(M):
        ost, want = oracle.gemm_i64(A, B, 9, 1 << 62, row0=row, rows=1)
        assert ost == 0
        np.testing.assert_array_equal(C[row:row + 1], want)


def test_c2_finite_field_251_4096(gpu_ctx):
    M = N = K = 4096
    A = inputs.bytes_below(21, (M, K), 251)
    B = inputs.bytes_below(22, (K, N), 251)
    desc = r.gemm_desc(r.FINITE_FIELD_U8, r.BOUND_NONE, M, N, K, finite_modulus=251)
    st, C = r.gemm_finite_u8_oneshot(gpu_ctx, desc, 251, A, B, True)
    assert st == r.SUCCESS
    assert C.max() < 251
    for i in range(3):  # exact over the field itself
        assert freivalds(A.astype(np.int64), B.astype(np.int64), C.astype(np.int64), 251, seed=10 + i)
    for row in sample_rows(M):
        want = oracle.gemm_finite_u8(A, B, 251, row0=row, rows=1)
        np.testing.assert_array_equal(C[row:row + 1], want)


def _limbs_mod_p(limbs: np.ndarray, L: int, p: int) -> np.ndarray:
    """Signed L-limb little-endian two's complement values -> residues mod p."""
    rows, cols = limbs.shape[0], limbs.shape[1] // L
    v = limbs.reshape(rows, cols, L)
    acc = np.zeros((rows, cols), dtype=np.int64)
    for l in range(L):
        acc = (acc + _mod_p_u64(v[:, :, l], p) * pow(2, 64 * l, p)) % p
    negative = (v[:, :, L - 1] >> np.uint64(63)).astype(bool)
    acc = (acc - negative.astype(np.int64) * pow(2, 64 * L, p)) % p
    return acc


def test_c4_exact_wide_signed_2048_prefix20(gpu_ctx):
    M = N = K = 2048
    L = 3
    A = inputs.full_int64(inputs.operand_seed(31, "A"), (M, K))
    B = inputs.full_int64(inputs.operand_seed(31, "B"), (K, N))
    desc = r.gemm_desc(r.EXACT_WIDE_SIGNED, r.BOUND_NONE, M, N, K, max_prefix=20, flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(gpu_ctx, desc)
    assert plan.prefix == 20
    mk = lambda rows, cols: r.Matrix(gpu_ctx, r.matrix_desc(rows, cols, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, 20))
    Am, Bm, Cm = mk(M, K), mk(K, N), mk(M, N)
    ws = r.Workspace(gpu_ctx, plan)
    r.check(r.pack_i64(gpu_ctx, Am, A, 1), "pack A")
    r.check(r.pack_i64(gpu_ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(gpu_ctx, plan, Am, Bm, Cm, ws), "gemm")
    out = np.zeros((M, N * L), dtype=np.uint64)
    assert r.export_exact_wide_signed_limbs(gpu_ctx, plan, Cm, out, L) == r.SUCCESS
    for i, p in enumerate(PRIMES):
        assert freivalds(np.mod(A, p), np.mod(B, p), _limbs_mod_p(out, L, p), p, seed=20 + i)
    for row in sample_rows(M)[:4]:
        ost, want = oracle.gemm_exact_wide_signed(A, B, 20, L, row0=row, rows=1)
        assert ost == 0
        np.testing.assert_array_equal(out[row:row + 1], want)


def test_c5_bounded_u64_tall_skinny_full(gpu_ctx):
    M = N = 128
    K = 65536
    A = inputs.uint_range(inputs.operand_seed(41, "A"), (M, K), 23)
    B = inputs.uint_range(inputs.operand_seed(41, "B"), (K, N), 23)
    desc = r.gemm_desc(r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, M, N, K, bound=1 << 62)
    st, C = r.gemm_u64_oneshot(gpu_ctx, desc, A, B)
    assert st == r.SUCCESS
    for i, p in enumerate(PRIMES):
        assert freivalds(_mod_p_u64(A, p), _mod_p_u64(B, p), _mod_p_u64(C, p), p, seed=30 + i)
    ost, want = oracle.gemm_u64(A, B, 8, 1 << 62, row0=0, rows=M)
    assert ost == 0
    np.testing.assert_array_equal(C, want)
