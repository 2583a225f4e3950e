"""Every modulus prefix and every export contract on the GPU, through the C ABI.

C = A x I (B the identity) goes through pack, the plane GEMM and the Garner
export of each contract, with A spanning the whole range the prefix admits
(including both ends). The export kernels are instantiated per prefix, so each
prefix is its own code path. Results are compared bit-exactly with A itself
and with the oracle (planes and exports). Finite contracts are swept over every
modulus 2..256 against the closed form (A x B) mod m.
"""
import numpy as np
import pytest

import oracle
import rns8_amd as r

pytestmark = pytest.mark.gpu

I64_MIN = int(np.iinfo(np.int64).min)
I64_MAX = int(np.iinfo(np.int64).max)
U64_MAX = int(np.iinfo(np.uint64).max)
M_ROWS, N_COLS = 37, 24


def _identity(n, dtype):
    return np.eye(n, dtype=dtype)


def _run(ctx, sem, bk, A, B, prefix, bound=0, limbs=1):
    m, k = A.shape
    n = B.shape[1]
    desc = r.gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(ctx, desc)
    assert plan.prefix == prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, prefix))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    pack = r.pack_u64 if sem in (r.BOUNDED_U64, r.EXACT_WIDE_UNSIGNED) else r.pack_i64
    r.check(pack(ctx, Am, A, 1), "pack A")
    r.check(pack(ctx, Bm, B, 2), "pack B")
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm")
    return plan, Cm


def _sweep_i64(ctx, prefix, cols):
    P = oracle.modulus_product(prefix)
    bound = min((P - 1) // 2, 1 << 63)  # 2 * bound < P
    hi = min(bound, I64_MAX)
    rng = np.random.default_rng(prefix + 1000 * (cols != N_COLS))
    A = rng.integers(-bound, hi, size=(M_ROWS, cols), endpoint=True, dtype=np.int64)
    A.reshape(-1)[:5] = [-bound, hi, 0, 1, -1]
    A[-1, -5:] = [-bound, hi, 0, 1, -1]
    plan, Cm = _run(ctx, r.BOUNDED_I64, r.BOUND_GLOBAL_MAX_ABS, A, _identity(cols, np.int64), prefix, bound)
    planes = Cm.read_residues(prefix)
    np.testing.assert_array_equal(planes, oracle.pack_i64(A, prefix))
    out = np.zeros_like(A)
    assert r.export_i64(ctx, plan, Cm, out) == r.SUCCESS
    np.testing.assert_array_equal(out, A)
    ost, oout = oracle.export_i64(planes, prefix, bound)
    assert ost == 0
    np.testing.assert_array_equal(out, oout)


@pytest.mark.parametrize("prefix", range(1, 21))
def test_bounded_i64_every_prefix(gpu_ctx, prefix):
    _sweep_i64(gpu_ctx, prefix, N_COLS)


def _sweep_u64(ctx, prefix, cols):
    P = oracle.modulus_product(prefix)
    bound = min(P - 1, U64_MAX)
    rng = np.random.default_rng(100 + prefix + 1000 * (cols != N_COLS))
    A = rng.integers(0, bound, size=(M_ROWS, cols), endpoint=True, dtype=np.uint64)
    A.reshape(-1)[:3] = [0, bound, 1]
    A[-1, -3:] = [0, bound, 1]
    plan, Cm = _run(ctx, r.BOUNDED_U64, r.BOUND_GLOBAL_MAX_UNSIGNED, A, _identity(cols, np.uint64), prefix, bound)
    out = np.zeros_like(A)
    assert r.export_u64(ctx, plan, Cm, out) == r.SUCCESS
    np.testing.assert_array_equal(out, A)
    ost, oout = oracle.export_u64(Cm.read_residues(prefix), prefix, bound)
    assert ost == 0
    np.testing.assert_array_equal(out, oout)


@pytest.mark.parametrize("prefix", range(1, 21))
def test_bounded_u64_every_prefix(gpu_ctx, prefix):
    _sweep_u64(gpu_ctx, prefix, N_COLS)


# Results at least 256 columns wide export through the matrix-core form at
# prefixes 9..11; 260 columns = one full 256-column chunk and a ragged one.
@pytest.mark.parametrize("prefix", [9, 10, 11])
@pytest.mark.parametrize("unsigned", [False, True])
def test_bounded_64bit_wide_results(gpu_ctx, prefix, unsigned):
    (_sweep_u64 if unsigned else _sweep_i64)(gpu_ctx, prefix, 260)


def _wide_limbs(values, limbs):
    out = np.zeros((values.shape[0], values.shape[1] * limbs), dtype=np.uint64)
    for i in range(values.shape[0]):
        for j in range(values.shape[1]):
            x = int(values[i, j]) % (1 << (64 * limbs))
            for l in range(limbs):
                out[i, j * limbs + l] = (x >> (64 * l)) & U64_MAX
    return out


@pytest.mark.parametrize("prefix", [17, 18, 19, 20])
@pytest.mark.parametrize("limbs", [1, 2, 3, 4])
def test_exact_wide_signed_every_admissible_prefix(gpu_ctx, prefix, limbs):
    rng = np.random.default_rng(200 + prefix)
    A = rng.integers(I64_MIN, I64_MAX, size=(M_ROWS, N_COLS), endpoint=True, dtype=np.int64)
    A.reshape(-1)[:4] = [I64_MIN, I64_MAX, 0, -1]
    plan, Cm = _run(gpu_ctx, r.EXACT_WIDE_SIGNED, r.BOUND_NONE, A, _identity(N_COLS, np.int64), prefix)
    out = np.full((M_ROWS, N_COLS * limbs), 0xA5A5, dtype=np.uint64)
    assert r.export_exact_wide_signed_limbs(gpu_ctx, plan, Cm, out, limbs) == r.SUCCESS
    np.testing.assert_array_equal(out, _wide_limbs(A, limbs))
    ost, oout = oracle.export_exact_wide(Cm.read_residues(prefix), prefix, limbs, True)
    assert ost == 0
    np.testing.assert_array_equal(out, oout)


@pytest.mark.parametrize("prefix", [18, 19, 20])
@pytest.mark.parametrize("limbs", [1, 2, 3])
def test_exact_wide_unsigned_every_admissible_prefix(gpu_ctx, prefix, limbs):
    rng = np.random.default_rng(300 + prefix)
    A = rng.integers(0, U64_MAX, size=(M_ROWS, N_COLS), endpoint=True, dtype=np.uint64)
    A.reshape(-1)[:3] = [0, U64_MAX, 1 << 63]
    plan, Cm = _run(gpu_ctx, r.EXACT_WIDE_UNSIGNED, r.BOUND_NONE, A, _identity(N_COLS, np.uint64), prefix)
    out = np.full((M_ROWS, N_COLS * limbs), 0xA5A5, dtype=np.uint64)
    assert r.export_exact_wide_unsigned_limbs(gpu_ctx, plan, Cm, out, limbs) == r.SUCCESS
    np.testing.assert_array_equal(out, _wide_limbs(A.astype(object), limbs))
    ost, oout = oracle.export_exact_wide(Cm.read_residues(prefix), prefix, limbs, False)
    assert ost == 0
    np.testing.assert_array_equal(out, oout)


def _is_prime(m):
    return m >= 2 and all(m % d for d in range(2, int(m ** 0.5) + 1))


def test_finite_ring_every_modulus(gpu_ctx):
    m_, n_, k_ = 33, 17, 45
    rng = np.random.default_rng(7)
    A = rng.integers(0, 256, size=(m_, k_), dtype=np.uint8)
    B = rng.integers(0, 256, size=(k_, n_), dtype=np.uint8)
    for modulus in range(2, 257):
        Am = (A % modulus).astype(np.uint8) if modulus < 256 else A
        Bm = (B % modulus).astype(np.uint8) if modulus < 256 else B
        field = _is_prime(modulus)
        sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
        desc = r.gemm_desc(sem, r.BOUND_NONE, m_, n_, k_, finite_modulus=modulus)
        st, C = r.gemm_finite_u8_oneshot(gpu_ctx, desc, modulus, Am, Bm, field)
        assert st == 0, modulus
        want = ((Am.astype(np.int64) @ Bm.astype(np.int64)) % modulus).astype(np.uint8)
        np.testing.assert_array_equal(C, want, err_msg=f"modulus {modulus}")
