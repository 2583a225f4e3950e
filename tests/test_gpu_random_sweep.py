"""Seeded random sweep of the public path against the CPU oracle.

Each case draws its own route, semantics, shape, value range, bound, prefix
and row strides from a seeded generator, so the cases land on combinations
the hand-written parity tests do not name: ragged tile edges next to the 128
and 256 tile sizes, outputs up to 4500 x 4500 (the 256 x 256 tile
configuration) with a short K, K just past the 64-deep step, past 65536 and up to
10^6 (several accumulation blocks or K slices), forced prefixes above what the bound needs,
false bounds (the export must then report what the oracle reports), strided
host sources and both exact-wide signednesses. Every comparison is bit-exact:
residue planes byte for byte, exports value for value and status for status.

Routes: resident pack -> GEMM -> export through host arrays (int64, uint64;
the GEMM through rns8_gemm_rns or the entry that allocates nothing), the
host-array oneshot entries, the fused native-input GEMM on device
operands, finite-field / finite-ring oneshots, the exact-wide path, and
exact-wide chains D = (A x B) x E whose second product's admission (the
refined bound from C's carried summaries, reference exact_range.hpp,
restated in oracle/exact_range.py) falls on either side of the range, packed
from host arrays or from device memory; per-tile bound plans (true tile
maxima, or one lowered by one); grouped GEMMs of 2-40 tasks (bounded and
finite, through the host or the stream entries); and the device-pointer packs, stream GEMMs and device exports
(bounded, finite and exact-wide limbs, destinations with padded rows).

RNS8_SWEEP_CASES sets the number of cases (default 400), RNS8_SWEEP_BASE the
first seed (default 0).
"""
import ctypes
import os

import numpy as np
import pytest

import oracle
import rns8_amd as r
from oracle import exact_range as xr
from rns8_amd import hip, inputs

pytestmark = pytest.mark.gpu

CASES = int(os.environ.get("RNS8_SWEEP_CASES", "400"))
BASE = int(os.environ.get("RNS8_SWEEP_BASE", "0"))
EDGES = [1, 2, 31, 32, 33, 63, 64, 65, 127, 128, 129, 255, 256, 257, 511, 513]
I64_MIN = np.iinfo(np.int64).min
I64_MAX = np.iinfo(np.int64).max


def _dim(rng, cap):
    u = rng.random()
    if u < 0.55:
        v = int(rng.integers(1, 65))
    elif u < 0.8:
        v = int(rng.integers(65, 600))
    else:
        v = int(rng.choice(EDGES))
    return min(v, cap)


def _depth(rng, m, n):
    u = rng.random()
    if u < 0.45:
        k = int(rng.integers(1, 129))
    elif u < 0.8:
        k = int(rng.integers(129, 2049))
    elif u < 0.93:
        k = int(rng.choice([63, 64, 65, 1023, 1024, 1025, 4095, 4097]))
    elif u < 0.98:
        k = int(rng.choice([65535, 65536, 65537, 70001, 131073]))
    else:
        k = int(rng.choice([262145, 524288, 1000003]))
    # keep the oracle's work per case in the tens of millions of products
    return max(1, min(k, 60_000_000 // max(1, m * n)))


def _signed_values(rng, seed, shape, bits):
    a = inputs.int_range(seed, shape, bits)
    if rng.random() < 0.3 and a.size:
        # the range's extremes at random positions
        flat = a.reshape(-1)
        idx = rng.integers(0, flat.size, size=min(4, flat.size))
        flat[idx] = rng.choice([-(1 << bits), (1 << bits) - 1], size=idx.size)
    return a


def _unsigned_values(rng, seed, shape, bits):
    a = inputs.uint_range(seed, shape, bits)
    if rng.random() < 0.3 and a.size:
        flat = a.reshape(-1)
        idx = rng.integers(0, flat.size, size=min(4, flat.size))
        flat[idx] = np.uint64((1 << bits) - 1)
    return a


def _strided(rng, a):
    """The operand as a host array with a row stride at or above its width."""
    if rng.random() < 0.7:
        return a, a.shape[1]
    ld = a.shape[1] + int(rng.integers(1, 9))
    full = np.zeros((a.shape[0], ld), dtype=a.dtype)
    full[:, : a.shape[1]] = a
    full[:, a.shape[1]:] = a.dtype.type(0x5A) if a.dtype != np.uint8 else 0x5A
    return full, ld


def _large(rng):
    """A large output (the 256 x 256 tile configuration) with a short K."""
    m, n = int(rng.integers(1000, 4500)), int(rng.integers(1000, 4500))
    return m, n, int(rng.integers(1, max(2, 30_000_000 // (m * n)) + 1))


def _bounded_case(ctx, rng, seed, signed, route):
    if route != "fused" and rng.random() < 0.1:
        m, n, k = _large(rng)
    else:
        m, n = _dim(rng, 700), _dim(rng, 700)
        k = _depth(rng, m, n)
    kb = max(1, int(k).bit_length())
    # value bits so that k * 2^(2 bits) stays below 2^62
    top = max(1, (62 - kb) // 2)
    bits = int(rng.integers(1, top + 1))
    if signed:
        A = _signed_values(rng, seed * 2 + 1, (m, k), bits)
        B = _signed_values(rng, seed * 2 + 2, (k, n), bits)
        true_bound = k << (2 * bits)
    else:
        A = _unsigned_values(rng, seed * 2 + 1, (m, k), bits)
        B = _unsigned_values(rng, seed * 2 + 2, (k, n), bits)
        true_bound = k * ((1 << bits) - 1) ** 2
    false_bound = rng.random() < 0.12
    bound = max(1, true_bound >> int(rng.integers(4, 40))) if false_bound else true_bound
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    forced = rng.random() < 0.25
    need = r.select_prefix(r.gemm_desc(sem, bk, m, n, k, bound=bound))[1]
    max_prefix = int(rng.integers(need, 21)) if forced else 0
    desc = r.gemm_desc(sem, bk, m, n, k, bound=bound, max_prefix=max_prefix,
                       flags=r.PLAN_FORCE_FIXED_PREFIX if forced else 0)
    label = f"{route} {'i64' if signed else 'u64'} {m}x{n}x{k} bits={bits} bound={bound} forced={max_prefix}"
    print(f"[sweep {seed}] {label}", flush=True)
    st_ref, want = (oracle.gemm_i64 if signed else oracle.gemm_u64)(
        A, B, max_prefix or need, bound)
    if route == "oneshot":
        fn = r.gemm_i64_oneshot if signed else r.gemm_u64_oneshot
        st, C = fn(ctx, desc, A, B)
        assert st == st_ref, label
        if st == r.SUCCESS:
            np.testing.assert_array_equal(C, want, err_msg=label)
        return
    plan = r.Plan(ctx, desc)
    p = plan.prefix
    assert p == (max_prefix or need), label
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, p))
    Cm = mk(m, n)
    ws = r.Workspace(ctx, plan)
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    want_planes = oracle.gemm_rns(pack_ref(A, p), pack_ref(B, p), p)
    if route == "fused":
        # the fused entry loads 16-byte chunks: even row strides (padded
        # with nonzero filler the kernel must not read as operand values)
        pa = np.full((m, k + (k & 1)), 0x5A, dtype=A.dtype)
        pb = np.full((k, n + (n & 1)), 0x5A, dtype=B.dtype)
        pa[:, :k], pb[:, :n] = A, B
        dA = hip.malloc(max(pa.nbytes, 16))
        dB = hip.malloc(max(pb.nbytes, 16))
        try:
            hip.to_device(dA, pa)
            hip.to_device(dB, pb)
            fn = r.lib().rns8_mi355x_gemm_native_i64_async if signed else r.lib().rns8_mi355x_gemm_native_u64_async
            st = fn(ctx.ptr, plan.ptr, ctypes.c_void_p(dA), pa.shape[1], ctypes.c_void_p(dB), pb.shape[1], Cm.ptr,
                    ws.ptr, None)
            hip.synchronize()
        finally:
            hip.free(dA)
            hip.free(dB)
        # the fused form is offered for small outputs only; elsewhere the
        # call refuses without writing
        print(f"[sweep {seed}] fused status {st}", flush=True)
        if st == r.UNSUPPORTED_BACKEND:
            return
        assert st == r.SUCCESS, label
    else:
        Am, Bm = mk(m, k), mk(k, n)
        pack = r.pack_i64 if signed else r.pack_u64
        sa, lda = _strided(rng, A)
        sb, ldb = _strided(rng, B)
        r.check(pack(ctx, Am, sa, 1, ld=lda), "pack A")
        r.check(pack(ctx, Bm, sb, 2, ld=ldb), "pack B")
        if rng.random() < 0.25:
            # the entry that allocates nothing (split-K residues in the
            # library's 4 MiB static scratch)
            st = r.lib().rns8_mi355x_gemm_rns_noalloc(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, None)
            hip.synchronize()
            print(f"[sweep {seed}] noalloc status {st}", flush=True)
            if st == r.abi.WORKSPACE_TOO_SMALL:
                return
            assert st == r.SUCCESS, label
        else:
            r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, ws), "gemm")
    np.testing.assert_array_equal(Cm.read_residues(p), want_planes, err_msg=label)
    out = np.full((m, n), 0x77, dtype=np.int64 if signed else np.uint64)
    st = (r.export_i64 if signed else r.export_u64)(ctx, plan, Cm, out)
    ost, oout = (oracle.export_i64 if signed else oracle.export_u64)(want_planes, p, bound)
    assert st == ost == st_ref, label
    if st == r.SUCCESS:
        np.testing.assert_array_equal(out, oout, err_msg=label)
        np.testing.assert_array_equal(out, want, err_msg=label)
    else:
        assert (out == 0x77).all(), label


def _finite_case(ctx, rng, seed):
    m, n = _dim(rng, 600), _dim(rng, 600)
    k = min(_depth(rng, m, n), 20000)
    field = rng.random() < 0.5
    modulus = int(rng.choice([2, 3, 5, 7, 13, 127, 211, 241, 251])) if field else int(rng.integers(2, 257))
    label = f"finite {'field' if field else 'ring'} mod {modulus} {m}x{n}x{k}"
    print(f"[sweep {seed}] {label}", flush=True)
    A = inputs.bytes_below(seed * 2 + 1, (m, k), 256)
    B = inputs.bytes_below(seed * 2 + 2, (k, n), 256)
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus)
    st, C = r.gemm_finite_u8_oneshot(ctx, desc, modulus, A, B, field)
    assert st == r.SUCCESS, label
    np.testing.assert_array_equal(C, ((A.astype(np.int64) @ B.astype(np.int64)) % modulus).astype(np.uint8),
                                  err_msg=label)


def _wide_min_prefix(signed, k):
    """The smallest prefix an exact-wide plan of inner dimension k accepts:
    its modulus product must exceed k * 2^127 (signed) or k * 2^128."""
    need = k << (127 if signed else 128)
    return next(p for p in range(1, 21) if oracle.modulus_product(p) > need)


def _wide_case(ctx, rng, seed):
    signed = rng.random() < 0.6
    m, n = _dim(rng, 48), _dim(rng, 48)
    k = min(_depth(rng, m, n), 3000)
    prefix = int(rng.integers(_wide_min_prefix(signed, k), 21))
    limbs = int(rng.integers(1, 7))
    full = rng.random() < 0.5
    bits = 63 if full else int(rng.integers(1, 62))
    if signed:
        A = inputs.full_int64(seed * 2 + 1, (m, k)) if full else _signed_values(rng, seed * 2 + 1, (m, k), bits)
        B = inputs.full_int64(seed * 2 + 2, (k, n)) if full else _signed_values(rng, seed * 2 + 2, (k, n), bits)
    else:
        A = _unsigned_values(rng, seed * 2 + 1, (m, k), 64 if full else bits)
        B = _unsigned_values(rng, seed * 2 + 2, (k, n), 64 if full else bits)
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    label = f"wide {'signed' if signed else 'unsigned'} {m}x{n}x{k} prefix={prefix} limbs={limbs} full={full}"
    print(f"[sweep {seed}] {label}", flush=True)
    desc = r.gemm_desc(sem, r.BOUND_NONE, m, n, k, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX)
    plan = r.Plan(ctx, desc)
    assert plan.prefix == prefix, label
    product = oracle.modulus_product(prefix)
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, prefix))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    pack = r.pack_i64 if signed else r.pack_u64
    rows_a = A.tolist()
    rows_b = B.tolist()
    for mat, src, rows, tag in ((Am, A, rows_a, "A"), (Bm, B, rows_b, "B")):
        st = pack(ctx, mat, src, 1)
        admits = xr.pack_admits(signed, rows, product)
        assert st == (r.SUCCESS if admits else r.RANGE_ERROR), f"{label} pack {tag}"
        if not admits:
            return
    st = r.gemm_rns(ctx, plan, Am, Bm, Cm, ws)
    bound, _ = xr.gemm_bound(xr.native_operand(rows_a), xr.native_operand(rows_b), m, n, k)
    fits = xr.fits(signed, bound, product)
    assert st == (r.SUCCESS if fits else r.RANGE_ERROR), f"{label} gemm (bound {bound})"
    if not fits:
        return
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    planes = oracle.gemm_rns(pack_ref(A, prefix), pack_ref(B, prefix), prefix)
    np.testing.assert_array_equal(Cm.read_residues(prefix), planes, err_msg=label)
    out = np.full((m, n * limbs), 0xA5A5, dtype=np.uint64)
    export = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    st = export(ctx, plan, Cm, out, limbs)
    ost, oout = oracle.export_exact_wide(planes, prefix, limbs, signed)
    assert st == ost, label
    if st == r.SUCCESS:
        np.testing.assert_array_equal(out, oout, err_msg=label)
        exact = (oracle.exact_gemm_i64 if signed else oracle.exact_gemm_u64)(A[:2], B[:, :2], limbs=4)
        for i in range(min(2, m)):
            for j in range(min(2, n)):
                assert (oracle.limbs_to_int(out[i, limbs * j:limbs * (j + 1)], signed)
                        == oracle.limbs_to_int(exact[i, 4 * j:4 * (j + 1)], signed)), label
    else:
        assert (out == 0xA5A5).all(), label


def _int_matmul(A, B):
    return [[sum(x * y for x, y in zip(row, col)) for col in zip(*B)] for row in A]


def _chain_case(ctx, rng, seed):
    """D = (A x B) x E, exact-wide: C = A x B is always admitted; D's
    admission is the refined bound from C's carried summaries, drawn to land
    on either side of the prefix's range."""
    signed = rng.random() < 0.6
    device = rng.random() < 0.5
    m, k1, k2, n = (int(rng.integers(1, 25)) for _ in range(4))
    prefix = int(rng.integers(_wide_min_prefix(signed, max(k1, k2)), 21))
    P = oracle.modulus_product(prefix)
    # operand bits summing to about the range's bits less the inner dimensions'
    total = P.bit_length() - (k1 * k2).bit_length() + int(rng.integers(-3, 6))
    third = total // 3
    ba, bb = (third + int(rng.integers(-8, 9)) for _ in range(2))
    bits = [max(1, min(63, b)) for b in (ba, bb, total - ba - bb)]

    def draw(rows, cols, b):
        hi = (1 << b) - 1
        lo = -(1 << b) if signed else 0
        return [[int(v) for v in rng.integers(lo, hi, size=cols, endpoint=True)] for _ in range(rows)]

    A, B, E = draw(m, k1, bits[0]), draw(k1, k2, bits[1]), draw(k2, n, bits[2])
    label = (f"chain {'signed' if signed else 'unsigned'} {'device' if device else 'host'} "
             f"{m}x{k1}x{k2}x{n} prefix={prefix} bits={bits}")
    print(f"[sweep {seed}] {label}", flush=True)
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    dt = np.int64 if signed else np.uint64
    flags = r.PLAN_FORCE_FIXED_PREFIX
    p1 = r.Plan(ctx, r.gemm_desc(sem, r.BOUND_NONE, m, k2, k1, max_prefix=prefix, flags=flags))
    p2 = r.Plan(ctx, r.gemm_desc(sem, r.BOUND_NONE, m, n, k2, max_prefix=prefix, flags=flags))
    mats = {name: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, prefix))
            for name, rows, cols in (("A", m, k1), ("B", k1, k2), ("C", m, k2), ("E", k2, n), ("D", m, n))}
    for version, (name, src) in enumerate((("A", A), ("B", B), ("E", E)), start=1):
        arr = np.array(src, dtype=object).astype(dt)
        if device:
            d = hip.malloc(arr.nbytes)
            try:
                hip.to_device(d, arr)
                fn = r.lib().rns8_mi355x_pack_i64_device if signed else r.lib().rns8_mi355x_pack_u64_device
                st = fn(ctx.ptr, mats[name].ptr, ctypes.c_void_p(d), arr.shape[1], 0, None)
                hip.synchronize()
            finally:
                hip.free(d)
        else:
            st = (r.pack_i64 if signed else r.pack_u64)(ctx, mats[name], arr, version)
        assert st == r.SUCCESS, f"{label} pack {name}"
    ws1, ws2 = r.Workspace(ctx, p1), r.Workspace(ctx, p2)
    if device:
        st1 = r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p1.ptr, mats["A"].ptr, mats["B"].ptr, mats["C"].ptr,
                                                 ws1.ptr, None)
        st2 = r.lib().rns8_mi355x_gemm_rns_async(ctx.ptr, p2.ptr, mats["C"].ptr, mats["E"].ptr, mats["D"].ptr,
                                                 ws2.ptr, None)
        hip.synchronize()
    else:
        st1 = r.gemm_rns(ctx, p1, mats["A"], mats["B"], mats["C"], ws1)
        st2 = r.gemm_rns(ctx, p2, mats["C"], mats["E"], mats["D"], ws2)
    assert st1 == r.SUCCESS, label
    _, c_op = xr.gemm_bound(xr.native_operand(A), xr.native_operand(B), m, k2, k1)
    bound, _ = xr.gemm_bound(c_op, xr.native_operand(E), m, n, k2)
    fits = xr.fits(signed, bound, P)
    print(f"[sweep {seed}] D {'admitted' if fits else 'refused'}", flush=True)
    assert st2 == (r.SUCCESS if fits else r.RANGE_ERROR), f"{label} D (bound {bound.bit_length()} bits)"
    if not fits:
        return
    L = P.bit_length() // 64 + 2
    out = np.zeros((m, n * L), dtype=np.uint64)
    export = r.export_exact_wide_signed_limbs if signed else r.export_exact_wide_unsigned_limbs
    assert export(ctx, p2, mats["D"], out, L) == r.SUCCESS, label
    got = [[oracle.limbs_to_int(out[i, L * j:L * (j + 1)], signed) for j in range(n)] for i in range(m)]
    assert got == _int_matmul(_int_matmul(A, B), E), label


SENTINEL = -91


def _tiled_case(ctx, rng, seed):
    """Per-tile bounds: A's rows and B's columns get their own magnitudes in
    blocks, so tiles select different prefixes; the bounds are the tiles'
    true maxima, or one of them one below it (a RANGE_ERROR the oracle's
    tiled export also reports)."""
    signed = rng.random() < 0.6
    m, n = _dim(rng, 900), _dim(rng, 900)
    k = int(rng.integers(1, 25))
    tile_m, tile_n = (int(rng.choice([64, 128, 256, 512])) for _ in range(2))
    block = int(rng.choice([16, 64, 100]))
    rb = np.repeat(rng.integers(1, 29, size=-(-m // block)), block)[:m]
    cb = np.repeat(rng.integers(1, 29, size=-(-n // block)), block)[:n]
    A = rng.integers(0, 1 << 28, size=(m, k)) >> (28 - rb[:, None])
    B = rng.integers(0, 1 << 28, size=(k, n)) >> (28 - cb[None, :])
    if signed:
        A = A * np.where(rng.random((m, k)) < 0.5, -1, 1)
    dt = np.int64 if signed else np.uint64
    A, B = A.astype(dt), B.astype(dt)
    exact = A @ B  # |C| < 24 * 2^56: exact in 64 bits
    mag = np.abs(exact) if signed else exact
    rows = np.maximum.reduceat(mag, np.arange(0, m, tile_m), axis=0)
    bounds = [int(x) for x in np.maximum.reduceat(rows, np.arange(0, n, tile_n), axis=1).reshape(-1)]
    lowered = rng.random() < 0.15 and max(bounds) > 0
    if lowered:
        t = int(rng.choice([i for i, b in enumerate(bounds) if b > 0]))
        bounds[t] -= 1
    label = (f"tiled {'i64' if signed else 'u64'} {m}x{n}x{k} tiles {tile_m}x{tile_n} block {block}"
             f" lowered={lowered}")
    print(f"[sweep {seed}] {label}", flush=True)
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.abi.BOUND_PER_TILE_MAX_ABS if signed else r.abi.BOUND_PER_TILE_MAX_UNSIGNED
    desc = r.gemm_desc(sem, bk, m, n, k, max_prefix=9, tile_m=tile_m, tile_n=tile_n, tile_bounds=bounds)
    plan = r.Plan(ctx, desc)
    sp = plan.prefix
    st, entries, summary = oracle.tile_schedule(signed, m, n, tile_m, tile_n, bounds, 9, 0)
    assert st == 0 and summary.max_selected == sp, label
    mk = lambda rows_, cols_: r.Matrix(ctx, r.matrix_desc(rows_, cols_, sem, bk, sp, tile_m=tile_m, tile_n=tile_n))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    pack = r.pack_i64 if signed else r.pack_u64
    r.check(pack(ctx, Am, A, 1), "pack A")
    r.check(pack(ctx, Bm, B, 2), "pack B")
    ptr, _, pitch, count = Cm.planes()
    hip.memset(ptr, SENTINEL & 0xFF, pitch * count)
    hip.synchronize()
    r.check(r.gemm_rns(ctx, plan, Am, Bm, Cm, r.Workspace(ctx, plan)), "gemm")
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    Cp = oracle.gemm_rns_tiled(pack_ref(A, sp), pack_ref(B, sp), np.full((sp, m, n), SENTINEL, dtype=np.int8),
                               entries)
    np.testing.assert_array_equal(Cm.read_residues(sp), Cp, err_msg=label)
    out = np.full((m, n), 77, dtype=dt)
    est = (r.export_i64 if signed else r.export_u64)(ctx, plan, Cm, out)
    ost, oout = oracle.export_tiled(Cp, tile_m, tile_n, entries, bounds, signed)
    assert est == ost == (r.RANGE_ERROR if lowered else r.SUCCESS), label
    if est == r.SUCCESS:
        np.testing.assert_array_equal(out, oout, err_msg=label)
        np.testing.assert_array_equal(out, exact, err_msg=label)
    else:
        assert (out == 77).all(), label


def _grouped_case(ctx, rng, seed):
    """A group of same-shape tasks in one launch: every task's planes equal
    the oracle's (bounded) or the exact modular product (finite)."""
    kind = str(rng.choice(["i64", "u64", "field", "ring"]))
    count = int(rng.integers(2, 41))
    m, n = _dim(rng, 400), _dim(rng, 400)
    k = max(1, min(_depth(rng, m, n), 8_000_000 // max(1, m * n * count)))
    label = f"grouped {kind} x{count} {m}x{n}x{k}"
    print(f"[sweep {seed}] {label}", flush=True)
    if kind in ("field", "ring"):
        field = kind == "field"
        modulus = int(rng.choice([2, 13, 251])) if field else int(rng.integers(2, 257))
        sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
        plan = r.Plan(ctx, r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus))
        mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, 0))
        ops = [(inputs.bytes_below(seed * 100 + 2 * i, (m, k), 256), inputs.bytes_below(seed * 100 + 2 * i + 1,
                                                                                        (k, n), 256))
               for i in range(count)]
        tasks = [(mk(m, k), mk(k, n), mk(m, n), r.Workspace(ctx, plan)) for _ in range(count)]
        for i, ((A, B), (Am, Bm, _, _)) in enumerate(zip(ops, tasks)):
            r.check(r.pack_finite_u8(ctx, Am, modulus, A, 2 * i + 1), "pack A")
            r.check(r.pack_finite_u8(ctx, Bm, modulus, B, 2 * i + 2), "pack B")
        if rng.random() < 0.4:
            # the stream entry on the context stream, then a synchronization
            r.check(r.lib().rns8_mi355x_gemm_finite_u8_grouped_async(ctx.ptr, plan.ptr, modulus, r.grouped_tasks(tasks),
                                                                     len(tasks), None), label)
            hip.synchronize()
        else:
            r.check(r.gemm_finite_u8_grouped(ctx, plan, modulus, tasks), label)
        for (A, B), (_, _, Cm, _) in zip(ops, tasks):
            out = np.zeros((m, n), dtype=np.uint8)
            r.check(r.export_finite_u8(ctx, plan, modulus, Cm, out), "export")
            want = ((A.astype(np.int64) @ B.astype(np.int64)) % modulus).astype(np.uint8)
            np.testing.assert_array_equal(out, want, err_msg=label)
        return
    signed = kind == "i64"
    kb = max(1, int(k).bit_length())
    bits = int(rng.integers(1, max(1, (62 - kb) // 2) + 1))
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    bound = (k << (2 * bits)) if signed else k * ((1 << bits) - 1) ** 2
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, bound=bound))
    p = plan.prefix
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, p))
    draw = _signed_values if signed else _unsigned_values
    ops = [(draw(rng, seed * 100 + 2 * i, (m, k), bits), draw(rng, seed * 100 + 2 * i + 1, (k, n), bits))
           for i in range(count)]
    tasks = [(mk(m, k), mk(k, n), mk(m, n), r.Workspace(ctx, plan)) for _ in range(count)]
    pack = r.pack_i64 if signed else r.pack_u64
    for i, ((A, B), (Am, Bm, _, _)) in enumerate(zip(ops, tasks)):
        r.check(pack(ctx, Am, A, 2 * i + 1), "pack A")
        r.check(pack(ctx, Bm, B, 2 * i + 2), "pack B")
    if rng.random() < 0.4:
        r.check(r.lib().rns8_mi355x_gemm_rns_grouped_async(ctx.ptr, plan.ptr, r.grouped_tasks(tasks), len(tasks), None),
                label)
        hip.synchronize()
    else:
        r.check(r.gemm_rns_grouped(ctx, plan, tasks), label)
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    for (A, B), (_, _, Cm, _) in zip(ops, tasks):
        want = oracle.gemm_rns(pack_ref(A, p), pack_ref(B, p), p)
        np.testing.assert_array_equal(Cm.read_residues(p), want, err_msg=label)


def _device_case(ctx, rng, seed):
    """Device-pointer packs (strided sources), the stream GEMM entry and the
    device export (status word on the device) against the oracle."""
    signed = rng.random() < 0.6
    if rng.random() < 0.15:
        m, n, k = _large(rng)
    else:
        m, n = _dim(rng, 700), _dim(rng, 700)
        k = _depth(rng, m, n)
    kb = max(1, int(k).bit_length())
    bits = int(rng.integers(1, max(1, (62 - kb) // 2) + 1))
    draw = _signed_values if signed else _unsigned_values
    A, B = draw(rng, seed * 2 + 1, (m, k), bits), draw(rng, seed * 2 + 2, (k, n), bits)
    true_bound = (k << (2 * bits)) if signed else k * ((1 << bits) - 1) ** 2
    bound = max(1, true_bound >> int(rng.integers(4, 40))) if rng.random() < 0.12 else true_bound
    sem = r.BOUNDED_I64 if signed else r.BOUNDED_U64
    bk = r.BOUND_GLOBAL_MAX_ABS if signed else r.BOUND_GLOBAL_MAX_UNSIGNED
    plan = r.Plan(ctx, r.gemm_desc(sem, bk, m, n, k, bound=bound))
    p = plan.prefix
    label = f"device {'i64' if signed else 'u64'} {m}x{n}x{k} bits={bits} bound={bound} prefix={p}"
    print(f"[sweep {seed}] {label}", flush=True)
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, bk, p))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    L = r.lib()
    pack = L.rns8_mi355x_pack_i64_device if signed else L.rns8_mi355x_pack_u64_device
    ptrs = []
    try:
        for mat, src in ((Am, A), (Bm, B)):
            full, ld = _strided(rng, src)
            d = hip.malloc(max(full.nbytes, 16))
            ptrs.append(d)
            hip.to_device(d, np.ascontiguousarray(full))
            r.check(pack(ctx.ptr, mat.ptr, ctypes.c_void_p(d), ld, 0, None), "device pack")
        r.check(L.rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, None), "gemm")
        ld_out = n + int(rng.integers(0, 3))
        dt = np.int64 if signed else np.uint64
        out = np.full((m, ld_out), 0x77, dtype=dt)
        d_out = hip.malloc(max(out.nbytes, 16))
        d_status = hip.malloc(16)
        ptrs += [d_out, d_status]
        hip.to_device(d_out, out)
        hip.memset(d_status, 0, 16)
        export = L.rns8_mi355x_export_i64_device if signed else L.rns8_mi355x_export_u64_device
        r.check(export(ctx.ptr, plan.ptr, Cm.ptr, ctypes.c_void_p(d_out), ld_out, ctypes.c_void_p(d_status), None),
                "device export")
        hip.synchronize()
        status = np.zeros(4, dtype=np.uint32)
        hip.from_device(status, d_status)
        hip.from_device(out, d_out)
    finally:
        for d in ptrs:
            hip.free(d)
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    want_planes = oracle.gemm_rns(pack_ref(A, p), pack_ref(B, p), p)
    np.testing.assert_array_equal(Cm.read_residues(p), want_planes, err_msg=label)
    ost, oout = (oracle.export_i64 if signed else oracle.export_u64)(want_planes, p, bound)
    assert (status[0] == 0) == (ost == r.SUCCESS), label
    if ost == r.SUCCESS:
        np.testing.assert_array_equal(out[:, :n], oout, err_msg=label)
        assert (out[:, n:] == 0x77).all(), label


def _to_device(arr):
    d = hip.malloc(max(arr.nbytes, 16))
    hip.to_device(d, np.ascontiguousarray(arr))
    return d


def _finite_device_case(ctx, rng, seed):
    """Finite field / ring through the device entries: device packs from
    strided byte sources, the stream GEMM and the device export into a
    destination with a row stride above its width."""
    m, n = _dim(rng, 600), _dim(rng, 600)
    k = min(_depth(rng, m, n), 20000)
    field = rng.random() < 0.5
    modulus = int(rng.choice([2, 3, 5, 7, 13, 127, 211, 241, 251])) if field else int(rng.integers(2, 257))
    label = f"finite-device {'field' if field else 'ring'} mod {modulus} {m}x{n}x{k}"
    print(f"[sweep {seed}] {label}", flush=True)
    A = inputs.bytes_below(seed * 2 + 1, (m, k), 256)
    B = inputs.bytes_below(seed * 2 + 2, (k, n), 256)
    sem = r.FINITE_FIELD_U8 if field else r.FINITE_RING_U8
    plan = r.Plan(ctx, r.gemm_desc(sem, r.BOUND_NONE, m, n, k, finite_modulus=modulus))
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, 0))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    L = r.lib()
    ld_out = n + int(rng.integers(0, 40))
    out = np.full((m, ld_out), 0xA7, dtype=np.uint8)
    ptrs = []
    try:
        for mat, src in ((Am, A), (Bm, B)):
            full, ld = _strided(rng, src)
            ptrs.append(_to_device(full))
            r.check(L.rns8_mi355x_pack_finite_u8_device(ctx.ptr, mat.ptr, modulus, ctypes.c_void_p(ptrs[-1]), ld, 0,
                                                        None), "device pack")
        r.check(L.rns8_mi355x_gemm_finite_u8_async(ctx.ptr, plan.ptr, modulus, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, None),
                "gemm")
        ptrs.append(_to_device(out))
        r.check(L.rns8_mi355x_export_finite_u8_device(ctx.ptr, plan.ptr, modulus, Cm.ptr, ctypes.c_void_p(ptrs[-1]),
                                                      ld_out, None), "device export")
        hip.synchronize()
        hip.from_device(out, ptrs[-1])
    finally:
        for d in ptrs:
            hip.free(d)
    want = ((A.astype(np.int64) @ B.astype(np.int64)) % modulus).astype(np.uint8)
    np.testing.assert_array_equal(out[:, :n], want, err_msg=label)
    assert (out[:, n:] == 0xA7).all(), label


def _wide_device_case(ctx, rng, seed):
    """Exact-wide through the device entries: device packs (their magnitude
    proofs on the device), the stream GEMM and the limb export into a device
    destination with a row stride above its width, status on the device."""
    signed = rng.random() < 0.6
    m, n = _dim(rng, 300), _dim(rng, 300)
    k = min(_depth(rng, m, n), 3000)
    prefix = int(rng.integers(_wide_min_prefix(signed, k), 21))
    limbs = int(rng.integers(1, 7))
    full = rng.random() < 0.5
    bits = 63 if full else int(rng.integers(1, 62))
    if signed:
        A = inputs.full_int64(seed * 2 + 1, (m, k)) if full else _signed_values(rng, seed * 2 + 1, (m, k), bits)
        B = inputs.full_int64(seed * 2 + 2, (k, n)) if full else _signed_values(rng, seed * 2 + 2, (k, n), bits)
    else:
        A = _unsigned_values(rng, seed * 2 + 1, (m, k), 64 if full else bits)
        B = _unsigned_values(rng, seed * 2 + 2, (k, n), 64 if full else bits)
    sem = r.EXACT_WIDE_SIGNED if signed else r.EXACT_WIDE_UNSIGNED
    label = f"wide-device {'signed' if signed else 'unsigned'} {m}x{n}x{k} prefix={prefix} limbs={limbs} full={full}"
    print(f"[sweep {seed}] {label}", flush=True)
    plan = r.Plan(ctx, r.gemm_desc(sem, r.BOUND_NONE, m, n, k, max_prefix=prefix, flags=r.PLAN_FORCE_FIXED_PREFIX))
    mk = lambda rows, cols: r.Matrix(ctx, r.matrix_desc(rows, cols, sem, r.BOUND_NONE, prefix))
    Am, Bm, Cm = mk(m, k), mk(k, n), mk(m, n)
    ws = r.Workspace(ctx, plan)
    L = r.lib()
    pack = L.rns8_mi355x_pack_i64_device if signed else L.rns8_mi355x_pack_u64_device
    export = (L.rns8_mi355x_export_exact_wide_signed_limbs_device if signed
              else L.rns8_mi355x_export_exact_wide_unsigned_limbs_device)
    ld_out = n + int(rng.integers(0, 5))
    out = np.full((m, ld_out * limbs), 0xA5A5, dtype=np.uint64)
    status = np.zeros(4, dtype=np.uint32)
    ptrs = []
    try:
        for mat, src in ((Am, A), (Bm, B)):
            full_src, ld = _strided(rng, src)
            ptrs.append(_to_device(full_src))
            r.check(pack(ctx.ptr, mat.ptr, ctypes.c_void_p(ptrs[-1]), ld, 0, None), "device pack")
        r.check(L.rns8_mi355x_gemm_rns_async(ctx.ptr, plan.ptr, Am.ptr, Bm.ptr, Cm.ptr, ws.ptr, None), "gemm")
        ptrs.append(_to_device(out))
        ptrs.append(_to_device(status))
        r.check(export(ctx.ptr, plan.ptr, Cm.ptr, ctypes.c_void_p(ptrs[-2]), ld_out, limbs,
                       ctypes.c_void_p(ptrs[-1]), None), "device export")
        hip.synchronize()
        hip.from_device(out, ptrs[-2])
        hip.from_device(status, ptrs[-1])
    finally:
        for d in ptrs:
            hip.free(d)
    pack_ref = oracle.pack_i64 if signed else oracle.pack_u64
    planes = oracle.gemm_rns(pack_ref(A, prefix), pack_ref(B, prefix), prefix)
    np.testing.assert_array_equal(Cm.read_residues(prefix), planes, err_msg=label)
    ost, oout = oracle.export_exact_wide(planes, prefix, limbs, signed)
    assert (status[0] == 0) == (ost == r.SUCCESS), label
    if ost == r.SUCCESS:
        got = out.reshape(m, ld_out, limbs)[:, :n, :].reshape(m, n * limbs)
        np.testing.assert_array_equal(got, oout, err_msg=label)
        assert (out.reshape(m, ld_out, limbs)[:, n:, :] == 0xA5A5).all(), label


ROUTES = ["resident_i64", "resident_u64", "oneshot_i64", "oneshot_u64", "fused_i64", "fused_u64", "finite",
          "wide", "chain", "tiled", "grouped", "device", "finite_device", "wide_device"]
WEIGHTS = [0.12, 0.06, 0.05, 0.05, 0.07, 0.06, 0.06, 0.09, 0.09, 0.08, 0.08, 0.08, 0.05, 0.06]


@pytest.mark.parametrize("seed", range(BASE, BASE + CASES))
def test_random_case(gpu_ctx, seed):
    rng = np.random.default_rng(0x5EED0000 + seed)
    route = ROUTES[int(rng.choice(len(ROUTES), p=WEIGHTS))]
    if route == "finite":
        _finite_case(gpu_ctx, rng, seed)
    elif route == "wide":
        _wide_case(gpu_ctx, rng, seed)
    elif route == "chain":
        _chain_case(gpu_ctx, rng, seed)
    elif route == "tiled":
        _tiled_case(gpu_ctx, rng, seed)
    elif route == "grouped":
        _grouped_case(gpu_ctx, rng, seed)
    elif route == "device":
        _device_case(gpu_ctx, rng, seed)
    elif route == "finite_device":
        _finite_device_case(gpu_ctx, rng, seed)
    elif route == "wide_device":
        _wide_device_case(gpu_ctx, rng, seed)
    else:
        kind, sem = route.split("_")
        _bounded_case(gpu_ctx, rng, seed, sem == "i64", kind)
