"""Pins for the oracle's RNS layer: BConv, ModUp, ModDown, rescale, key switching, automorphism.

Each check ties the oracle to an independent statement: CRT reconstruction with Python big integers
(BConv/ModUp/ModDown/rescale identities), the exact-division special case ModDown(P*y) = y,
decryption noise after key switching, the key-noise audit of hpc_gpu_port/seeded_keys.hpp:417-449,
polynomial substitution X -> X^g by brute force, and the reference's rotation-index contract
(tests/golden/contract_r17.json, from results/dense-demo-s31/pod_2xbw_20260917/pod_pull/contract_r17.json).
"""
import json
import os
from functools import reduce

import numpy as np
import pytest

from conftest import GOLDEN


def crt(res, mods):
    """CRT reconstruction of one coefficient from its residues, in [0, prod)."""
    M = reduce(lambda a, b: a * b, mods, 1)
    x = 0
    for r, m in zip(res, mods):
        Mi = M // m
        x += int(r) * Mi * pow(Mi, -1, m)
    return x % M, M


def centered(x, M):
    return x - M if x > M // 2 else x


@pytest.fixture(scope="module")
def small(oracle):
    """logN = 10, L = 6 Q limbs (40-bit), K = 2 P limbs (45-bit), dnum = 3 (alpha = 2)."""
    logN = 10
    qs = oracle.gen_primes(40, 6, 2 << logN)
    ps = oracle.gen_primes(45, 2, 2 << logN)
    return oracle.Ctx(logN, qs + ps, 6, 2, 3)


def rand_limbs(ctx, idx, rng):
    return np.stack([rng.integers(0, ctx.q[i], ctx.N, dtype=np.uint64) for i in idx])


def test_bconv_is_the_approximate_crt_switch(small):
    """out_j = (X + u Q) mod p_j exactly, with u = floor(sum_i y_i / q_i), y_i = [x_i q_hat_i^-1]_{q_i} (OpenFHE's
    approximate switch, HYBRID ModUp: the sum sum_i y_i (Q / q_i) is reduced mod p_j without the correction of u Q);
    u is computed here with big integers, so an exact CRT conversion (u = 0 everywhere) or any other u fails."""
    rng = np.random.default_rng(11)
    src, dst = [0, 1, 2], [3, 4, 6, 7]
    x = rand_limbs(small, src, rng)
    y = small.bconv(x, src, dst)
    qs = [small.q[i] for i in src]
    Q = qs[0] * qs[1] * qs[2]
    seen_u = set()
    for k in range(0, small.N, 7):
        X, _ = crt([x[i][k] for i in range(3)], qs)
        yi = [int(x[i][k]) * pow(Q // q, -1, q) % q for i, q in enumerate(qs)]
        S = sum(v * (Q // q) for v, q in zip(yi, qs))   # = X + u Q over the integers
        u = S // Q
        assert S == X + u * Q and 0 <= u < len(src)
        seen_u.add(u)
        for j, pj in enumerate(dst):
            assert int(y[j][k]) == S % small.q[pj], (k, j)
    # the samples exercise the approximation: exact CRT would have given u = 0 at every coefficient
    assert seen_u - {0}


def test_modup_digits(small):
    rng = np.random.default_rng(12)
    l = 5  # below the top level: digits {0,1},{2,3},{4}
    D = small.num_digits(l)
    assert D == 3
    x = rand_limbs(small, range(l), rng)
    ext = small.modup(x, l)
    E = l + small.K
    pidx = list(range(l)) + [small.L + k for k in range(small.K)]
    coef_x = small.ntt_inv(x, list(range(l)))
    for d in range(D):
        lo, hi = 2 * d, min(2 * d + 2, l)
        assert np.array_equal(ext[d][lo:hi], x[lo:hi])
        coef = small.ntt_inv(ext[d], pidx)
        mods = [small.q[i] for i in range(lo, hi)]
        Qd = reduce(lambda a, b: a * b, mods)
        for k in range(0, small.N, 53):
            X, _ = crt([coef_x[i][k] for i in range(lo, hi)], mods)
            for t in range(E):
                if lo <= t < hi:
                    continue
                p = small.q[pidx[t]]
                assert any((X + u * Qd - int(coef[t][k])) % p == 0 for u in range(hi - lo))


def test_moddown_exact_on_multiples_of_P(small):
    rng = np.random.default_rng(13)
    l = 6
    y = rand_limbs(small, range(l), rng)
    P = small.q[6] * small.q[7]
    x = np.zeros((l + 2, small.N), dtype=np.uint64)
    for i in range(l):
        x[i] = ((y[i].astype(object) * (P % small.q[i])) % small.q[i]).astype(np.uint64)
    # P limbs of P*y are zero
    assert np.array_equal(small.moddown(x, l), y)


def test_moddown_identity(small):
    """P*z = X_Q - X_P - v*P (mod Q) with v in [0, K): the division by P is exact up to BConv's overflow."""
    rng = np.random.default_rng(14)
    l = 4
    pidx = list(range(l)) + [6, 7]
    x = rand_limbs(small, pidx, rng)
    z = small.moddown(x, l)
    xc = small.ntt_inv(x, pidx)
    zc = small.ntt_inv(z, list(range(l)))
    P = small.q[6] * small.q[7]
    Qm = [small.q[i] for i in range(l)]
    for k in range(0, small.N, 41):
        XQ, Q = crt([xc[i][k] for i in range(l)], Qm)
        XP, _ = crt([xc[l][k], xc[l + 1][k]], [small.q[6], small.q[7]])
        Z, _ = crt([zc[i][k] for i in range(l)], Qm)
        assert any((P * Z - (XQ - XP - v * P)) % Q == 0 for v in range(2))


def test_rescale_identity(small):
    """q_l * Z + centered(c_l) = C (mod Q/q_l) and Z is C/q_l rounded (|C - q_l Z| <= q_l/2)."""
    rng = np.random.default_rng(15)
    l = 6
    c = rand_limbs(small, range(l), rng)
    z = small.rescale(np.stack([c, c]), l)
    assert z.shape == (2, l - 1, small.N) and np.array_equal(z[0], z[1])
    cc = small.ntt_inv(c, list(range(l)))
    zc = small.ntt_inv(z[0], list(range(l - 1)))
    ql = small.q[l - 1]
    mods = [small.q[i] for i in range(l - 1)]
    for k in range(0, small.N, 29):
        C, QQ = crt([cc[i][k] for i in range(l)], [small.q[i] for i in range(l)])
        Z, Qp = crt([zc[i][k] for i in range(l - 1)], mods)
        cl = centered(int(cc[l - 1][k]), ql)
        assert (ql * Z + cl - C) % Qp == 0
        # as integers on the centered representatives: Z = round(C / q_l)
        Cc, Zc = centered(C, QQ), centered(Z, Qp)
        assert abs(Cc - ql * Zc) <= ql // 2


def _secret_and_keys(oracle, ctx, h=16):
    s = oracle.sample_ternary(b"\x05" * 32, ctx.N, h)
    s_eval = ctx.small_to_eval(s, list(range(ctx.L)))
    return s, s_eval


def test_ksk_noise_audit(oracle, small):
    """seeded_keys.hpp:417-449: b_j + a_j * s_new - [digit] PModq * s_old is a few sigma."""
    s, s_eval = _secret_and_keys(oracle, small)
    s2 = oracle.sample_ternary(b"\x06" * 32, small.N, 16)
    evk = small.ksk_gen(s_eval, s2, b"\x09" * 32, b"\x0a" * 32)
    T = small.L + small.K
    sn = small.small_to_eval(s2, list(range(T)))
    P = small.q[6] * small.q[7]
    for d in range(small.dnum):
        lo, hi = 2 * d, min(2 * d + 2, small.L)
        e = np.zeros((T, small.N), dtype=np.uint64)
        for i in range(T):
            q = small.q[i]
            v = (evk[d][0][i].astype(object) + evk[d][1][i].astype(object) * sn[i].astype(object)) % q
            if lo <= i < hi:
                v = (v - (P % q) * s_eval[i].astype(object)) % q
            e[i] = v.astype(np.uint64)
        ec = small.ntt_inv(e, list(range(T)))
        for i in range(T):
            q = small.q[i]
            cen = np.where(ec[i] > q // 2, ec[i].astype(np.float64) - q, ec[i].astype(np.float64))
            assert np.abs(cen).max() < 40


def test_keyswitch_decrypts(oracle, small):
    """KS(x) = (o0, o1) with o0 + o1 * s_new = x * s_old + small, at every level."""
    s, s_eval = _secret_and_keys(oracle, small)
    s2 = oracle.sample_ternary(b"\x07" * 32, small.N, 16)
    evk = small.ksk_gen(s_eval, s2, b"\x0b" * 32, b"\x0c" * 32)
    rng = np.random.default_rng(16)
    for l in (6, 5, 3, 1):
        x = rand_limbs(small, range(l), rng)
        o = small.keyswitch(x, l, evk)
        sn = small.small_to_eval(s2, list(range(l)))
        err = np.zeros((l, small.N), dtype=np.uint64)
        for i in range(l):
            q = small.q[i]
            v = (o[0][i].astype(object) + o[1][i].astype(object) * sn[i].astype(object)
                 - x[i].astype(object) * s_eval[i].astype(object)) % q
            err[i] = v.astype(np.uint64)
        ec = small.ntt_inv(err, list(range(l)))
        for i in range(l):
            q = small.q[i]
            cen = np.where(ec[i] > q // 2, ec[i].astype(np.float64) - q, ec[i].astype(np.float64))
            # error ~ (digit * e) / P + rounding: far below q / 2^10
            assert np.abs(cen).max() < 2.0**25, (l, i, np.abs(cen).max())


def test_automorph_coef_is_substitution(oracle, small):
    rng = np.random.default_rng(17)
    N = small.N
    a = rng.integers(0, small.q[0], N, dtype=np.uint64)
    q = small.q[0]
    for g in (5, 25, 2 * N - 1, small.rot_index(-3)):
        got = small.automorph_coef(a[None], [0], g)[0]
        want = [0] * N
        for j in range(N):
            e = (j * g) % (2 * N)
            if e < N:
                want[e] = (want[e] + int(a[j])) % q
            else:
                want[e - N] = (want[e - N] - int(a[j])) % q
        assert [int(x) for x in got] == want


def test_automorph_eval_commutes_with_ntt(oracle, small):
    rng = np.random.default_rng(18)
    x = rand_limbs(small, [0, 1, 7], rng)
    X = small.ntt_fwd(x, [0, 1, 7])
    for g in (5, 125, 2 * small.N - 1, small.rot_index(7), small.rot_index(-100)):
        lhs = small.automorph_eval(X, g)
        rhs = small.ntt_fwd(small.automorph_coef(x, [0, 1, 7], g), [0, 1, 7])
        assert np.array_equal(lhs, rhs)


def test_rot_index_matches_reference_contract(oracle):
    """contract_r17.json lists, at N = 2^17, every 5^k mod 2N for its rotation amounts and bootstrap
    steps plus the conjugate 2N-1 (gpu_real_model.cu:1337-1369)."""
    c = json.load(open(os.path.join(GOLDEN, "contract_r17.json")))
    N = c["ring"]
    q = oracle.gen_primes(40, 1, 2 * N)[0]
    ctx = oracle.Ctx(17, [q], 1, 0, 1)
    need = {ctx.rot_index(k) for k in c["rotationAmounts"] + c["bootstrapSteps"] if k != 0}
    need.add(2 * N - 1)
    assert need == set(c["autoIndices"])
    assert ctx.rot_index(1) == 5 and ctx.rot_index(-1) == pow(5, -1, 2 * N)


def test_rotate_decrypts_to_rotated_message(oracle, small):
    """EvalRotate: KS of c1 under evk_g (s -> tau_{g^-1}(s)), add c0, then X -> X^g.  The decryption
    under s is tau_g(m) + small (checked in coefficient form)."""
    s, s_eval = _secret_and_keys(oracle, small)
    N, l = small.N, 6
    g = small.rot_index(3)
    ginv = pow(g, -1, 2 * N)
    # tau_{g^-1}(s) as signed coefficients
    sp = np.zeros(N, dtype=np.int8)
    for j in range(N):
        e = (j * ginv) % (2 * N)
        if e < N:
            sp[e] += s[j]
        else:
            sp[e - N] -= s[j]
    evk = small.ksk_gen(s_eval, sp, b"\x0d" * 32, b"\x0e" * 32)
    rng = np.random.default_rng(19)
    m = rng.integers(-1000, 1000, N)
    a = rand_limbs(small, range(l), rng)
    mm = small.small_to_eval(m.astype(np.int32), list(range(l)))
    c0 = np.stack([((mm[i].astype(object) - a[i].astype(object) * s_eval[i].astype(object)) % small.q[i]).astype(np.uint64)
                   for i in range(l)])
    out = small.rotate(np.stack([c0, a]), l, g, evk)
    dec = np.stack([((out[0][i].astype(object) + out[1][i].astype(object) * s_eval[i].astype(object)) % small.q[i]).astype(np.uint64)
                    for i in range(l)])
    dc = small.ntt_inv(dec, list(range(l)))[0]
    q0 = small.q[0]
    got = np.where(dc > q0 // 2, dc.astype(np.int64) - np.int64(q0), dc.astype(np.int64))
    want = np.zeros(N, dtype=np.int64)
    for j in range(N):
        e = (j * g) % (2 * N)
        if e < N:
            want[e] += m[j]
        else:
            want[e - N] -= m[j]
    assert np.abs(got - want).max() < 2**25


def test_moddown_exact_is_rounded_division(oracle):
    """exact ModDown (centered conversion) == round(X / P) per coefficient, X the integer whose residues the
    Q and P limbs hold (closed form by big-integer CRT); the approximate form is floor(X / P) - u, u in [0, K)"""
    N = 1 << 16
    qs = oracle.gen_primes(40, 3, 2 * N)
    ps = oracle.gen_primes(60, 3, 2 * N)
    l, K = 3, 3
    ex = oracle.Ctx(16, qs + ps, l, K, 1, moddown_exact=True)
    ap = oracle.Ctx(16, qs + ps, l, K, 1, moddown_exact=False)
    P = 1
    for p in ps:
        P *= p
    QP = P
    for q in qs:
        QP *= q
    rng = np.random.default_rng(5)
    X = [int.from_bytes(rng.bytes(40), "little") % QP for _ in range(N)]
    coef = np.array([[x % m for x in X] for m in qs + ps], dtype=np.uint64)
    ev = ex.ntt_fwd(coef, list(range(l + K)))
    got_ex = ex.ntt_inv(ex.moddown(ev, l), list(range(l)))
    got_ap = ap.ntt_inv(ap.moddown(ev, l), list(range(l)))
    for k in range(0, N, 331):
        r = (X[k] + P // 2) // P  # round(X / P) (P odd: no ties)
        f = X[k] // P
        for i, q in enumerate(qs):
            assert int(got_ex[i, k]) == r % q, (k, i)
            u = (f - int(got_ap[i, k])) % q
            assert u < K, (k, i, u)


def test_hmult_batch_equals_single_calls(oracle, small):
    """the all-core CPU baseline's batch form: the same words as one call per pair, whatever the thread count"""
    rng = np.random.default_rng(21)
    l, n = 6, 5
    T = small.L + small.K
    a = np.stack([np.stack([rand_limbs(small, range(l), rng) for _ in range(2)]) for _ in range(n)])
    b = np.stack([np.stack([rand_limbs(small, range(l), rng) for _ in range(2)]) for _ in range(n)])
    evk = np.stack([np.stack([rand_limbs(small, range(T), rng) for _ in range(2)]) for _ in range(3)])
    want = np.stack([small.hmult_relin_rescale(a[i], b[i], l, evk) for i in range(n)])
    for threads in (1, 3):
        assert oracle.set_threads(threads) == threads
        assert np.array_equal(small.hmult_relin_rescale_batch(a, b, l, evk), want)
    oracle.set_threads(0)
