"""Pins the CPU oracle (oracle/psgd_oracle.py) against closed forms, library routines, invariants and brute force.
Each check is chosen so that a plausible slip in the restatement (a dropped term, a wrong sign or index, a
transposed operand, a wrong draw order) fails it."""
import math

import pytest
import torch

from oracle import psgd_oracle as O
from tests.metrics import rel_err_norm

torch.set_default_dtype(torch.float32)


def spd(n, seed, rank=None, dtype=torch.float64):
    g = torch.Generator().manual_seed(seed)
    X = torch.randn(n, rank or n, generator=g, dtype=dtype)
    return X @ X.T


# --------------------------------------------------------------------------- factor rule (psgd_pro.py:189)
@pytest.mark.parametrize("shape,skew,size,expect", [
    ((1024, 1024), 1.0, math.inf, (True, True)),            # one 1024 x 1024 fp32 weight
    ((768, 2304), 1.0, 8192, (True, False)),                  # ViT-B qkv, reference default skew
    ((768, 768), 1.0, 8192, (True, True)),                    # proj
    ((768, 3072), 1.0, 8192, (True, False)),                  # fc1
    ((3072, 768), 1.0, 8192, (False, True)),                  # fc2
    ((768, 2304), math.inf, 8192, (True, True)),              # skew = inf: every side dense
    ((3072, 768), math.inf, 8192, (True, True)),
    ((4096, 14336), math.inf, 14336, (True, True)),           # Llama MLP with max_size >= 14336
    ((4096, 14336), math.inf, 8192, (True, False)),           # 14336 > max_size -> diagonal
    ((1, 5), 1.0, math.inf, (False, False)),                  # size 1 is always diagonal
    ((768,), 1.0, math.inf, (False,)),                        # a vector: 768^2 > 768
    ((768,), math.inf, math.inf, (True,)),
])
def test_factor_rule(shape, skew, size, expect):
    numel = math.prod(shape)
    got = tuple(O.is_dense(d, numel, size, skew) for d in shape)
    assert got == expect


def test_init_factors_closed_form():
    Q, L = O.init_factors((6, 40), 4.0, max_skew=1.0, dtype=torch.float64)
    # 6^2 <= 240 dense; 40^2 > 240 diagonal; scale^(1/order) = 2
    assert Q[0].shape == (6, 6) and torch.equal(Q[0], 2.0 * torch.eye(6, dtype=torch.float64))
    assert Q[1].shape == (40,) and torch.equal(Q[1], torch.full((40,), 2.0, dtype=torch.float64))
    assert all(float(l) == 0.0 for l in L) and L[0].dtype == torch.float64
    Qs, Ls = O.init_factors((), 3.0)
    assert Qs[0].dim() == 0 and float(Qs[0]) == 3.0  # a scalar keeps Scale itself (psgd_pro.py:170)
    Qb, Lb = O.init_factors((4, 4), 1.0, dtype=torch.bfloat16)
    assert Lb[0].dtype == torch.float32  # lift2single (psgd_pro.py:67-69)


def test_init_scale_on_the_fly():
    g = [torch.full((2, 2), 2.0), torch.full((3,), 1.0)]
    s = O.init_scale_on_the_fly(g, 1e-9)
    assert s == pytest.approx((16.0 + 1e-36) ** (-1 / 8))


# --------------------------------------------------------------------------- norm lower bounds (psgd_pro.py:19-65)
@pytest.mark.parametrize("n,seed", [(8, 0), (33, 1), (64, 2), (150, 3)])
def test_nlb_spd_is_a_tight_lower_bound(n, seed):
    A = spd(n, seed)
    V = torch.randn(32, n, generator=torch.Generator().manual_seed(seed + 100), dtype=torch.float64)
    b = float(O.norm_lower_bound(A, V, skew=False))
    top = float(torch.linalg.matrix_norm(A, 2))
    assert b <= top * (1 + 1e-12)
    assert b >= 0.5 * top  # 4 subspace products on a Wishart spectrum get well within a factor 2


@pytest.mark.parametrize("n,seed", [(8, 0), (64, 1), (130, 2)])
def test_nlb_spd_exact_for_rank1(n, seed):
    v = torch.randn(n, 1, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    A = v @ v.T
    V = torch.randn(32, n, generator=torch.Generator().manual_seed(seed + 7), dtype=torch.float64)
    assert float(O.norm_lower_bound(A, V, skew=False)) == pytest.approx(float(v.norm() ** 2), rel=1e-12)


@pytest.mark.parametrize("n,seed", [(8, 0), (64, 1), (131, 2)])
def test_nlb_skew(n, seed):
    g = torch.Generator().manual_seed(seed)
    u = torch.randn(n, 1, generator=g, dtype=torch.float64)
    w = torch.randn(n, 1, generator=g, dtype=torch.float64)
    R = u @ w.T - w @ u.T  # rank-2 skew: both singular values are equal -> the bound is exact
    V = torch.randn(32, n, generator=g, dtype=torch.float64)
    top = float(torch.linalg.matrix_norm(R, 2))
    assert float(O.norm_lower_bound(R, V, skew=True)) == pytest.approx(top, rel=1e-10)
    X = torch.randn(n, n, generator=g, dtype=torch.float64)
    R = X - X.T
    b = float(O.norm_lower_bound(R, V, skew=True))
    top = float(torch.linalg.matrix_norm(R, 2))
    assert 0.5 * top <= b <= top * (1 + 1e-12)


def test_nlb_uses_max_diag_for_spd_and_max_abs_for_skew():
    # The normalising factor cancels in exact arithmetic; a matrix whose diagonal max differs from |A| max
    # exercises both branches through the rank-1 exactness.
    v = torch.tensor([[1.0], [-3.0], [2.0]], dtype=torch.float64)
    A = v @ v.T  # max diag 9 = max|A|; exact bound 14
    V = torch.randn(32, 3, generator=torch.Generator().manual_seed(0), dtype=torch.float64)
    assert float(O.norm_lower_bound(A, V, skew=False)) == pytest.approx(14.0, rel=1e-12)
    Z = torch.zeros(5, 5, dtype=torch.float64)
    assert float(O.norm_lower_bound(Z, torch.randn(32, 5, dtype=torch.float64), skew=True)) == 0.0


# --------------------------------------------------------------------------- Procrustes (psgd_pro.py:71-94)
def test_procrustes_fixed_point_for_symmetric_q():
    A = spd(20, 5) / 20 + torch.eye(20, dtype=torch.float64)
    Q = A.clone()
    V = torch.randn(32, 20, dtype=torch.float64)
    O.procrustes_step2(Q, V)
    assert torch.equal(Q, A)


def test_procrustes_reduces_asymmetry_and_caps_step():
    g = torch.Generator().manual_seed(3)
    n = 24
    S = spd(n, 4) / n + torch.eye(n, dtype=torch.float64)
    K = torch.randn(n, n, generator=g, dtype=torch.float64)
    Q = S + 0.05 * (K - K.T)
    V = torch.randn(32, n, generator=g, dtype=torch.float64)
    asym0 = float((Q - Q.T).norm())
    Q1 = Q.clone()
    a = float(O.procrustes_step2(Q1, V))
    assert 0 < a <= 1 / 8
    assert float((Q1 - Q1.T).norm()) < asym0


def test_procrustes_r2_equals_step2():
    g = torch.Generator().manual_seed(9)
    n = 40
    S = spd(n, 10) / n + torch.eye(n, dtype=torch.float64)
    K = torch.randn(n, n, generator=g, dtype=torch.float64)
    Q = S + 0.1 * (K - K.T) + 0.02 * torch.randn(n, n, generator=g, dtype=torch.float64)
    V = torch.randn(32, n, generator=g, dtype=torch.float64)
    Qa, Qb = Q.clone(), Q.clone()
    a1 = O.procrustes_step2(Qa, V)
    a2 = O.procrustes_step_r2(Qb, V)
    assert float(a1) == pytest.approx(float(a2), rel=1e-10)
    assert rel_err_norm(Qb, Qa) < 1e-12


def test_procrustes_step_matches_second_order_rotation():
    # Q + aRQ + a^2/2 R^2 Q with R skew is exp(aR) Q to second order: the result's deviation from the exact
    # rotation is O(a^3 |R|^3).
    g = torch.Generator().manual_seed(2)
    n = 16
    K = torch.randn(n, n, generator=g, dtype=torch.float64)
    Q = torch.eye(n, dtype=torch.float64) + 0.01 * (K - K.T)
    V = torch.randn(32, n, generator=g, dtype=torch.float64)
    Q1 = Q.clone()
    a = float(O.procrustes_step2(Q1, V))
    R = Q.T - Q
    R = R / (O.norm_lower_bound(R, V, skew=True) + O.smallest_normal(R.dtype))
    exact = torch.linalg.matrix_exp(a * R) @ Q
    assert rel_err_norm(Q1, exact) < 10 * a ** 3


# --------------------------------------------------------------------------- balance (psgd_pro.py:96-105)
def test_balance_keeps_kron_product():
    g = torch.Generator().manual_seed(1)
    q1 = torch.randn(4, 4, generator=g, dtype=torch.float64) * 10
    q2 = torch.randn(3, generator=g, dtype=torch.float64) * 0.01
    K0 = torch.kron(q1, torch.diag(q2))
    Q = [q1.clone(), q2.clone()]
    O.balance(Q)
    assert rel_err_norm(torch.kron(Q[0], torch.diag(Q[1])), K0) < 1e-14
    m0, m1 = float(Q[0].abs().max()), float(Q[1].abs().max())
    assert m0 == pytest.approx(m1, rel=1e-12)  # both at the geometric mean
    one = [q1.clone()]
    O.balance(one)
    assert torch.equal(one[0], q1)


# --------------------------------------------------------------------------- preconditioning / Gram (exprP, exprGs)
def test_precondition_matches_kronecker_brute_force():
    g = torch.Generator().manual_seed(0)
    m, n = 5, 7
    Q1 = torch.randn(m, m, generator=g, dtype=torch.float64)
    Q2 = torch.randn(n, n, generator=g, dtype=torch.float64)
    G = torch.randn(m, n, generator=g, dtype=torch.float64)
    P1, P2 = Q1.T @ Q1, Q2.T @ Q2
    # row-major vec: vec(P1 G P2) = (P1 kron P2^T) vec(G)
    ref = (torch.kron(P1, P2.T.contiguous()) @ G.reshape(-1)).reshape(m, n)
    assert rel_err_norm(O.precondition([Q1, Q2], G), ref) < 1e-13
    # diagonal second factor, and the general N-D path on the same data
    q2 = torch.randn(n, generator=g, dtype=torch.float64)
    ref = P1 @ G * (q2 * q2)[None, :]
    assert rel_err_norm(O.precondition([Q1, q2], G), ref) < 1e-13
    q1 = torch.randn(m, generator=g, dtype=torch.float64)
    ref = (q1 * q1)[:, None] * G @ P2
    assert rel_err_norm(O.precondition([q1, Q2], G), ref) < 1e-13
    T = torch.randn(3, 4, 2, generator=g, dtype=torch.float64)
    Qs = [torch.randn(3, 3, generator=g, dtype=torch.float64), torch.randn(4, generator=g, dtype=torch.float64),
          torch.randn(2, 2, generator=g, dtype=torch.float64)]
    Ps = [Qs[0].T @ Qs[0], torch.diag(Qs[1] * Qs[1]), Qs[2].T @ Qs[2]]
    ref = torch.einsum("aA,bB,cC,ABC->abc", Ps[0], Ps[1], Ps[2], T)
    assert rel_err_norm(O.precondition(Qs, T), ref) < 1e-13
    s = torch.tensor(3.0, dtype=torch.float64)
    assert float(O.precondition([torch.tensor(2.0, dtype=torch.float64)], s)) == 12.0


def test_gram_orientation():
    g = torch.Generator().manual_seed(0)
    Pg = torch.randn(5, 7, generator=g, dtype=torch.float64)
    assert torch.allclose(O.gram(Pg, 0, True), Pg @ Pg.T)
    assert torch.allclose(O.gram(Pg, 1, True), Pg.T @ Pg)
    assert torch.allclose(O.gram(Pg, 0, False), (Pg * Pg).sum(1))
    assert torch.allclose(O.gram(Pg, 1, False), (Pg * Pg).sum(0))


# --------------------------------------------------------------------------- the update (psgd_pro.py:114-139)
def test_first_update_from_identity_closed_form():
    """From Q = I, L = 0: Pg = X (the noised gradient), L = ell = nlb(term1) + term2 and Q_i = I - (lr/ell)(term1 -
    term2 I); term1 is symmetric, so the Procrustes step leaves Q unchanged (its fixed point)."""
    m, n, lr = 6, 9, 0.1
    G = torch.randn(m, n, generator=torch.Generator().manual_seed(5), dtype=torch.float64)
    Q, L = O.init_factors((m, n), 1.0, max_skew=math.inf, dtype=torch.float64)  # both factors dense
    dr = O.Draws(7)
    O.update_preconditioner(Q, L, G, dr, lr=lr, betaL=0.9, damping=1e-9)
    # replay the draws
    d2 = O.Draws(7)
    N = d2.normal((m, n)).double()
    X = G + (1e-9 + torch.finfo(torch.float64).eps * G.abs()) * N
    for i, d in enumerate((m, n)):
        T = X @ X.T if i == 0 else X.T @ X
        T = (T + T.T) / 2  # the restatement's product is symmetric up to rounding
        V1 = d2.normal((32, d)).double()
        ell = float(O.norm_lower_bound(T, V1, skew=False)) + m * n / d
        d2.normal((32, d))
        assert float(L[i]) == pytest.approx(ell, rel=1e-12)
        Qi = torch.eye(d, dtype=torch.float64) - lr / ell * (T - m * n / d * torch.eye(d, dtype=torch.float64))
        assert rel_err_norm(Q[i], Qi) < 1e-12


def test_draw_order_follows_psgd_pro():
    """The oracle consumes: update coin; per parameter noise (G's shape), then per dense factor spd and skew
    starts (32 x d), then the balancing coin (psgd_pro.py:345,123,35,59,138)."""
    W = torch.zeros(6, 40)
    opt = O.OracleKron([W], preconditioner_init_scale=1.0, seed=11, dtype=torch.float64)
    g = torch.randn(6, 40, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    opt.step([g])
    gen = torch.Generator().manual_seed(11)
    torch.rand([], generator=gen)           # update coin
    torch.randn(6, 40, generator=gen)       # damping noise
    torch.randn(32, 6, generator=gen)       # dense factor 0 (6 x 6): spd start
    torch.randn(32, 6, generator=gen)       #                          skew start (factor 1 is diagonal: no draws)
    torch.rand([], generator=gen)           # balancing coin
    assert torch.equal(opt.draws.gen.get_state(), gen.get_state())


def test_clip_closed_form():
    p = torch.zeros(4)
    g = torch.tensor([30.0, -1.0, 0.5, 2.0])
    out = O.clip_and_update(p, g.clone(), 0.1, 2.0, 10.0)
    avg = math.sqrt(float((g * g).mean()))
    ref = (g * (2.0 / avg)).clamp(-10, 10)
    assert torch.allclose(out, ref)
    assert torch.allclose(p, -0.1 * ref)
    small = torch.tensor([0.1, -0.2])
    assert torch.equal(O.clip_and_update(torch.zeros(2), small.clone(), 1.0), small)


@pytest.mark.parametrize("shape,skew", [((48, 64), 1.0), ((32, 40), math.inf), ((20,), math.inf), ((17,), 1.0)])
def test_fp32_step_tracks_fp64(shape, skew):
    """The whole optimizer step in float32 stays within float32 rounding of the same step in float64 on the same
    draws (brute-force pin of the restatement's arithmetic)."""
    steps = 5
    W64 = torch.zeros(shape, dtype=torch.float64)
    W32 = torch.zeros(shape, dtype=torch.float32)
    o64 = O.OracleKron([W64], preconditioner_max_skew=skew, preconditioner_init_scale=1.0, seed=3,
                       dtype=torch.float64)
    o32 = O.OracleKron([W32], preconditioner_max_skew=skew, preconditioner_init_scale=1.0, seed=3,
                       dtype=torch.float32)
    gen = torch.Generator().manual_seed(4)
    for _ in range(steps):
        g = 0.01 * torch.randn(shape, generator=gen, dtype=torch.float64)
        o64.step([g])
        o32.step([g.float()])
        for q32, q64 in zip(o32.Q[0], o64.Q[0]):
            assert rel_err_norm(q32, q64) < 1e-5
        assert rel_err_norm(o32.pre[0], o64.pre[0]) < 1e-5
    assert rel_err_norm(W32, W64) < 1e-5


def test_flops_formula():
    shapes = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
    assert 12 * sum(O.flops_2d(m, n) for m, n in shapes) / 1e12 == pytest.approx(7.7236, rel=1e-4)
    assert O.flops_2d(1024, 1024) / 1e9 == pytest.approx(26.852, rel=1e-4)
