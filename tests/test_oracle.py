"""Pins the CPU oracle (oracle/psgd_oracle.py) against closed forms, library routines, invariants and brute force.
Each check is chosen so that a plausible slip in the restatement (a dropped term, a wrong sign or index, a
transposed operand, a wrong draw order) fails it."""
import math

import pytest
import torch

from oracle import psgd_oracle as O
from tests.metrics import rel_err_floor, rel_err_norm

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


@pytest.mark.parametrize("d,k,seed", [(40, 8, 0), (96, 24, 1), (200, 48, 2)])
def test_nlb_spd_of_a_gram_product_in_k_space(d, k, seed):
    """The library's bound of A = P P^T (psgdk_norm_lower_bound_gram) never forms A. Its iterate V (32 x d) is kept as
    X = V P (32 x k), each product V A / nf as X <- s (X H / nf) with H = P^T P, and each squared row norm of V as the
    row dot of X H with X. In float64 that sequence gives the oracle's bound of P P^T to rounding."""
    g = torch.Generator().manual_seed(seed)
    P = torch.randn(d, k, generator=g, dtype=torch.float64) * torch.linspace(0.2, 2.0, k, dtype=torch.float64)
    V = torch.randn(32, d, generator=g, dtype=torch.float64)
    sn = O.smallest_normal(torch.float64)
    H = P.T @ P
    nf = (P * P).sum(dim=1).amax() + sn          # the diagonal of P P^T
    j = int(torch.argmax(((P @ H) * P).sum(dim=1)))  # its squared row norms, rowsum((P H) * P)
    row = (P @ P[j]) / nf                        # row j of P P^T / nf
    V0 = row + torch.sgn((row * V).sum(dim=1, keepdim=True)) * V
    Y = V0 @ P                                   # U0; the first product scales by 1 / nf
    scale = torch.full((32, 1), 1 / float(nf), dtype=torch.float64)
    for it in range(4):
        X = scale * Y
        Y = X @ H
        dots = (Y * X).sum(dim=1, keepdim=True)  # squared row norms of the d-space iterate
        scale = (1 / (dots.sqrt() + sn) if it % 2 == 0 else torch.ones_like(dots)) / nf
    got = float(nf * dots.amax().sqrt())
    want = float(O.norm_lower_bound(P @ P.T, V, skew=False))
    assert got == pytest.approx(want, rel=1e-10)


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


# --------------------------------------------------------------------------- closed forms of the step's remaining rules
# Each check below is also run against the oracle with a planted mistake (a swapped betaL / 1 - betaL, a flipped
# sign, the other update order), which it must reject: a check that a slip shared by two restatements passes pins
# nothing.
def _noised(G, N, damping):
    return G + (damping + torch.finfo(G.dtype).eps * G.abs()) * N


def _diag_first_step_err(seed=4, lr=0.1, damping=1e-9, oracle_lr=None):
    """Both factors diagonal (12 x 10 with max_skew 0.5: 144, 100 > 60), q = ones, L = 0. The first update is
    Pg = X, term1_0 = rowsum(X^2), term1_1 = colsum(X^2), ell_i = max term1_i + numel / d_i, L_i = ell_i and
    q_i = 1 - (lr / ell_i)(term1_i - numel / d_i) (psgd_pro.py:126-130). Returns the worst relative error of the
    oracle's q and L against that closed form."""
    m, n = 12, 10
    G = torch.randn(m, n, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    W = torch.zeros(m, n, dtype=torch.float64)
    ora = O.OracleKron([W], preconditioner_max_skew=0.5, preconditioner_init_scale=1.0, seed=seed,
                       lr_preconditioner=oracle_lr if oracle_lr is not None else lr, damping=damping,
                       dtype=torch.float64, grad_clip_max_amps=(1e9, 1e9))
    ora.step([G])
    assert ora.Q[0][0].dim() == 1 and ora.Q[0][1].dim() == 1
    gen = torch.Generator().manual_seed(seed)
    torch.rand([], generator=gen)
    X = _noised(G, torch.randn(m, n, generator=gen, dtype=torch.float32).double(), damping)
    err = 0.0
    for i, (t1, d) in enumerate((((X * X).sum(1), m), ((X * X).sum(0), n))):
        t2 = m * n / d
        ell = float(t1.max()) + t2
        q = 1.0 - lr / ell * (t1 - t2)
        err = max(err, rel_err_norm(ora.Q[0][i], q), abs(float(ora.L[0][i]) - ell) / ell)
    return err


def test_diag_factor_first_step_closed_form():
    assert _diag_first_step_err() < 1e-13
    assert _diag_first_step_err(oracle_lr=-0.1) > 1e-3  # planted: the update's sign flipped


def _second_step_err(betaL_oracle=0.9, shape=(12, 10), skew=0.5, lr=0.1, seed=6):
    """Step 1 on a random gradient, then step 2 on G = 0 with damping 0: X = 0, so Pg = 0, term1 = 0 and the norm
    bound of the zero matrix is 0, hence ell = numel / d for every factor. L_1 = ell_1 > numel / d, so the EMA takes
    its first branch, L_2 = betaL L_1 + (1 - betaL) numel / d (psgd_pro.py:129,134), and the update scales the
    factor: q_2 = q_1 (1 + lr (numel / d) / L_2) for diagonal (psgd_pro.py:130) and dense factors (psgd_pro.py:135;
    Q_1 is symmetric up to rounding, the Procrustes fixed point). betaL 0.9 throughout; betaL_oracle plants a
    swap."""
    beta = 0.9
    G = torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)
    W = torch.zeros(shape, dtype=torch.float64)
    ora = O.OracleKron([W], preconditioner_max_skew=skew, preconditioner_init_scale=1.0, seed=seed,
                       betaL=betaL_oracle, lr_preconditioner=lr, dtype=torch.float64, grad_clip_max_amps=(1e9, 1e9))
    ora.step([G])
    L1 = [float(l) for l in ora.L[0]]
    Q1 = [q.clone() for q in ora.Q[0]]
    ora.damping = 0.0
    ora.step([torch.zeros(shape, dtype=torch.float64)])
    err = 0.0
    numel = math.prod(shape)
    for i, d in enumerate(shape):
        t2 = numel / d
        assert L1[i] > t2 * (1 + 1e-6)
        L2 = beta * L1[i] + (1 - beta) * t2
        err = max(err, abs(float(ora.L[0][i]) - L2) / L2,
                  rel_err_norm(ora.Q[0][i], Q1[i] * (1 + lr * t2 / L2)))
    return err


@pytest.mark.parametrize("shape,skew", [((12, 10), 0.5), ((6, 9), math.inf)], ids=["diag", "dense"])
def test_smoothness_ema_second_step_closed_form(shape, skew):
    assert _second_step_err(shape=shape, skew=skew) < 1e-12
    assert _second_step_err(betaL_oracle=0.1, shape=shape, skew=skew) > 1e-3  # planted: betaL and 1 - betaL swapped


def test_smoothness_ema_planted_swap_in_the_rule(monkeypatch):
    """The same closed form against the oracle whose EMA rule itself has betaL and 1 - betaL swapped."""
    monkeypatch.setattr(O, "smoothness_ema", lambda L, ell, b: torch.maximum((1 - b) * L + b * ell, ell))
    assert _second_step_err() > 1e-3


def _momentum_err(steps=12, momentum=0.9):
    """momentum 0.9 with no preconditioner update (probability 0) from Q = I: the buffer after step t is
    m_t = beta_t m_{t-1} + (1 - beta_t) g_t with beta_t = min((t - 1) / t, 0.9) (psgd_pro.py:334-341), i.e. the
    running mean of g_1..g_t for t <= 10, then 0.9 m_{t-1} + 0.1 g_t; the preconditioned gradient is m_t itself
    (P = I) and the parameter moves by -lr m_t (no clipping at this scale). Returns the worst relative error."""
    shape = (5, 7)
    gen = torch.Generator().manual_seed(2)
    gs = [0.01 * torch.randn(shape, generator=gen, dtype=torch.float64) for _ in range(steps)]
    W = torch.zeros(shape, dtype=torch.float64)
    ora = O.OracleKron([W], preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, momentum=momentum,
                       preconditioner_update_probability=0.0, lr_params=0.5, dtype=torch.float64, seed=1)
    err, Wref, mref = 0.0, torch.zeros(shape, dtype=torch.float64), None
    for t, g in enumerate(gs, start=1):
        ora.step([g])
        mref = torch.stack(gs[:t]).mean(0) if t <= 10 else 0.9 * mref + 0.1 * g
        Wref = Wref - 0.5 * mref
        err = max(err, rel_err_norm(ora.ms[0], mref), rel_err_norm(ora.pre[0], mref), rel_err_norm(W, Wref))
    return err


def test_momentum_closed_form():
    assert _momentum_err() < 1e-13


def test_momentum_planted_swap(monkeypatch):
    """The oracle with m = (1 - beta) m + beta g (beta and 1 - beta swapped) fails the closed form."""
    monkeypatch.setattr(O, "momentum_beta", lambda c, mo: 1 - min(c / (1 + c), mo))
    assert _momentum_err() > 1e-3


def _first_step_dense(G, seed, lr=0.1, damping=1e-9):
    """Closed-form Q_1, Q_2 and L after one optimizer step of a 2-D weight with two dense factors from Q = I,
    replaying OracleKron's draws (update coin, noise, then per factor the SPD and skew starts)."""
    m, n = G.shape
    gen = torch.Generator().manual_seed(seed)
    torch.rand([], generator=gen)
    X = _noised(G, torch.randn(m, n, generator=gen, dtype=torch.float32).double(), damping)
    Qs, Ls = [], []
    for i, d in enumerate((m, n)):
        T = X @ X.T if i == 0 else X.T @ X
        T = (T + T.T) / 2
        V1 = torch.randn(32, d, generator=gen, dtype=torch.float32).double()
        torch.randn(32, d, generator=gen, dtype=torch.float32)
        ell = float(O.norm_lower_bound(T, V1, skew=False)) + m * n / d
        Qs.append(torch.eye(d, dtype=torch.float64) - lr / ell * (T - m * n / d * torch.eye(d, dtype=torch.float64)))
        Ls.append(ell)
    return Qs, Ls


def _order_err(update_first_oracle, update_first_expected, seed=8):
    """Two steps of a 6 x 9 weight with dense factors from Q = I. Update last (psgd_pro.py:363-369): step 1 applies
    the identity preconditioner, pre_1 = G_1, and step 2 applies Q_1 (the closed-form first update), pre_2 =
    Q_1a^T Q_1a G_2 Q_1b^T Q_1b. Update first: pre_1 = Q_1a^T Q_1a G_1 Q_1b^T Q_1b. W moves by -lr pre (no clipping
    at this scale). Returns the worst relative error of pre and W against the expected order's closed form."""
    m, n, lr = 6, 9, 0.01
    gen = torch.Generator().manual_seed(seed)
    G1 = 0.1 * torch.randn(m, n, generator=gen, dtype=torch.float64)
    G2 = 0.1 * torch.randn(m, n, generator=gen, dtype=torch.float64)
    W = torch.zeros(m, n, dtype=torch.float64)
    ora = O.OracleKron([W], preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, seed=seed,
                       lr_params=lr, dtype=torch.float64, update_preconditioner_first=update_first_oracle)
    Qc, _ = _first_step_dense(G1, seed)
    P = [q.T @ q for q in Qc]
    ora.step([G1])
    exp1 = P[0] @ G1 @ P[1] if update_first_expected else G1
    err = max(rel_err_norm(ora.pre[0], exp1), rel_err_norm(W, -lr * exp1))
    if not update_first_expected:
        exp2 = P[0] @ G2 @ P[1]
        ora.step([G2])
        err = max(err, rel_err_norm(ora.pre[0], exp2), rel_err_norm(W, -lr * (exp1 + exp2)))
    return err


@pytest.mark.parametrize("first", [False, True], ids=["update_last", "update_first"])
def test_update_order_closed_form(first):
    assert _order_err(first, first) < 1e-12
    assert _order_err(not first, first) > 1e-3  # planted: the other order


def test_clip_passes_non_finite_values_through():
    """psgd_pro.py:371-381 with torch semantics: a NaN element makes the RMS NaN, so no rescale, and the clamp
    keeps the NaN (the parameter gets NaN there, the other elements their normal step); an inf element makes the
    RMS inf, so the rescale multiplies by 2 / inf = 0 (inf * 0 = NaN at that element, 0 elsewhere)."""
    g = torch.tensor([0.5, float("nan"), -30.0, 1.0])
    p = torch.ones(4)
    out = O.clip_and_update(p, g.clone(), 0.1, 2.0, 10.0)
    assert math.isnan(float(out[1])) and math.isnan(float(p[1]))
    assert torch.equal(out[[0, 2, 3]], torch.tensor([0.5, -10.0, 1.0]))
    assert torch.allclose(p[[0, 2, 3]], torch.tensor([0.95, 2.0, 0.9]))
    g = torch.tensor([0.5, float("inf"), -3.0, 1.0])
    p = torch.ones(4)
    out = O.clip_and_update(p, g.clone(), 0.1, 2.0, 10.0)
    assert math.isnan(float(out[1])) and math.isnan(float(p[1]))
    assert torch.equal(out[[0, 2, 3]], torch.zeros(3)) and torch.equal(p[[0, 2, 3]], torch.ones(3))


# --------------------------------------------------------------------------- the rounded-operand oracle (bf16 floor)
def _rounded_run(rounding, shapes=((24, 40), (40, 24), (16,)), skew=math.inf, steps=4, r2=False):
    gen = torch.Generator().manual_seed(12)
    W = [torch.zeros(s, dtype=torch.float64) for s in shapes]
    ora = O.OracleKron(W, preconditioner_max_skew=skew, preconditioner_init_scale=1.0, seed=5, dtype=torch.float64,
                       rounding=rounding, r2=r2)
    for _ in range(steps):
        ora.step([0.01 * torch.randn(s, generator=gen, dtype=torch.float64) for s in shapes])
    return ora


@pytest.mark.parametrize("skew", [math.inf, 1.0], ids=["dense", "mixed"])
@pytest.mark.parametrize("r2", [False, True], ids=["step2", "r2"])
def test_rounded_oracle_reduces_to_oracle_and_scales_with_unit_roundoff(skew, r2):
    """With the identity as its rounding the rounded-operand oracle is the oracle (the same algebra, associated as
    the bf16 kernels associate it); its distance from the oracle grows with the rounding's unit roundoff (float32:
    ~1e-7, bfloat16: ~1e-3), so a rounding point that is missing or applied to the wrong operand shows up."""
    base = _rounded_run(None, skew=skew, r2=r2)
    ident = _rounded_run(lambda x: x, skew=skew, r2=r2)
    f32 = _rounded_run(lambda x: x.float().double(), skew=skew, r2=r2)
    b16 = _rounded_run(O.round_bf16, skew=skew, r2=r2)

    def dist(o):  # per-element on Q (floor 1e-3 max), normwise on the preconditioned gradient
        dq = max(max(rel_err_floor(q, qb) for q, qb in zip(Qa, Qb)) for Qa, Qb in zip(o.Q, base.Q))
        return max(dq, max(rel_err_norm(a, b) for a, b in zip(o.pre, base.pre)))
    assert dist(ident) < 1e-12
    e32, e16 = dist(f32), dist(b16)
    assert 1e-9 < e32 < 1e-6, e32
    assert 1e-4 < e16 < 2e-2, e16
    assert 1e3 < e16 / e32 < 1e6, (e16, e32)  # bf16 / fp32 unit roundoff = 2^16


def test_package_flop_count_matches_the_oracle():
    """The measurement's FLOP count (psgd_pro_amd.flops, used by bench.py) equals the oracle's on every config shape,
    dense and diagonal sides, step2 and r2."""
    from psgd_pro_amd import flops as F
    shapes = [(1024, 1024), (768, 2304), (768, 768), (768, 3072), (3072, 768), (4096, 4096), (4096, 14336), (77, 5)]
    for m, n in shapes:
        for d1 in (True, False):
            for d2 in (True, False):
                for r2 in (False, True):
                    assert F.flops_2d(m, n, d1, d2, r2) == O.flops_2d(m, n, d1, d2, r2)
        for skew in (1.0, math.inf):
            for d in (m, n):
                assert F.is_dense(d, m * n, 8192, skew) == O.is_dense(d, m * n, 8192, skew)
