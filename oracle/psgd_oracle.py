"""CPU oracle for the PSGD-Kron "Pro" preconditioner (dQ = Q^0.5 E Q^1.5).

TEST INFRASTRUCTURE ONLY. This module is the reference against which results are compared: it is imported by
tests/, by __graft_entry__.smoke() and by bench.py's cpu_baseline leg, and by nothing under psgd_pro_amd/. The
product path never calls it.

A clean-room restatement, in plain PyTorch on the CPU (float64 or float32), of the arithmetic in the reference's
psgd_pro.py (line numbers below are that file's unless another file is named). Every random draw comes from one
explicit CPU generator in the order psgd_pro.py makes them on the CPU, so a GPU run that is fed the same draws can be
compared value by value.

Pinning (see tests/test_oracle.py): norm bounds against torch.linalg spectral norms (lower bound, exact for rank-1),
the Procrustes step against its fixed point (symmetric Q) and the r2 identity, the factor rule and the first update
from Q = I against closed forms, balancing against the invariance of the Kronecker product, the whole step in
float32 against the same step in float64, and the clip against its closed form. The one part no check fixes exactly
is opt_einsum's contraction order for the preconditioned gradient (psgd_pro.py:123,235-238): this restatement
multiplies P1 @ (X @ P2) with P_i = Q_i^T Q_i, which differs from the reference only in rounding order.
"""
import math

import torch

K_SUBSPACE = 32       # rows of the random start V in the norm lower bounds (psgd_pro.py:19,43 default k=32)
HALF_ITERS = 2        # psgd_pro.py:19,43 default half_iters=2
MAX_PROCRUSTES = 1.0 / 8  # psgd_pro.py:71 max_step_size
BALANCE_PROB = 0.01   # psgd_pro.py:138


class Draws:
    """The random stream of psgd_pro.py on one CPU generator.

    Order per optimizer step (psgd_pro.py:345,123,35,59,138): one uniform coin for "update this step"; then, per
    parameter whose preconditioner is updated, one normal tensor shaped like the gradient (damping noise), then per
    dense factor in dimension order a (32, d) normal block for the SPD norm bound of term1 followed by a (32, d)
    block for the skew norm bound inside the Procrustes step; then one uniform coin for balancing."""

    def __init__(self, seed=0):
        self.gen = torch.Generator().manual_seed(seed)

    def coin(self):
        return float(torch.rand([], generator=self.gen))

    def normal(self, shape, dtype=torch.float32):
        return torch.randn(tuple(shape), generator=self.gen, dtype=dtype)

    def state(self):
        return self.gen.get_state()

    def set_state(self, s):
        self.gen.set_state(s)


def smallest_normal(dtype):
    return torch.finfo(dtype).smallest_normal


def is_dense(size, numel, max_size, max_skew):
    """Factor rule of init_kron (psgd_pro.py:189): a dimension gets a dense factor unless size <= 1, size > max_size
    or size**2 > max_skew * numel."""
    return not (size <= 1 or size > max_size or size ** 2 > max_skew * numel)


def init_factors(shape, scale, max_size=math.inf, max_skew=1.0, dtype=torch.float32):
    """Q and L of init_kron (psgd_pro.py:141-210): Q_i = scale**(1/order) * I (dense) or * ones (diagonal),
    a scalar tensor gets Q = [scale]; L_i = 0 in at least single precision (lift2single, psgd_pro.py:67-69,188)."""
    ldtype = torch.float32 if torch.finfo(dtype).eps > 1e-6 else dtype
    if len(shape) == 0:
        return [torch.full([], float(scale), dtype=dtype)], [torch.zeros([], dtype=ldtype)]
    numel = math.prod(shape)
    s = scale ** (1.0 / len(shape))
    Q, L = [], []
    for d in shape:
        Q.append(s * (torch.eye(d, dtype=dtype) if is_dense(d, numel, max_size, max_skew) else torch.ones(d, dtype=dtype)))
        L.append(torch.zeros([], dtype=ldtype))
    return Q, L


def init_scale_on_the_fly(grads, damping):
    """psgd_pro.py:329-331: (max_p mean|g|^4 + damping^4)^(-1/8)."""
    m = max(float(torch.mean(g.double().abs() ** 4)) for g in grads)
    return (m + damping ** 4) ** (-1.0 / 8)


def norm_lower_bound(A, V, skew):
    """psgd_pro.py:19-41 (SPD, skew=False) and :43-65 (skew-symmetric, skew=True) with the random start V (32 x n)
    passed in. nf = max diagonal (SPD) or max |A_ij| (skew), plus the smallest normal; the rows of V are first
    pulled towards the largest row of A/nf (sign of their inner product), then two half-iterations of
    V <- V A, normalise rows, V <- V A; the bound is nf * max row norm of V."""
    sn = smallest_normal(A.dtype)
    nf = (A.abs().amax() if skew else A.diagonal().amax()) + sn
    An = A / nf
    j = int(torch.argmax(torch.linalg.vector_norm(An, dim=1)))
    row = An[j]
    V = row + torch.sgn((row * V).sum(dim=1, keepdim=True)) * V
    for _ in range(HALF_ITERS):
        V = V @ An
        V = V / (torch.linalg.vector_norm(V, dim=1, keepdim=True) + sn)
        V = V @ An
    return nf * torch.linalg.vector_norm(V, dim=1).amax()


def procrustes_step2(Q, V, max_step=MAX_PROCRUSTES):
    """In-place online Procrustes rotation, psgd_pro.py:71-94: R = Q^T - Q scaled by its norm lower bound,
    a = min(-tr(RQ)/tr(RRQ), max_step) when tr(RRQ) < 0 else max_step, Q += a (RQ + a/2 RRQ)."""
    R = Q.T - Q
    R = R / (norm_lower_bound(R, V, skew=True) + smallest_normal(R.dtype))
    RQ = R @ Q
    RRQ = R @ RQ
    t1 = RQ.diagonal().sum()
    t2 = RRQ.diagonal().sum()
    a = torch.where(t2 < 0, torch.clamp(-t1 / t2, max=max_step), torch.tensor(max_step, dtype=Q.dtype))
    Q.add_(a * (RQ + 0.5 * a * RRQ))
    return a


def procrustes_step_r2(Q, V, max_step=MAX_PROCRUSTES):
    """psgd_pro_fast.py:141-153: the same rotation with Rn = Q - Q^T = -R and S = Rn^T Rn = -R R, so that
    tr(RQ) = sum(Rn * Q), tr(RRQ) = -sum(S * Q) and Q + aRQ + a^2/2 RRQ = Q - (a Rn + a^2/2 S) Q."""
    Rn = Q - Q.T
    Rn = Rn / (norm_lower_bound(Rn, V, skew=True) + smallest_normal(Rn.dtype))
    S = Rn.T @ Rn
    t1 = (Rn * Q).sum()
    t2 = -(S * Q).sum()
    a = torch.where(t2 < 0, torch.clamp(-t1 / t2, max=max_step), torch.tensor(max_step, dtype=Q.dtype))
    Q.sub_((a * Rn + 0.5 * a * a * S) @ Q)
    return a


def balance(Q):
    """psgd_pro.py:96-105: rescale the factors to the geometric mean of their max-abs values (in place)."""
    if len(Q) < 2:
        return
    norms = [q.abs().amax() for q in Q]
    g = torch.prod(torch.stack(norms)) ** (1.0 / len(Q))
    for q, n in zip(Q, norms):
        q.mul_(g / n)


def _mode_apply(X, M, i):
    """Contract dimension i of X with the symmetric matrix M (M's second index)."""
    return torch.movedim(torch.tensordot(M, X, dims=([1], [i])), 0, i)


def precondition(Q, G):
    """Q_1^T Q_1 x_1 ... x_n Q_n^T Q_n applied to G (the exprP contraction of psgd_pro.py:107-112,123,237-238):
    dense factors contract their dimension with P_i = Q_i^T Q_i, diagonal ones scale it by q_i * q_i. For a 2-D G
    with two dense factors this is P1 @ G @ P2."""
    if G.dim() == 0:
        return Q[0] * Q[0] * G
    if G.dim() == 2 and all(q.dim() == 2 for q in Q):
        P1, P2 = Q[0].T @ Q[0], Q[1].T @ Q[1]
        return P1 @ (G @ P2)
    X = G
    for i, q in enumerate(Q):
        if q.dim() == 2:
            X = _mode_apply(X, q.T @ q, i)
        else:
            shape = [1] * G.dim()
            shape[i] = q.shape[0]
            X = X * (q * q).view(shape)
    return X


def gram(Pg, i, dense):
    """exprGs[i] of psgd_pro.py:125,205,228: Pg Pg^T along dimension i (dense) or the sums of squares of the other
    dimensions (diagonal); Pg * Pg for a scalar."""
    if Pg.dim() == 0:
        return Pg * Pg
    X = torch.movedim(Pg, i, 0).reshape(Pg.shape[i], -1)
    return X @ X.T if dense else (X * X).sum(dim=1)


def smoothness_ema(L, ell, betaL):
    """The Lipschitz smoothness estimate of psgd_pro.py:129,134: L <- max(betaL L + (1 - betaL) ell, ell)."""
    return torch.maximum(betaL * L + (1 - betaL) * ell, ell)


def momentum_beta(counter, momentum):
    """psgd_pro.py:335: the momentum EMA factor of step `counter` (0-based), min(c / (1 + c), momentum): the buffer
    is the running mean of the gradients while c / (1 + c) < momentum."""
    return min(counter / (1 + counter), momentum)


def round_bf16(x):
    """x rounded to bfloat16 (round to nearest even) and returned in x's dtype."""
    return x.to(torch.bfloat16).to(x.dtype)


def precondition_rounded(Q, X, rd, final):
    """P1 X P2 of a 2-D tensor with the operands of each product rounded by rd, where bf16-operand kernels round
    them: a dense factor's P = rd(rd(Q)^T rd(Q)) (P is formed from the rounded Q and stored rounded), a diagonal
    factor's p = q * q scales X before the rounding (the scaled X is the product's operand), X P2 is rounded (the
    second product's operand), and the result is rounded when `final` (Pg, stored rounded) but not for the apply
    (its output is the float32 preconditioned gradient). Tensors that are not 2-D, and weights whose factors are
    both diagonal (no product), take `precondition`."""
    if X.dim() != 2 or len(Q) != 2 or (Q[0].dim() < 2 and Q[1].dim() < 2):
        return precondition(Q, X)
    d1, d2 = Q[0].dim() == 2, Q[1].dim() == 2
    P1 = rd(rd(Q[0]).T @ rd(Q[0])) if d1 else Q[0] * Q[0]
    P2 = rd(rd(Q[1]).T @ rd(Q[1])) if d2 else Q[1] * Q[1]
    if d1 and d2:
        out = P1 @ rd(rd(X) @ P2)
    elif d1:
        out = P1 @ rd(X * P2[None, :])
    else:
        out = rd(P1[:, None] * X) @ P2
    return rd(out) if final else out


def procrustes_step2_rounded(Q, V, rd, max_step=MAX_PROCRUSTES):
    """procrustes_step2 with rounded operands: R = rd(Q^T - Q) (stored rounded), its bound's start V rounded,
    RQ = rs R rd(Q) with rs = 1 / (bound + smallest normal), tr(RQ) from RQ before rounding, RRQ = rs R rd(RQ) and
    Q += a (rd(RQ) + a/2 RRQ) (the second product reads RQ rounded, the update adds that same RQ)."""
    R = rd(Q.T - Q)
    rs = 1.0 / (norm_lower_bound(R, V, skew=True) + smallest_normal(R.dtype))
    RQ = (R @ rd(Q)) * rs
    t1 = RQ.diagonal().sum()
    RQ = rd(RQ)
    RRQ = (R @ RQ) * rs
    t2 = RRQ.diagonal().sum()
    a = torch.where(t2 < 0, torch.clamp(-t1 / t2, max=max_step), torch.tensor(max_step, dtype=Q.dtype))
    Q.add_(a * (RQ + 0.5 * a * RRQ))
    return a


def procrustes_step_r2_rounded(Q, V, rd, max_step=MAX_PROCRUSTES):
    """procrustes_step_r2 with rounded operands: Rn = rd(Q - Q^T), S = rd(rs^2 Rn^T Rn) (stored rounded),
    M = rd(a rs Rn + a^2/2 S) and Q -= M rd(Q)."""
    Rn = rd(Q - Q.T)
    rs = 1.0 / (norm_lower_bound(Rn, V, skew=True) + smallest_normal(Rn.dtype))
    S = rd((Rn.T @ Rn) * rs * rs)
    t1 = (Rn * Q).sum() * rs
    t2 = -(S * Q).sum()
    a = torch.where(t2 < 0, torch.clamp(-t1 / t2, max=max_step), torch.tensor(max_step, dtype=Q.dtype))
    Q.sub_(rd(a * rs * Rn + 0.5 * a * a * S) @ rd(Q))
    return a


def update_preconditioner(Q, L, G, draws, lr=0.1, betaL=0.9, damping=1e-9, grad_eps=None, r2=False, trace=None,
                          draw_dtype=torch.float32, noise_dtype=None, rd=None):
    """psgd_pro.py:114-139 (update_precond_kron_whiten_q0p5eq1p5), in place on Q and L, with the draws taken from
    `draws` in psgd_pro.py's order. The normals are drawn in draw_dtype (psgd_pro.py draws them in the gradient's
    dtype: float32 for the float32 models every comparison here uses) and cast to the working dtype; noise_dtype
    (default draw_dtype) overrides the dtype of the gradient-shaped noise alone, as psgd_pro_fast.draw_normals draws
    it like the gradient and the 32 x d starts like the factors (psgd_pro_fast.py:200-206): a bfloat16 gradient
    upcast for this oracle passes bfloat16. grad_eps overrides finfo(G.dtype).eps in the damping scale (the
    reference uses the gradient's own dtype; a bfloat16 gradient upcast for this oracle passes bfloat16's eps).
    rd (optional, e.g. round_bf16) rounds the operands of every product and the stored intermediates at the points
    where bf16-operand kernels round them (see precondition_rounded, procrustes_step2_rounded); None computes in the
    working dtype throughout, as the reference does."""
    eps = torch.finfo(G.dtype).eps if grad_eps is None else grad_eps
    numel = G.numel()
    damp = damping + eps * G.abs()
    noise = draws.normal(G.shape, noise_dtype or draw_dtype).to(G.dtype)
    Pg = precondition(Q, G + damp * noise) if rd is None else precondition_rounded(Q, G + damp * noise, rd, True)
    for i, q in enumerate(Q):
        if q.dim() < 2:
            term1 = gram(Pg, i, dense=False)
            term2 = numel / max(q.numel(), 1)
            ell = term1.amax() + term2
            L[i].copy_(smoothness_ema(L[i], ell, betaL))
            q.mul_(1 - lr / L[i] * (term1 - term2))
        else:
            d = q.shape[0]
            term1 = gram(Pg, i, dense=True)
            term2 = numel / d
            V1 = draws.normal((K_SUBSPACE, d), draw_dtype).to(q.dtype)
            if rd is not None:
                term1, V1 = rd(term1), rd(V1)
            ell = norm_lower_bound(term1, V1, skew=False) + term2
            L[i].copy_(smoothness_ema(L[i], ell, betaL))
            q.sub_(lr / L[i] * (term1 @ (q if rd is None else rd(q)) - term2 * q))
            V2 = draws.normal((K_SUBSPACE, d), draw_dtype).to(q.dtype)
            if rd is None:
                a = (procrustes_step_r2 if r2 else procrustes_step2)(q, V2)
            else:
                a = (procrustes_step_r2_rounded if r2 else procrustes_step2_rounded)(q, rd(V2), rd)
            if trace is not None:
                trace.append(dict(factor=i, ell=float(ell), L=float(L[i]), a=float(a)))
    if draws.coin() < BALANCE_PROB:
        balance(Q)
        if trace is not None:
            trace.append(dict(balanced=True))


def clip_and_update(param, g, lr_params, max_avg_amp=2.0, max_element_amp=10.0):
    """psgd_pro.py:371-381: scale g so its RMS is at most max_avg_amp, clamp to +-max_element_amp, param -= lr g.
    Returns the clipped g."""
    avg = torch.sqrt(torch.mean(g * g))
    if avg > max_avg_amp:
        g = g * (max_avg_amp / avg)
    g = g.clamp(-max_element_amp, max_element_amp)
    param.sub_(lr_params * g.view_as(param))
    return g


class OracleKron:
    """KronWhiten.step of psgd_pro.py:251-384 on the CPU with the gradients passed in (no closure), for 0-D, 1-D,
    2-D and higher-order parameters. `pre` keeps the unclipped preconditioned gradients of the last step,
    `clipped` the clipped ones. rounding=round_bf16 gives the floor a bf16-operand implementation cannot beat: the
    same step with every product's operands rounded to bfloat16 where those kernels round them (its distance from
    the float32 oracle measures what bf16 operands alone cost)."""

    def __init__(self, params, preconditioner_max_size=math.inf, preconditioner_max_skew=1.0,
                 preconditioner_init_scale=None, lr_params=0.001, lr_preconditioner=0.1, betaL=0.9, damping=1e-9,
                 momentum=0.0, grad_clip_max_amps=(2.0, 10.0), preconditioner_update_probability=1.0,
                 update_preconditioner_first=True, whiten_grad=True, seed=0, dtype=None, grad_eps=None, r2=False,
                 noise_dtype=None, rounding=None):
        self.params = list(params)  # updated in place
        self.max_size, self.max_skew = preconditioner_max_size, preconditioner_max_skew
        self.lr_params, self.lr_preconditioner = lr_params, lr_preconditioner
        self.betaL, self.damping = betaL, damping
        self.momentum = momentum if 0 < momentum < 1 else 0.0
        self.grad_clip_max_amps = grad_clip_max_amps
        self.update_probability = preconditioner_update_probability
        self.update_first = update_preconditioner_first
        self.whiten_grad = whiten_grad
        self.dtype = dtype
        self.grad_eps, self.r2 = grad_eps, r2
        self.noise_dtype = noise_dtype
        self.rounding = rounding  # e.g. round_bf16: operands rounded where bf16-operand kernels round them
        self.draws = Draws(seed)
        self.Q = self.L = None
        self.ms, self.counter_m = None, 0
        self.trace = []
        self.pre, self.clipped = None, None
        if preconditioner_init_scale is not None:
            self._init([p.squeeze() for p in self.params], preconditioner_init_scale)

    def _init(self, grads, scale):
        dt = lambda g: self.dtype or g.dtype
        fac = [init_factors(tuple(g.shape), scale, self.max_size, self.max_skew, dt(g)) for g in grads]
        self.Q = [f[0] for f in fac]
        self.L = [f[1] for f in fac]

    def _update(self, srcs):
        for Q, L, g in zip(self.Q, self.L, srcs):
            update_preconditioner(Q, L, g, self.draws, lr=self.lr_preconditioner, betaL=self.betaL,
                                  damping=self.damping, grad_eps=self.grad_eps, r2=self.r2, trace=self.trace,
                                  noise_dtype=self.noise_dtype, rd=self.rounding)

    @torch.no_grad()
    def step(self, grads):
        grads = [g.squeeze() for g in grads]
        if self.dtype is not None:
            grads = [g.to(self.dtype) for g in grads]
        if self.Q is None:
            self._init(grads, init_scale_on_the_fly(grads, self.damping))
        if self.momentum > 0:  # psgd_pro.py:334-343
            beta = momentum_beta(self.counter_m, self.momentum)
            self.counter_m += 1
            if self.ms is None:
                self.ms = [torch.zeros_like(g) for g in grads]
            for m, g in zip(self.ms, grads):
                m.mul_(beta).add_(g, alpha=1 - beta)
        else:
            self.ms, self.counter_m = None, 0
        upd = self.draws.coin() < self.update_probability
        src = grads if self.whiten_grad else self.ms
        if upd and self.update_first:
            self._update(src)
        pc = precondition if self.rounding is None else (lambda Q, m: precondition_rounded(Q, m, self.rounding, False))
        self.pre = [pc(Q, m) for Q, m in zip(self.Q, self.ms if self.momentum > 0 else grads)]
        if upd and not self.update_first:
            self._update(src)
        max_avg, max_el = self.grad_clip_max_amps
        self.clipped = [clip_and_update(p, g.clone(), self.lr_params, max_avg, max_el)
                        for p, g in zip(self.params, self.pre)]
        return self.pre


def flops_2d(m, n, dense1=True, dense2=True, r2=False):
    """Algorithmic FLOPs of one update + apply of an m x n parameter with the P = Q^T Q cached decomposition:
    two P1 G P2 applies, the term1 SYRKs, term1 @ Q, the Procrustes products, the P refresh and the norm bounds
    (5 passes of 2 * 32 flops per stored element, 4 V @ A plus one row-norm pass, counted as 514 d^2)."""
    f = 0
    f += 2 * ((2 * m * m * n if dense1 else m * n) + (2 * m * n * n if dense2 else m * n))  # update + apply
    for d, o, dense in ((m, n, dense1), (n, m, dense2)):
        if not dense:
            continue
        f += d * (d + 1) * o       # term1 SYRK
        f += 2 * d ** 3            # term1 @ Q
        f += (3 if r2 else 4) * d ** 3  # Procrustes
        f += d * d * (d + 1)       # P = Q^T Q refresh (SYRK)
        f += 514 * d * d           # two norm lower bounds
    return f
