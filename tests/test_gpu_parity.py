"""KronWhiten on the HIP engine against the CPU oracle, both fed psgd_pro.py's draw stream from one seed.

Tolerances (per element, |x - y| / max(|y|, 1e-3 max|y|), on Q, on the preconditioned gradient and on the
parameters): fp32 path 1e-5 against the float64 oracle, within a small factor of what the float32 oracle itself
scores against float64 on the same inputs; bf16 path 2e-2 against the float32 oracle on the same gradients
upcast (damping scaled with bfloat16's eps, as the reference does for a bfloat16 gradient).
"""
import math

import pytest
import torch

from oracle import psgd_oracle as O
from psgd_pro_amd import KronWhiten
from psgd_pro_amd import _lib as L
from tests.metrics import rel_err_floor, rel_err_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL32 = 1e-5
TOL16 = 2e-2


def grads_for(shapes, step, dtype=torch.float32):
    g = torch.Generator().manual_seed(1000 + step)
    return [(0.01 * torch.randn(*s, generator=g)).to(dtype) for s in shapes]


def run_pair(shapes, steps, seed=0, skew=1.0, max_size=math.inf, prec="fp32", gdt=torch.float32, odt=torch.float64,
             grad_eps=None, momentum=0.0, update_first=True, tri=None, whiten_grad=True):
    Wg = [torch.zeros(s, device=DEV, dtype=torch.float32, requires_grad=True) for s in shapes]
    Wo = [torch.zeros(s, dtype=odt) for s in shapes]
    kw = dict(preconditioner_max_skew=skew, preconditioner_max_size=max_size, preconditioner_init_scale=1.0,
              momentum=momentum, update_preconditioner_first=update_first, whiten_grad=whiten_grad)
    opt = KronWhiten(Wg, precision=prec, draws="host", seed=seed, tri=tri, **kw)
    opt.capture = True
    ora = O.OracleKron(Wo, seed=seed, dtype=odt, grad_eps=grad_eps, **kw)
    worst = dict(Q=0.0, pre=0.0, W=0.0, L=0.0)
    for t in range(steps):
        gs = grads_for(shapes, t, gdt)
        opt.step_math([g.to(DEV) for g in gs])
        ora.step([g.to(odt) for g in gs])
        torch.cuda.synchronize()
        for i in range(len(shapes)):
            Qg, Lg = opt.factors(i)
            for qg, qo in zip(Qg, ora.Q[i]):
                worst["Q"] = max(worst["Q"], rel_err_floor(qg, qo))
            for lg, lo in zip(Lg, ora.L[i]):
                worst["L"] = max(worst["L"], abs(float(lg) - float(lo)) / max(abs(float(lo)), 1e-30))
            worst["pre"] = max(worst["pre"], rel_err_floor(opt.pre[i], ora.pre[i]))
            worst["W"] = max(worst["W"], rel_err_floor(Wg[i].detach(), Wo[i]))
    return worst, opt, ora


@pytest.mark.parametrize("shapes,skew", [
    ([(64, 96)], math.inf),                 # two dense factors
    ([(96, 64)], 1.0),                      # diagonal rows (96^2 > 6144), dense columns
    ([(200, 136)], math.inf),               # ragged sizes
    ([(128,)], math.inf),                   # a vector with a dense factor
    ([(77,)], 1.0),                         # a vector with a diagonal factor
    ([()], 1.0),                            # a scalar
    ([(48, 64), (48, 64), (32,), (64, 48), ()], math.inf),  # grouped same-shape parameters + mixed structure
])
def test_fp32_parity(hip, shapes, skew):
    worst, _, _ = run_pair(shapes, steps=6, skew=skew)
    assert worst["Q"] < TOL32 and worst["pre"] < TOL32 and worst["W"] < TOL32 and worst["L"] < TOL32, worst


def test_fp32_parity_1024_weight(hip):
    """One fp32 1024 x 1024 weight, N(0, 1e-4) gradients, Q = I, update every step, lr 1e-3 (12 steps: Q grows
    about 10% per step until the preconditioned gradient reaches unit RMS)."""
    worst, _, _ = run_pair([(1024, 1024)], steps=12, odt=torch.float32)
    assert worst["Q"] < TOL32 and worst["pre"] < TOL32 and worst["W"] < TOL32, worst


def test_bf16_parity(hip):
    eps16 = torch.finfo(torch.bfloat16).eps
    worst, _, _ = run_pair([(256, 384), (384, 256)], steps=8, skew=math.inf, prec="bf16", gdt=torch.bfloat16,
                           odt=torch.float32, grad_eps=eps16)
    assert worst["Q"] < TOL16 and worst["pre"] < TOL16 and worst["W"] < TOL16, worst


def test_momentum_and_update_last(hip):
    worst, _, _ = run_pair([(64, 80), (80,)], steps=6, skew=math.inf, momentum=0.9, update_first=False)
    assert worst["Q"] < TOL32 and worst["pre"] < TOL32 and worst["W"] < TOL32, worst
    worst, _, _ = run_pair([(64, 80)], steps=5, skew=math.inf, momentum=0.5, whiten_grad=False)
    assert worst["Q"] < TOL32 and worst["pre"] < TOL32 and worst["W"] < TOL32, worst


def test_triangle_storage_parity(hip):
    worst, _, _ = run_pair([(64, 96), (130, 70)], steps=5, skew=math.inf, tri=True)
    assert worst["Q"] < TOL32 and worst["pre"] < TOL32 and worst["W"] < TOL32, worst


def test_balance_matches_oracle(hip):
    """psgdk_kron2d_balance on the optimizer's factors against oracle balance() (the coin fires 1% of steps, so
    it is driven directly here)."""
    W = torch.zeros(64, 96, device=DEV, requires_grad=True)
    opt = KronWhiten([W], preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=1)
    for t in range(3):
        opt.step_math(grads_for([(64, 96)], t))
    Q, _ = opt.factors(0)
    Q[0].mul_(7.0)
    Qo = [q.double().cpu().clone() for q in Q]
    grp = opt._params[0].group
    import ctypes
    L.call_ws(L.lib().psgdk_kron2d_balance, grp.struct, (ctypes.c_int32 * 1)(1), 0, ws=L.Workspace(),
              device=W.device, stream=L.stream_of(W))
    O.balance(Qo)
    torch.cuda.synchronize()
    for qg, qo in zip(Q, Qo):
        assert rel_err_norm(qg, qo) < 1e-6
    P = grp.Ps[0][0]
    assert rel_err_norm(P, Q[0].double().cpu().T @ Q[0].double().cpu()) < 1e-6


def test_state_dict_round_trip(hip):
    shapes = [(64, 96), (32,)]
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=5,
                     momentum=0.9)
    for t in range(3):
        opt.step_math([g.to(DEV) for g in grads_for(shapes, t)])
    st = opt.state_dict()
    W0 = [w.detach().clone() for w in W]
    opt.step_math([g.to(DEV) for g in grads_for(shapes, 3)])
    after = [w.detach().clone() for w in W]
    W2 = [w0.clone().requires_grad_(True) for w0 in W0]
    opt2 = KronWhiten(W2, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=99,
                      momentum=0.9)
    opt2.load_state_dict(st)
    opt2.step_math([g.to(DEV) for g in grads_for(shapes, 3)])
    for a, b in zip(after, W2):
        assert torch.equal(a, b.detach())


def test_step_closure_and_loss_curve(hip):
    """A least-squares model trained 100 steps by both optimizers (each taking gradients of its own parameters)
    gives matching loss curves."""
    g = torch.Generator().manual_seed(0)
    X = torch.randn(256, 48, generator=g)
    Wt = torch.randn(48, 24, generator=g)
    Y = X @ Wt + 0.01 * torch.randn(256, 24, generator=g)
    Wg = torch.zeros(48, 24, device=DEV, requires_grad=True)
    Wo = torch.zeros(48, 24, dtype=torch.float64, requires_grad=True)
    kw = dict(preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, lr_params=0.01)
    opt = KronWhiten([Wg], draws="host", seed=3, **kw)
    ora = O.OracleKron([Wo], seed=3, dtype=torch.float64, **kw)
    Xd, Yd = X.to(DEV), Y.to(DEV)
    lg, lo = [], []
    for _ in range(100):
        loss = opt.step(lambda: ((Xd @ Wg - Yd) ** 2).mean())
        lg.append(float(loss))
        with torch.enable_grad():
            l2 = ((X.double() @ Wo - Y.double()) ** 2).mean()
            (gr,) = torch.autograd.grad(l2, [Wo])
        lo.append(float(l2))
        with torch.no_grad():
            ora.step([gr])
    assert lg[-1] < 0.1 * lg[0]
    for a, b in zip(lg, lo):
        assert abs(a - b) <= 1e-4 * max(abs(b), 1e-12), (a, b)
