"""The optimizer on the benchmarked configurations, at their own sizes and on their own code path.

- One ViT-B/16 block (768x2304, 768x768, 768x3072, 3072x768; bf16 gradients, every factor dense) through the
  benchmarked options (bf16 MFMA, fused groups, side streams) for 5 steps against the float32 oracle fed the same
  draws. Bar, per element (floor 1e-3 max) on Q and on the preconditioned gradient: max(2e-2, 2x the error of the
  rounded-operand oracle), where the rounded-operand oracle is the same step with every product's operands rounded
  to bfloat16 where the bf16 kernels round them: what bf16 operands alone cost against float32 arithmetic.
- The whole 48-weight ViT-B set: the first step from Q = I against its closed form (Pg = X, L = ell,
  Q_i = I - (lr / ell)(term1 - term2 I), the Procrustes step a no-op), then bitwise equality of the benchmarked
  options with one stream and one call per group over two steps; the device-draw path (the benchmark's) checked
  for finite state, L > 0 and bitwise repeatability from one seed.
- Llama-shaped weights (4096x4096, 4096x14336, factors up to 14336^2): the first step against its closed form.
- The end-to-end ViT's parameter set (vit_pro.py's architecture, max_skew 2, momentum 0.9, init scale from the
  gradients) against the oracle for 3 steps, and the model's loss going down over 30 steps of training.
"""
import math

import pytest
import torch

from oracle import psgd_oracle as O
from psgd_pro_amd import KronWhiten
from tests.metrics import rel_err_floor, rel_err_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL16 = 2e-2
VIT_B = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
EPS16 = torch.finfo(torch.bfloat16).eps


def _grads(shapes, step, dtype=torch.bfloat16, scale=0.01):
    g = torch.Generator().manual_seed(1000 + step)
    return [(scale * torch.randn(s, generator=g)).to(dtype) for s in shapes]


def _gpu_state(opt, n):
    fac = [opt.factors(i) for i in range(n)]
    return [f[0] for f in fac], [f[1] for f in fac]


def _worst(Qs, Ls, pre, ref):
    """Per-element errors of Q and pre (floor 1e-3 max), relative error of L, against `ref` (an OracleKron)."""
    out = dict(Q=0.0, pre=0.0, L=0.0)
    for i in range(len(Qs)):
        for q, qo in zip(Qs[i], ref.Q[i]):
            out["Q"] = max(out["Q"], rel_err_floor(q, qo))
        for l, lo in zip(Ls[i], ref.L[i]):
            out["L"] = max(out["L"], abs(float(l) - float(lo)) / abs(float(lo)))
        out["pre"] = max(out["pre"], rel_err_floor(pre[i], ref.pre[i]))
    return out


def test_vitb_block_bf16_parity(hip):
    """The benchmarked path (precision bf16, fuse_groups, streams=3) on one ViT-B block, host draws, 5 steps."""
    shapes = VIT_B
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    kw = dict(preconditioner_max_size=8192, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0)
    opt = KronWhiten(W, precision="bf16", draws="host", seed=0, streams=3, fuse_groups=True, **kw)
    opt.capture = True
    mk = lambda rounding: O.OracleKron([torch.zeros(s) for s in shapes], seed=0, dtype=torch.float32,
                                       grad_eps=EPS16, noise_dtype=torch.bfloat16, rounding=rounding, **kw)
    o32, o16 = mk(None), mk(O.round_bf16)
    gpu, floor = dict(Q=0.0, pre=0.0, L=0.0), dict(Q=0.0, pre=0.0, L=0.0)
    for t in range(5):
        gs = _grads(shapes, t)
        opt.step_math([g.to(DEV) for g in gs])
        o32.step([g.float() for g in gs])
        o16.step([g.float() for g in gs])
        torch.cuda.synchronize()
        Qs, Ls = _gpu_state(opt, len(shapes))
        m = _worst(Qs, Ls, opt.pre, o32)
        f = _worst(o16.Q, o16.L, o16.pre, o32)
        gpu = {k: max(gpu[k], m[k]) for k in gpu}
        floor = {k: max(floor[k], f[k]) for k in floor}
    w = max(rel_err_norm(a, b) for a, b in zip(W, o32.params))
    print(f"ViT-B block, per element vs the float32 oracle: gpu {gpu}, rounded-operand oracle {floor}, "
          f"W normwise {w:.2e}", flush=True)
    for k in ("Q", "pre", "L"):
        assert gpu[k] <= max(TOL16, 2 * floor[k]), (k, gpu, floor)
    assert w < TOL16


def _closed_form_first_step(G16, noise16, V, lr=0.1, damping=1e-9):
    """Q_i and L_i after the first update from Q = I of a bf16 gradient with two dense factors: X is the noised
    gradient rounded to bf16 (the bf16 operands' own rounding), term1 = X X^T or X^T X, ell = the norm lower bound
    of term1 (float64 oracle, the same start V) + numel / d, L = ell (the EMA from 0), Q_i = I - (lr / ell)(term1 -
    numel / d I); Q_i is symmetric, so the Procrustes step leaves it. Products in float32 on the CPU (bf16 X: exact
    products, fp32 accumulation), the bound in float64."""
    m, n = G16.shape
    G = G16.float()
    X = (G + (damping + EPS16 * G.abs()) * noise16.float()).to(torch.bfloat16).float()
    out = []
    for i, d in enumerate((m, n)):
        T = X @ X.T if i == 0 else X.T @ X
        t2 = m * n / d
        ell = float(O.norm_lower_bound(T.double(), V[i].double(), skew=False)) + t2
        Q = -(lr / ell) * T
        Q.diagonal().add_(1.0 + lr / ell * t2)
        out.append((Q, ell))
    return out


def _host_draws(seed, shapes):
    """The draws of KronWhiten(draws="host", seed) for one update over bf16 gradients with dense factors: the update
    coin, then per weight the bf16 noise and per factor the (32, d) SPD start and the skew start, then the balancing
    coin (the order psgd_pro.py draws them in)."""
    gen = torch.Generator().manual_seed(seed)
    torch.rand([], generator=gen)
    out = []
    for (m, n) in shapes:
        noise = torch.randn(m * n, generator=gen, dtype=torch.bfloat16).view(m, n)
        V = []
        for d in (m, n):
            V.append(torch.randn(32 * d, generator=gen).view(32, d))
            torch.randn(32 * d, generator=gen)
        out.append((noise, V, float(torch.rand([], generator=gen)) < O.BALANCE_PROB))
    return out


def _check_first_step(opt, shapes, grads, seed, label):
    """Q (per element), its change from the identity Q - I (per element: the update term (lr / ell)(term1 - term2 I)
    itself, which Q's unit diagonal would otherwise dominate) and L against the closed form."""
    draws = _host_draws(seed, shapes)
    worst_q = worst_dq = worst_l = 0.0
    for i, (g, (noise, V, bal)) in enumerate(zip(grads, draws)):
        Qs, Ls = opt.factors(i)
        cf = _closed_form_first_step(g, noise, V)
        Qc = [q for q, _ in cf]
        if bal:  # the weight's balancing coin came up (psgd_pro.py:138-139): both factors rescaled
            O.balance(Qc)
        for f, ((_, ell), q) in enumerate(zip(cf, Qc)):
            qg = Qs[f].cpu()
            worst_q = max(worst_q, rel_err_floor(qg, q))
            if not bal:
                qg.diagonal().sub_(1.0)
                q = q.clone()
                q.diagonal().sub_(1.0)
                worst_dq = max(worst_dq, rel_err_floor(qg, q))
            worst_l = max(worst_l, abs(float(Ls[f]) - ell) / ell)
    print(f"{label}: first step vs closed form, per element Q {worst_q:.2e}, Q - I {worst_dq:.2e}, L {worst_l:.2e}",
          flush=True)
    assert worst_q < TOL16 and worst_dq < TOL16 and worst_l < TOL16, (worst_q, worst_dq, worst_l)


def _snapshot(opt, W, n):
    Qs, Ls = _gpu_state(opt, n)
    return [w.detach().clone() for w in W] + [q.clone() for qs in Qs for q in qs] + [l.clone() for ls in Ls for l in ls]


def test_vitb_full_set_first_step_and_paths(hip):
    """The 48-weight ViT-B set: step 1 against the closed form in every launch arrangement; over two steps the
    benchmarked options (fused groups on the library's side streams, 4 Python side streams) are bitwise equal to the
    same launches on one stream (library side streams off too), and within the bf16 bar of one update call per
    group (whose launches batch fewer problems, so the size rule may pick other tile configurations and k splits,
    which sum in another order)."""
    shapes = VIT_B * 12
    kw = dict(preconditioner_max_size=8192, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0)
    runs = []
    for streams, fuse, lib_streams in ((4, True, 3), (0, True, 0), (4, False, 3)):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, precision="bf16", draws="host", seed=3, streams=streams, fuse_groups=fuse, **kw)
        assert hip.psgdk_set_option(6, lib_streams) == 0
        try:
            g0 = _grads(shapes, 0)
            opt.step_math([g.to(DEV) for g in g0])
            torch.cuda.synchronize()
            _check_first_step(opt, shapes, g0, 3, f"ViT-B set (48 weights, streams {streams}, fuse {fuse})")
            opt.step_math([g.to(DEV) for g in _grads(shapes, 1)])
            torch.cuda.synchronize()
        finally:
            hip.psgdk_set_option(6, 3)
        runs.append(_snapshot(opt, W, len(shapes)))
        del opt, W
    for a, b in zip(runs[0], runs[1]):
        assert torch.equal(a, b)
    worst = max(rel_err_floor(a, b) for a, b in zip(runs[0], runs[2]))
    print(f"fused vs per-group update calls after 2 steps: worst per-element difference {worst:.2e}", flush=True)
    assert worst < TOL16


def test_vitb_device_draws(hip):
    """The benchmark's own configuration (device draws: normals from the library's counter-based generator keyed by
    the optimizer's CPU generator): after 3 steps every factor, L and parameter is finite, L > 0, and the same seed
    reproduces every value bit for bit."""
    shapes = VIT_B * 12
    kw = dict(preconditioner_max_size=8192, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0)
    runs = []
    for _ in range(2):
        torch.cuda.manual_seed(1234)
        W = [(0.02 * torch.randn(s, generator=torch.Generator().manual_seed(7))).to(DEV).requires_grad_(True)
             for s in shapes]
        opt = KronWhiten(W, precision="bf16", draws="device", seed=0, streams=3, fuse_groups=True, **kw)
        for t in range(3):
            opt.step_math([g.to(DEV) for g in _grads(shapes, t)])
        torch.cuda.synchronize()
        snap = _snapshot(opt, W, len(shapes))
        assert all(bool(torch.isfinite(x).all()) for x in snap)
        Qs, Ls = _gpu_state(opt, len(shapes))
        assert all(float(l) > 0 for ls in Ls for l in ls)
        runs.append(snap)
        del opt, W
    for a, b in zip(*runs):
        assert torch.equal(a, b)


def test_llama_shapes_first_step(hip):
    """4096x4096 and 4096x14336 bf16 gradients, every factor dense (14336^2 factors), the benchmark's options: the
    first step against its closed form, and every value finite after a second step."""
    shapes = [(4096, 4096), (4096, 14336)]
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    opt = KronWhiten(W, precision="bf16", draws="host", seed=5, streams=4, preconditioner_max_size=16384,
                     preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0)
    g0 = _grads(shapes, 0)
    opt.step_math([g.to(DEV) for g in g0])
    torch.cuda.synchronize()
    _check_first_step(opt, shapes, g0, 5, "Llama shapes")
    opt.step_math([g.to(DEV) for g in _grads(shapes, 1)])
    torch.cuda.synchronize()
    assert all(bool(torch.isfinite(x).all()) for x in _snapshot(opt, W, len(shapes)))


def _vit_param_shapes():
    import bench
    return [tuple(p.shape) for p in bench._vit().parameters()]


def test_e2e_vit_parameter_set_parity(hip):
    """The end-to-end ViT's 78 parameters (dim 512, depth 6, MLP 1024, patch 4, 10 classes), the benchmark's
    optimizer settings (max_skew 2, momentum 0.9, lr 1e-3, bf16 MFMA, init scale from the first gradients) with
    float32 gradients, 3 steps against the float32 oracle and the rounded-operand oracle, host draws."""
    shapes = _vit_param_shapes()
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    kw = dict(preconditioner_max_skew=2, lr_params=1e-3, momentum=0.9)
    opt = KronWhiten(W, precision="bf16", draws="host", seed=2, **kw)
    opt.capture = True
    mk = lambda rounding: O.OracleKron([torch.zeros(s) for s in shapes], seed=2, dtype=torch.float32,
                                       rounding=rounding, **kw)
    o32, o16 = mk(None), mk(O.round_bf16)
    gpu, floor = dict(Q=0.0, pre=0.0, L=0.0), dict(Q=0.0, pre=0.0, L=0.0)
    for t in range(3):
        gs = _grads(shapes, t, dtype=torch.float32)
        opt.step_math([g.to(DEV) for g in gs])
        o32.step(gs)
        o16.step(gs)
        torch.cuda.synchronize()
        sq = [tuple(s for s in sh if s != 1) for sh in shapes]
        Qs, Ls = _gpu_state(opt, len(shapes))
        pre = [p.reshape(s) for p, s in zip(opt.pre, sq)]
        m = _worst(Qs, Ls, pre, o32)
        f = _worst(o16.Q, o16.L, o16.pre, o32)
        gpu = {k: max(gpu[k], m[k]) for k in gpu}
        floor = {k: max(floor[k], f[k]) for k in floor}
    w = max(rel_err_norm(a.detach().reshape(b.shape), b) for a, b in zip(W, o32.params))
    print(f"e2e ViT parameters, per element vs the float32 oracle: gpu {gpu}, rounded-operand oracle {floor}, "
          f"W normwise {w:.2e}", flush=True)
    for k in ("Q", "pre", "L"):
        assert gpu[k] <= max(TOL16, 2 * floor[k]), (k, gpu, floor)
    assert w < TOL16


def test_e2e_vit_loss_decreases(hip):
    """vit_pro.py's architecture trained 30 steps with KronWhiten (the benchmark's settings, device draws, bf16
    autocast) on one fixed synthetic batch of 128 images with random labels: the loss goes down."""
    import bench
    torch.manual_seed(0)
    model = bench._vit().to(DEV)
    params = [p for p in model.parameters() if p.requires_grad]
    x = torch.randn(128, 3, 32, 32, device=DEV)
    y = torch.randint(0, 10, (128,), device=DEV)
    opt = KronWhiten(params, preconditioner_max_skew=2, lr_params=1e-3, momentum=0.9, precision="bf16", seed=0)

    def closure():
        with torch.autocast("cuda", dtype=torch.bfloat16):
            return torch.nn.functional.cross_entropy(model(x).float(), y)
    losses = [float(opt.step(closure)) for _ in range(30)]
    print("e2e ViT losses", [round(v, 3) for v in losses[::5]], losses[-1], flush=True)
    assert all(math.isfinite(v) for v in losses)
    assert min(losses[-5:]) < 0.9 * losses[0], losses
