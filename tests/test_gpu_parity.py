"""KronWhiten on the HIP engine against the CPU oracle, both fed psgd_pro.py's draw stream from one seed.

Tolerances (per element, |x - y| / max(|y|, 1e-3 max|y|), on Q and on the preconditioned gradient; normwise on the
parameters; relative on L): fp32 path 1e-5 against the float64 oracle, or 2x what the float32 oracle itself scores
against float64 on the same inputs where float32 arithmetic alone exceeds 1e-5; bf16 path 2e-2 against the float32
oracle on the same gradients upcast (damping scaled with bfloat16's eps, as the reference does for a bfloat16
gradient), or 2x what the rounded-operand oracle scores against the float32 oracle where bf16 operands alone exceed
2e-2 (the rounded-operand oracle is the same step with every product's operands rounded to bfloat16 where the bf16
kernels round them).
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
    return [(0.01 * torch.randn(tuple(s), generator=g)).to(dtype) for s in shapes]


def _metrics(Qs, Ls, pre, W, ref):
    """Worst errors of (Q, L, pre, W) against the reference oracle `ref` at one step."""
    out = dict(Q=0.0, L=0.0, pre=0.0, pre_norm=0.0, W=0.0)
    for i in range(len(W)):
        for q, qo in zip(Qs[i], ref.Q[i]):
            out["Q"] = max(out["Q"], rel_err_floor(q, qo))
        for l, lo in zip(Ls[i], ref.L[i]):
            e = abs(float(l) - float(lo)) / max(abs(float(lo)), 1e-30)
            out["L"] = max(out["L"], e if math.isfinite(e) else math.inf)
        out["pre"] = max(out["pre"], rel_err_floor(pre[i], ref.pre[i]))
        out["pre_norm"] = max(out["pre_norm"], rel_err_norm(pre[i], ref.pre[i]))
        out["W"] = max(out["W"], rel_err_norm(W[i], ref.params[i]))
    return out


def run_pair(shapes, steps, seed=0, skew=1.0, max_size=math.inf, prec="fp32", gdt=torch.float32, grad_eps=None,
             momentum=0.0, update_first=True, tri=None, whiten_grad=True, ref_dtype=torch.float64, baseline=True,
             r2=False, rounded=False):
    """Runs the GPU optimizer, the oracle in ref_dtype (the reference) and, with baseline, the oracle in float32 on
    the same gradients and draws (rounded: the float32 rounded-operand oracle instead). Returns the worst metrics of
    GPU vs reference and of the baseline oracle vs reference over all steps."""
    Wg = [torch.zeros(s, device=DEV, dtype=torch.float32, requires_grad=True) for s in shapes]
    kw = dict(preconditioner_max_skew=skew, preconditioner_max_size=max_size, preconditioner_init_scale=1.0,
              momentum=momentum, update_preconditioner_first=update_first, whiten_grad=whiten_grad)
    opt = KronWhiten(Wg, precision=prec, draws="host", seed=seed, tri=tri, r2=r2, **kw)
    opt.capture = True
    # the noise is drawn like the tensor the update reads (the gradient, or the float32 momentum buffer)
    ndt = gdt if whiten_grad else torch.float32
    ref = O.OracleKron([torch.zeros(s, dtype=ref_dtype) for s in shapes], seed=seed, dtype=ref_dtype,
                       grad_eps=grad_eps, r2=r2, noise_dtype=ndt, **kw)
    o32 = O.OracleKron([torch.zeros(s, dtype=torch.float32) for s in shapes], seed=seed, dtype=torch.float32,
                       grad_eps=grad_eps, r2=r2, noise_dtype=ndt, rounding=O.round_bf16 if rounded else None,
                       **kw) if (baseline or rounded) else None
    worst = {}
    base = {}
    for t in range(steps):
        gs = grads_for(shapes, t, gdt)
        opt.step_math([g.to(DEV) for g in gs])
        ref.step([g.to(ref_dtype) for g in gs])
        if o32 is not None:
            o32.step([g.float() for g in gs])
        torch.cuda.synchronize()
        fac = [opt.factors(i) for i in range(len(shapes))]
        m = _metrics([f[0] for f in fac], [f[1] for f in fac], opt.pre, [w.detach() for w in Wg], ref)
        worst = {k: max(worst.get(k, 0.0), v) for k, v in m.items()}
        if o32 is not None:
            mb = _metrics(o32.Q, o32.L, o32.pre, o32.params, ref)
            base = {k: max(base.get(k, 0.0), v) for k, v in mb.items()}
    fmt = lambda d: {k: f"{v:.2e}" for k, v in d.items()}
    print("parity", shapes, prec, "gpu", fmt(worst), "oracle-fp32", fmt(base), flush=True)
    return worst, base


def assert_bf16(worst, base):
    """Per-element 2e-2 on Q and the preconditioned gradient (floor 1e-3 max), normwise 2e-2 on the parameters,
    relative 2e-2 on L, or 2x the rounded-operand oracle's own error against the float32 oracle where bf16 operands
    alone exceed 2e-2."""
    for k in ("Q", "pre", "W", "L"):
        lim = max(TOL16, 2.0 * base.get(k, 0.0))
        assert worst[k] < lim, (k, worst, base)


def assert_fp32(worst, base):
    """Per-element 1e-5 on Q and the preconditioned gradient (floor 1e-3 max), normwise 1e-5 on the parameters,
    relative 1e-5 on L; where float32 arithmetic itself (the float32 oracle) exceeds that at a size, the GPU must
    stay within 2x of the float32 oracle's own error."""
    for k in ("Q", "pre", "W", "L"):
        lim = max(TOL32, 2.0 * base.get(k, 0.0))
        assert worst[k] < lim, (k, worst, base)


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
    worst, base = run_pair(shapes, steps=6, skew=skew)
    assert_fp32(worst, base)


def test_fp32_parity_1024_weight(hip):
    """The 1024 x 1024 configuration: one fp32 weight, gradients 0.01 randn from seeds 1000 + t, draws from seed 0,
    Q = I, update every step, lr_params 1e-3, lr_preconditioner 0.1, default betaL, damping, clip and skew; Q1, Q2,
    L, the preconditioned gradient and W compared at every one of 100 steps (Q grows about 10% per step for about
    12 steps until the preconditioned gradient reaches unit RMS, then settles)."""
    worst, base = run_pair([(1024, 1024)], steps=100)
    assert_fp32(worst, base)


@pytest.mark.parametrize("rq16", [1, 0], ids=["rq_bf16", "rq_fp32"])
def test_bf16_parity(hip, b16cfg, rq16):
    """bf16 gradients and bf16 MFMA inputs against the float32 oracle on the same gradients upcast, at the bf16 bar
    (assert_bf16: per element on Q and the preconditioned gradient, floored by the rounded-operand oracle). Run in
    every tile
    configuration of the bf16 kernel: 384 = 256 + 128 gives the 256-tile ones interior and ragged tiles, so every
    fused epilogue (factor update, RQ with traces, Q update, SYRK mirror) runs on both of its paths; with R Q kept
    in bf16 (the default) and in fp32 between the two Procrustes products."""
    eps16 = torch.finfo(torch.bfloat16).eps
    assert hip.psgdk_set_option(7, rq16) == 0
    try:
        worst, base = run_pair([(256, 384), (384, 256)], steps=8, skew=math.inf, prec="bf16", gdt=torch.bfloat16,
                               grad_eps=eps16, ref_dtype=torch.float32, baseline=False, rounded=True)
    finally:
        hip.psgdk_set_option(7, 1)
    assert_bf16(worst, base)


@pytest.mark.parametrize("shapes,skew", [([(96, 256), (256, 96)], math.inf), ([(96, 256)], 1.0)])
def test_fp32_precision_bf16_grads(hip, shapes, skew):
    """fp32 arithmetic on bf16 gradients (the apply widens a bf16 gradient to fp32 before its first fp32 product;
    the noise is drawn in bf16 like the gradient) against the float64 oracle on the same gradients upcast, at the
    fp32 bar."""
    eps16 = torch.finfo(torch.bfloat16).eps
    worst, base = run_pair(shapes, steps=4, skew=skew, prec="fp32", gdt=torch.bfloat16, grad_eps=eps16)
    assert_fp32(worst, base)


def test_bf16_parity_dense_diag(hip, b16cfg):
    """Weights with one dense and one diagonal factor on the bf16 path (max_skew 1: 96 x 256 and 64 x 264 have a
    diagonal column factor, 256 x 96 a diagonal row factor): the diagonal P scales X's rows or columns on the way to
    the bf16 operand (transposed for columns), the diagonal factor's term1 comes from the bf16 Pg; against the
    float32 oracle on the same gradients upcast at the bf16 bar, in every tile configuration (264: ragged)."""
    eps16 = torch.finfo(torch.bfloat16).eps
    worst, base = run_pair([(96, 256), (256, 96), (64, 264)], steps=8, skew=1.0, prec="bf16", gdt=torch.bfloat16,
                           grad_eps=eps16, ref_dtype=torch.float32, baseline=False, rounded=True)
    assert_bf16(worst, base)


@pytest.mark.parametrize("via_pg", [1, 0], ids=["pg", "term1"])
@pytest.mark.parametrize("r2", [False, True], ids=["step2", "r2"])
def test_bf16_parity_thin_weights(hip, b16cfg, r2, via_pg):
    """Weights whose other side is under half of a factor's side (128 x 384, 384 x 128, 96 x 264): the bf16 update
    forms term1 Q as Pg^T (Pg Q) or Pg (Pg^T Q) for those factors (the same product associated the other way).
    Against the float32 oracle on the same gradients upcast, at the bf16 bar, in every tile configuration (264 =
    256 + 8: ragged tiles), with both Procrustes forms."""
    eps16 = torch.finfo(torch.bfloat16).eps
    assert hip.psgdk_set_option(5, via_pg) == 0
    try:
        worst, base = run_pair([(128, 384), (384, 128), (96, 264)], steps=8, skew=math.inf, prec="bf16",
                               gdt=torch.bfloat16, grad_eps=eps16, ref_dtype=torch.float32, baseline=False, r2=r2,
                               rounded=True)
    finally:
        hip.psgdk_set_option(5, 1)
    assert_bf16(worst, base)


@pytest.mark.parametrize("shapes", [[(64, 96)], [(200, 136)], [(48, 64), (48, 64), (32,), (64, 48)]])
def test_fp32_parity_r2(hip, shapes):
    """r2=True (procrustes_step_r2, psgd_pro_fast.py:141-153) against the float64 oracle's r2 form at the fp32
    bar: S = Rn^T Rn by the SYRK with its trace epilogue, tr(RQ) from the R-forming kernel, Q - M Q in one GEMM."""
    assert_fp32(*run_pair(shapes, steps=6, skew=math.inf, r2=True))


def test_fp32_r2_tracks_step2(hip):
    """The two Procrustes forms are the same algebra: over 6 steps r2 and step2 on the GPU stay within the fp32
    bar of each other (both against the float64 step2 oracle)."""
    worst, base = run_pair([(96, 160)], steps=6, skew=math.inf, r2=True)  # vs float64 r2
    w2, b2 = run_pair([(96, 160)], steps=6, skew=math.inf, r2=False)     # vs float64 step2
    O.MAX_PROCRUSTES  # the oracle's step bound, 1/8, shared by both forms
    for k in ("Q", "pre", "W"):
        assert worst[k] < max(TOL32, 2 * base[k]) and w2[k] < max(TOL32, 2 * b2[k]), (k, worst, w2)


def test_bf16_parity_r2(hip, b16cfg):
    """r2 on the bf16 path (the SYRK of R with the trace epilogue on both of its tile paths in every tile
    configuration) against the float32 oracle's r2 form, at the bf16 bar."""
    eps16 = torch.finfo(torch.bfloat16).eps
    worst, base = run_pair([(256, 384), (384, 256)], steps=8, skew=math.inf, prec="bf16", gdt=torch.bfloat16,
                           grad_eps=eps16, ref_dtype=torch.float32, baseline=False, r2=True, rounded=True)
    assert_bf16(worst, base)


def test_momentum_and_update_last(hip):
    assert_fp32(*run_pair([(64, 80), (80,)], steps=6, skew=math.inf, momentum=0.9, update_first=False))
    assert_fp32(*run_pair([(64, 80)], steps=5, skew=math.inf, momentum=0.5, whiten_grad=False))


def test_triangle_storage_parity(hip):
    assert_fp32(*run_pair([(64, 96), (130, 70)], steps=5, skew=math.inf, tri=True))


def test_balance_matches_oracle(hip):
    """psgdk_kron2d_balance on the optimizer's factors against oracle balance() (the coin fires 1% of steps, so
    it is driven directly here)."""
    W = torch.zeros(64, 96, device=DEV, requires_grad=True)
    opt = KronWhiten([W], preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=1)
    for t in range(3):
        opt.step_math([g.to(DEV) for g in grads_for([(64, 96)], t)])
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


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_state_dict_round_trip(hip, prec):
    """A state_dict taken mid-run and loaded into a fresh optimizer continues bit-identically. On the bf16 path the
    update keeps only P's bf16 copy current, so state_dict refreshes P first: the saved P is Q^T Q of the
    bf16-rounded Q (fp32 accumulation of bf16 products)."""
    shapes = [(64, 96), (32,)]
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=5,
                     momentum=0.9, precision=prec)
    for t in range(3):
        opt.step_math([g.to(DEV) for g in grads_for(shapes, t)])
    st = opt.state_dict()
    Q0, P0 = st["params"][0]["Q"][0].double().cpu(), st["params"][0]["P"][0].double().cpu()
    Qr = Q0.to(torch.bfloat16).double() if prec == "bf16" else Q0
    assert rel_err_norm(P0, Qr.T @ Qr) < 1e-6
    W0 = [w.detach().clone() for w in W]
    opt.step_math([g.to(DEV) for g in grads_for(shapes, 3)])
    after = [w.detach().clone() for w in W]
    W2 = [w0.clone().requires_grad_(True) for w0 in W0]
    opt2 = KronWhiten(W2, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=99,
                      momentum=0.9, precision=prec)
    opt2.load_state_dict(st)
    opt2.step_math([g.to(DEV) for g in grads_for(shapes, 3)])
    for a, b in zip(after, W2):
        assert torch.equal(a, b.detach())


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_side_streams_bitwise_identical(hip, prec):
    """Weight groups on side streams (streams=4) give bit-identical factors and parameters to one stream
    (streams=0): the groups share no state and every kernel reduces in a fixed order."""
    shapes = [(64, 96), (96, 64), (128, 128), (32,), (64, 96)]
    runs = []
    for ns in (0, 4):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=7,
                         momentum=0.9, precision=prec, streams=ns)
        for t in range(4):
            opt.step_math([g.to(DEV) for g in grads_for(shapes, t)])
        torch.cuda.synchronize()
        qs = [q.detach().clone() for i in range(len(shapes)) for q in opt.factors(i)[0]]
        runs.append(([w.detach().clone() for w in W], qs))
    for a, b in zip(runs[0][0] + runs[0][1], runs[1][0] + runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_per_group_apply_scheduling_bitwise(hip, prec):
    """With the update first, each group's balance and apply wait only for that group's own update (a completion
    event per group from psgdk_kron2d_update_groups_ev, or from its own update call). Against the whole update, then
    every balance, then every apply: bitwise the same factors and parameters over 5 steps with momentum, balancing
    coins forced for some parameters on steps 1 and 3, and update-skipping steps (probability 0.6)."""
    shapes = [(64, 96), (96, 64), (128, 128), (32,), (64, 96), (256, 64)]
    runs = []
    for overlap in (False, True):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=9,
                         momentum=0.9, precision=prec, streams=3, preconditioner_update_probability=0.6)
        opt._overlap = overlap
        real = opt._draw_update

        def forced(srcs, real=real, opt=opt):
            noise, V, coins = real(srcs)
            if opt._t in (1, 3):
                coins = [c or i in (0, 2, 5) for i, c in enumerate(coins)]
            return noise, V, coins
        opt._draw_update = forced
        for t in range(5):
            opt._t = t
            opt.step_math([g.to(DEV) for g in grads_for(shapes, t)])
        torch.cuda.synchronize()
        qs = [q.detach().clone() for i in range(len(shapes)) for q in opt.factors(i)[0]]
        runs.append(([w.detach().clone() for w in W], qs))
    for a, b in zip(runs[0][0] + runs[0][1], runs[1][0] + runs[1][1]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("skew", [math.inf, 2.0], ids=["dense", "mixed"])
@pytest.mark.parametrize("r2", [False, True], ids=["step2", "r2"])
def test_fused_groups_bitwise_identical(hip, r2, skew):
    """fuse_groups=True (one psgdk_kron2d_update_groups call; factor work batched by side across groups and both
    dimensions) against one psgdk_kron2d_update per group: Q, L, the P shadows and the parameters bitwise equal
    after 4 steps, on a mixed set (bf16 groups sharing factor sides 128 and 384 across shapes, plus a vector and an
    fp32-gradient weight that stay on the per-group path). At these sizes every launch takes the 128-tile
    configuration and the same k splits either way, so the sums run in the same order (at the ViT-B sizes the
    arrangements differ: test_vitb_full_set_first_step_and_paths). The tiny-product kernel is switched off (option
    11 = 0): its size rule, like the tile configuration's, looks at the whole launch, so it would take some of the
    smaller per-group launches and none of the batched ones, and it sums k in another order."""
    shapes = [(128, 384), (128, 384), (128, 128), (384, 128), (384, 128), (128, 512), (96,), (64, 40), (32, 512),
              (512, 48)]  # the last two: a dense and a diagonal factor (512^2 > 2 x 32 x 512)
    gen = torch.Generator().manual_seed(5)
    grads = [[(0.01 * torch.randn(s, generator=gen)).to(torch.bfloat16 if len(s) == 2 and s != (64, 40)
                                                      else torch.float32).to(DEV) for s in shapes] for _ in range(4)]
    res = []
    assert hip.psgdk_set_option(11, 0) == 0
    try:
        for fuse in (True, False):
            W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
            opt = KronWhiten(W, precision="bf16", draws="host", seed=3, preconditioner_max_skew=skew,
                             preconditioner_init_scale=1.0, fuse_groups=fuse, r2=r2)
            for gs in grads:
                opt.step_math(gs)
            torch.cuda.synchronize()
            st = opt.state_dict()
            res.append(([w.detach().clone() for w in W], st))
    finally:
        hip.psgdk_set_option(11, 64)
    (Wa, sa), (Wb, sb) = res
    for a, b in zip(Wa, Wb):
        assert torch.equal(a, b)
    for pa, pb in zip(sa["params"], sb["params"]):
        for key in ("Q", "L", "P"):
            for x, y in zip(pa[key], pb[key]):
                assert torch.equal(x, y), key


@pytest.mark.parametrize("skew", [math.inf, 2.0], ids=["dense", "mixed"])
def test_noise_drawn_in_update_bitwise(hip, skew):
    """draws="device": the bf16 noise generated inside the grouped update (psgdk_kron2d_update_groups_drawn, no
    noise buffer) against the same normals filled into a buffer by psgdk_fill_normal and read back: bitwise equal
    Q, L, P and parameters after 3 steps with momentum. The set mixes bf16 and fp32 gradients (the fp32 noise stays
    in its buffer), dense-diagonal groups at skew 2 (the transposed noise kernel) and a gradient 8 bytes past a
    16-byte boundary (the noise kernel's per-element path)."""
    shapes = [(128, 384), (128, 384), (256, 128), (64, 40), (32, 512), (512, 48), (96,)]
    gen = torch.Generator().manual_seed(11)
    steps = []
    for _ in range(3):
        gs = []
        for i, s in enumerate(shapes):
            dt = torch.bfloat16 if len(s) == 2 and s != (64, 40) else torch.float32
            g = (0.01 * torch.randn(s, generator=gen)).to(dt).to(DEV)
            if i == 2:
                buf = torch.zeros(g.numel() + 8, dtype=dt, device=DEV)
                v = buf[4:4 + g.numel()].view(s)
                v.copy_(g)
                assert v.data_ptr() % 16 == 8
                g = v
            gs.append(g)
        steps.append(gs)
    res = []
    for inside in (True, False):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, precision="bf16", draws="device", seed=5, preconditioner_max_skew=skew,
                         preconditioner_init_scale=1.0, momentum=0.9)
        opt._draw_in_update = inside
        for gs in steps:
            opt.step_math(gs)
        torch.cuda.synchronize()
        assert (opt._draw_buf16 is None) == inside
        res.append(([w.detach().clone() for w in W], opt.state_dict()))
    (Wa, sa), (Wb, sb) = res
    for a, b in zip(Wa, Wb):
        assert torch.equal(a, b)
    for pa, pb in zip(sa["params"], sb["params"]):
        for key in ("Q", "L", "P"):
            for x, y in zip(pa[key], pb[key]):
                assert torch.equal(x, y), key


GRAPHS_OFF = ("graphs=True is switched off: a capture of the step (side streams forked inside torch.cuda.graph) "
              "aborted the process (SIGABRT) on the GPU, after an earlier segfault at capture end, and the cause is "
              "not established; KronWhiten(graphs=True) raises NotImplementedError")


@pytest.mark.skip(reason=GRAPHS_OFF)
@pytest.mark.parametrize("draws", ["host", "device"])
@pytest.mark.parametrize("first", [True, False])
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_graph_replay_matches_eager(hip, prec, first, draws):
    """graphs=True replays captured HIP graphs of the step's device segments; every step must equal the eager
    optimizer bit for bit. 16 steps: momentum's beta settles after 9 (new graph keys until then), the update coin
    (p = 0.5) makes both the update and the apply-only segments replay, and balancing coins forced on steps 11 and
    13 (on both optimizers) run between segments. Between replays the test synchronizes and compares on the
    device (eager work of its own). Host draws and the library's device draws."""
    shapes = [(64, 96), (96, 64), (128, 128), (32,), (64, 96)]
    opts, Ws = [], []
    for graphs in (False, True):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws=draws, seed=11,
                         momentum=0.9, precision=prec, preconditioner_update_probability=0.5,
                         update_preconditioner_first=first, graphs=graphs)
        real = opt._draw_update

        def forced(srcs, real=real, opt=opt):
            noise, V, coins = real(srcs)
            if opt._step_no in (11, 13):
                coins = [True] + coins[1:]
            return noise, V, coins
        opt._draw_update = forced
        opts.append(opt)
        Ws.append(W)
    for t in range(16):
        gs = grads_for(shapes, t)
        for opt in opts:
            opt._step_no = t
            opt.step_math([g.to(DEV) for g in gs])
        torch.cuda.synchronize()
        for a, b in zip(Ws[0], Ws[1]):
            assert torch.equal(a, b), f"step {t}"
        for i in range(len(shapes)):
            for qa, qb in zip(opts[0].factors(i)[0], opts[1].factors(i)[0]):
                assert torch.equal(qa, qb), f"step {t}, parameter {i}"
    assert len(opts[1]._graphs) >= 2


def test_step_closure_and_loss_curve(hip):
    """A least-squares model trained 100 steps through step(closure): the GPU optimizer (float32 model and
    gradients) and the float64 oracle (float64 model and gradients, same draws) give matching loss curves. The
    trajectories see different gradient rounding, so the bar is the divergence the float32 oracle itself shows
    against the float64 oracle on the same problem (its own float32 gradients), with a 1e-4 relative floor."""
    g = torch.Generator().manual_seed(0)
    X = torch.randn(256, 48, generator=g)
    Wt = torch.randn(48, 24, generator=g)
    Y = X @ Wt + 0.01 * torch.randn(256, 24, generator=g)
    kw = dict(preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, lr_params=0.01)
    Wg = torch.zeros(48, 24, device=DEV, requires_grad=True)
    opt = KronWhiten([Wg], draws="host", seed=3, **kw)
    Xd, Yd = X.to(DEV), Y.to(DEV)

    def oracle_curve(dt):
        W = torch.zeros(48, 24, dtype=dt, requires_grad=True)
        ora = O.OracleKron([W], seed=3, dtype=dt, **kw)
        out = []
        for _ in range(100):
            with torch.enable_grad():
                loss = ((X.to(dt) @ W - Y.to(dt)) ** 2).mean()
                (gr,) = torch.autograd.grad(loss, [W])
            out.append(float(loss))
            with torch.no_grad():
                ora.step([gr])
        return out

    lg = [float(opt.step(lambda: ((Xd @ Wg - Yd) ** 2).mean())) for _ in range(100)]
    l64 = oracle_curve(torch.float64)
    l32 = oracle_curve(torch.float32)
    assert lg[-1] < 0.5 * lg[0]
    d_gpu = max(abs(a - b) / abs(b) for a, b in zip(lg, l64))
    d_32 = max(abs(a - b) / abs(b) for a, b in zip(l32, l64))
    print(f"loss curve: gpu vs fp64 {d_gpu:.2e}, oracle-fp32 vs fp64 {d_32:.2e}", flush=True)
    assert d_gpu <= max(1e-4, 3 * d_32), (d_gpu, d_32)


def test_bf16_loss_curve(hip):
    """A least-squares model (X 512 x 128, W 128 x 64, both factors dense on the bf16 kernels) trained 100 steps
    through step(closure) with precision="bf16": its loss curve against the float32 oracle's (same draws, its own
    float32 gradients). The bar is 2e-2 relative per step, or 3x the divergence the rounded-operand oracle (every
    product's operands rounded to bfloat16 where the bf16 kernels round them) shows against the float32 oracle
    (7.2e-3 on this problem). lr 3e-3 keeps the run in the regime where the curve follows the draws smoothly: at
    lr 1e-2 the float32 and float64 oracles themselves part by 25% once discrete choices inside the norm bounds
    flip."""
    g = torch.Generator().manual_seed(0)
    X = torch.randn(512, 128, generator=g)
    Wt = torch.randn(128, 64, generator=g)
    Y = X @ Wt + 0.01 * torch.randn(512, 64, generator=g)
    kw = dict(preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, lr_params=3e-3)
    Wg = torch.zeros(128, 64, device=DEV, requires_grad=True)
    opt = KronWhiten([Wg], precision="bf16", draws="host", seed=3, **kw)
    Xd, Yd = X.to(DEV), Y.to(DEV)

    def oracle_curve(rounding):
        W = torch.zeros(128, 64, requires_grad=True)
        ora = O.OracleKron([W], seed=3, dtype=torch.float32, rounding=rounding, **kw)
        out = []
        for _ in range(100):
            with torch.enable_grad():
                loss = ((X @ W - Y) ** 2).mean()
                (gr,) = torch.autograd.grad(loss, [W])
            out.append(loss.item())
            with torch.no_grad():
                ora.step([gr])
        return out

    lg = [float(opt.step(lambda: ((Xd @ Wg - Yd) ** 2).mean())) for _ in range(100)]
    l32 = oracle_curve(None)
    l16 = oracle_curve(O.round_bf16)
    assert all(math.isfinite(v) for v in lg)
    assert lg[-1] < 0.75 * lg[0], (lg[0], lg[-1])
    d_gpu = max(abs(a - b) / abs(b) for a, b in zip(lg, l32))
    d_16 = max(abs(a - b) / abs(b) for a, b in zip(l16, l32))
    print(f"bf16 loss curve: gpu vs fp32 oracle {d_gpu:.2e}, rounded-operand oracle vs fp32 {d_16:.2e}, "
          f"loss {lg[0]:.3e} -> {lg[-1]:.3e}", flush=True)
    assert d_gpu <= max(TOL16, 3 * d_16), (d_gpu, d_16)


def test_bf16_parity_general_path(hip):
    """bf16 groups outside the bf16 kernel's reach (rows not a multiple of 8, a diagonal factor) use the general
    engine at bf16 input precision."""
    eps16 = torch.finfo(torch.bfloat16).eps
    worst, base = run_pair([(100, 70), (96, 64)], steps=6, skew=1.0, prec="bf16", gdt=torch.bfloat16,
                           grad_eps=eps16, ref_dtype=torch.float32, baseline=False, rounded=True)
    assert_bf16(worst, base)


@pytest.mark.parametrize("bad", [float("nan"), float("inf")], ids=["nan", "inf"])
@pytest.mark.parametrize("shape,skew,prec", [((96, 64), 0.5, "fp32"), ((77,), 1.0, "fp32"), ((96, 64), 0.5, "bf16")])
def test_clip_passes_non_finite_values_through(hip, bad, shape, skew, prec):
    """A gradient with one NaN or inf element, no preconditioner update (probability 0; diagonal factors, so the
    preconditioned gradient is elementwise and the bad value stays in one place): the parameters match the oracle's
    pattern of psgd_pro.py:371-381: NaN at that element only with the others taking their normal clipped step
    (NaN: no RMS rescale), or NaN there and every other element unchanged (inf: RMS inf, rescale by 0)."""
    g = 0.5 * torch.randn(shape, generator=torch.Generator().manual_seed(3))
    g.view(-1)[5] = bad
    kw = dict(preconditioner_max_skew=skew, preconditioner_init_scale=1.0, preconditioner_update_probability=0.0,
              lr_params=0.1, grad_clip_max_amps=(2.0, 1.0))
    W = torch.ones(shape, device=DEV, requires_grad=True)
    opt = KronWhiten([W], draws="host", seed=0, precision=prec, **kw)
    opt.step_math([g.to(DEV)])
    Wo = torch.ones(shape, dtype=torch.float64)
    ora = O.OracleKron([Wo], seed=0, dtype=torch.float64, **kw)
    ora.step([g.double()])
    torch.cuda.synchronize()
    Wg = W.detach().double().cpu()
    assert torch.equal(torch.isnan(Wg), torch.isnan(Wo)) and int(torch.isnan(Wo).sum()) == 1
    fin = ~torch.isnan(Wo)
    assert rel_err_norm(Wg[fin], Wo[fin]) < 1e-6
    if bad == float("inf"):
        assert torch.equal(Wg[fin], torch.ones_like(Wg[fin]))


@pytest.mark.skip(reason=GRAPHS_OFF)
@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_graph_replay_tracks_oracle(hip, prec):
    """graphs=True (captured HIP graph segments) against the oracle fed the same draws, 14 steps with momentum 0.9:
    the apply-only segment is captured on its second step, the update segment once beta settles (step 10), then
    both replay; at the fp32 or bf16 bar."""
    shapes = [(64, 96), (96, 64), (128,)]
    kw = dict(preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, momentum=0.9)
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    gdt = torch.bfloat16 if prec == "bf16" else torch.float32
    opt = KronWhiten(W, precision=prec, draws="host", seed=4, graphs=True, **kw)
    opt.capture = True
    ref_dt = torch.float32 if prec == "bf16" else torch.float64
    eps = torch.finfo(gdt).eps if prec == "bf16" else None
    mk = lambda dt, rounding: O.OracleKron([torch.zeros(s, dtype=dt) for s in shapes], seed=4, dtype=dt,
                                           grad_eps=eps, noise_dtype=gdt, rounding=rounding, **kw)
    ref = mk(ref_dt, None)
    bl = mk(torch.float32, O.round_bf16 if prec == "bf16" else None)  # the float32 or rounded-operand baseline
    worst, base = {}, {}
    for t in range(14):
        gs = grads_for(shapes, t, gdt)
        opt.step_math([g.to(DEV) for g in gs])
        ref.step([g.to(ref_dt) for g in gs])
        bl.step([g.float() for g in gs])
        torch.cuda.synchronize()
        fac = [opt.factors(i) for i in range(len(shapes))]
        m = _metrics([f[0] for f in fac], [f[1] for f in fac], opt.pre, [w.detach() for w in W], ref)
        worst = {k: max(worst.get(k, 0.0), v) for k, v in m.items()}
        mb = _metrics(bl.Q, bl.L, bl.pre, bl.params, ref)
        base = {k: max(base.get(k, 0.0), v) for k, v in mb.items()}
    assert len(opt._graphs) >= 2
    print("graph replay vs oracle", prec, {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)
    (assert_fp32 if prec == "fp32" else assert_bf16)(worst, base)


@pytest.mark.parametrize("prec", ["fp32", "bf16"])
def test_state_dict_continuation_tracks_oracle(hip, prec):
    """A run checkpointed after 3 steps and reloaded into a fresh optimizer (another seed, so the draws come from the
    saved generator state) tracks the oracle's uninterrupted run for 5 more steps, momentum included."""
    shapes = [(64, 96), (32,)]
    kw = dict(preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, momentum=0.9)
    gdt = torch.bfloat16 if prec == "bf16" else torch.float32
    ref_dt = torch.float32 if prec == "bf16" else torch.float64
    eps = torch.finfo(gdt).eps if prec == "bf16" else None
    mk = lambda dt, rounding: O.OracleKron([torch.zeros(s, dtype=dt) for s in shapes], seed=6, dtype=dt,
                                           grad_eps=eps, noise_dtype=gdt, rounding=rounding, **kw)
    ref = mk(ref_dt, None)
    bl = mk(torch.float32, O.round_bf16 if prec == "bf16" else None)  # the float32 or rounded-operand baseline
    W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
    opt = KronWhiten(W, precision=prec, draws="host", seed=6, **kw)
    for t in range(3):
        gs = grads_for(shapes, t, gdt)
        opt.step_math([g.to(DEV) for g in gs])
        ref.step([g.to(ref_dt) for g in gs])
        bl.step([g.float() for g in gs])
    st = opt.state_dict()
    W2 = [w.detach().clone().requires_grad_(True) for w in W]
    del opt
    opt2 = KronWhiten(W2, precision=prec, draws="host", seed=1234, **kw)
    opt2.load_state_dict(st)
    opt2.capture = True
    worst, base = {}, {}
    for t in range(3, 8):
        gs = grads_for(shapes, t, gdt)
        opt2.step_math([g.to(DEV) for g in gs])
        ref.step([g.to(ref_dt) for g in gs])
        bl.step([g.float() for g in gs])
        torch.cuda.synchronize()
        fac = [opt2.factors(i) for i in range(len(shapes))]
        m = _metrics([f[0] for f in fac], [f[1] for f in fac], opt2.pre, [w.detach() for w in W2], ref)
        worst = {k: max(worst.get(k, 0.0), v) for k, v in m.items()}
        mb = _metrics(bl.Q, bl.L, bl.pre, bl.params, ref)
        base = {k: max(base.get(k, 0.0), v) for k, v in mb.items()}
    print("state_dict continuation vs oracle", prec, {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)
    (assert_fp32 if prec == "fp32" else assert_bf16)(worst, base)
