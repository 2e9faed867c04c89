"""Each HIP kernel of libpsgdk.so against a float64 reference of the same operation (computed on the CPU).

fp32 path: elementwise |C - ref| <= 64 eps_f32 * (|A| |B|) (a few ulps of the accumulation's natural error bound).
bf16 path: the reference multiplies the bf16-rounded inputs in float64, so the only error is fp32 accumulation:
the same bound applies. Triangle-reading kernels get a NaN-filled strict lower triangle: any read of it would show.
"""
import math

import pytest
import torch

from psgd_pro_amd import _lib as L
from psgd_pro_amd import KronWhiten
from psgd_pro_amd import ops as K
from tests.metrics import rel_err_norm

pytestmark = pytest.mark.gpu
DEV = "cuda"
EPS32 = torch.finfo(torch.float32).eps


def rnd(*shape, seed=0, dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def bf(x):
    return x.to(torch.bfloat16).float()


def check_gemm_bound(C, A64, B64, tol=64):
    """|C - A B| <= tol * eps32 * |A| |B| elementwise (A64, B64: float64 CPU operands as multiplied)."""
    ref = A64 @ B64
    bound = tol * EPS32 * (A64.abs() @ B64.abs()) + 1e-30
    err = (C.double().cpu() - ref).abs()
    worst = float((err / bound).max())
    assert worst <= 1.0, f"max err/bound = {worst}"


def poison_lower(S):
    return S.masked_fill(torch.ones_like(S, dtype=torch.bool).tril(-1), float("nan"))


# --------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("prec", [0, 1, 2])
def test_mfma_lane_layout(hip, prec):
    t = 32 if prec == 2 else 16
    k = {0: 4, 1: 32, 2: 16}[prec]
    A = rnd(t, k, seed=1)
    B = rnd(k, t, seed=2)
    if prec:
        A, B = bf(A), bf(B)
    Ad, Bd = A.to(DEV), B.to(DEV)
    Cd = torch.empty(t, t, device=DEV)
    L.check(hip.psgdk_debug_mfma(prec, C_ptr(Ad), C_ptr(Bd), C_ptr(Cd), L.stream_of(Ad)))
    torch.cuda.synchronize()
    check_gemm_bound(Cd, A.double(), B.double(), tol=8)


def C_ptr(t):
    import ctypes
    return ctypes.c_void_p(t.data_ptr())


GEMM_SHAPES = [(128, 128, 128), (256, 384, 320), (100, 70, 33), (1, 50, 77), (33, 129, 200), (768, 256, 768),
               (32, 96, 1000)]


@pytest.mark.parametrize("m,n,k", GEMM_SHAPES)
@pytest.mark.parametrize("ta,tb", [(0, 0), (1, 0), (0, 1), (1, 1)])
@pytest.mark.parametrize("prec", [0, 1])
def test_gemm(hip, m, n, k, ta, tb, prec):
    A = rnd(*((k, m) if ta else (m, k)), seed=m + k)
    B = rnd(*((n, k) if tb else (k, n)), seed=n + 3 * k)
    C = K.gemm(A.to(DEV), B.to(DEV), bool(ta), bool(tb), bool(prec))
    A64 = (bf(A) if prec else A).double()
    B64 = (bf(B) if prec else B).double()
    check_gemm_bound(C, A64.T if ta else A64, B64.T if tb else B64)


@pytest.mark.parametrize("adt,bdt", [(torch.bfloat16, torch.float32), (torch.float32, torch.bfloat16),
                                     (torch.bfloat16, torch.bfloat16)])
@pytest.mark.parametrize("prec", [0, 1])
def test_gemm_storage_dtypes(hip, adt, bdt, prec):
    m, n, k = 200, 136, 264
    A = rnd(m, k, seed=5).to(adt)
    B = rnd(k, n, seed=6).to(bdt)
    C = K.gemm(A.to(DEV), B.to(DEV), False, False, bool(prec))
    A64 = (bf(A.float()) if prec else A.float()).double()
    B64 = (bf(B.float()) if prec else B.float()).double()
    check_gemm_bound(C, A64, B64)


def test_gemm_grouped_and_alpha_beta(hip):
    m, n, k, nb = 96, 160, 128, 5
    As = [rnd(m, k, seed=i).to(DEV) for i in range(nb)]
    Bs = [rnd(k, n, seed=10 + i).to(DEV) for i in range(nb)]
    Cs = [rnd(m, n, seed=20 + i).to(DEV) for i in range(nb)]
    C0 = [c.clone() for c in Cs]
    L.check(hip.psgdk_gemm(0, 0, 0, m, n, k, 0.5, 0, 0, nb, L.ptrs(As), k, L.ptrs(Bs), n, -2.0, L.ptrs(Cs), n,
                           L.stream_of(As[0])))
    for A, B, C, c0 in zip(As, Bs, Cs, C0):
        ref = 0.5 * (A.double().cpu() @ B.double().cpu()) - 2.0 * c0.double().cpu()
        assert rel_err_norm(C, ref) < 1e-6


# --------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n,k", [(128, 128), (256, 64), (200, 333), (768, 2304), (65, 17), (1, 9)])
@pytest.mark.parametrize("trans", [False, True])
@pytest.mark.parametrize("prec", [0, 1])
def test_syrk(hip, n, k, trans, prec):
    """Every output mode against float64 within the GEMM bound; the mirrored result exactly symmetric; the upper and
    mirrored modes (one kernel) bitwise equal on the upper triangle. With the tiny-product kernel off (option 11 = 0)
    every kernel sums k in order, and the packed mode (the general engine) is bitwise the mirrored one."""
    A = rnd(*((k, n) if trans else (n, k)), seed=n * 7 + k)
    Ad = A.to(DEV)
    X64 = (bf(A) if prec else A).double()
    X64 = X64.T if trans else X64
    triu = torch.ones(n, n, dtype=torch.bool, device=DEV).triu()
    try:
        for tiny in (64, 0):
            assert hip.psgdk_set_option(11, tiny) == 0
            full = K.syrk(Ad, trans, L.OUT_MIRROR, bool(prec))
            check_gemm_bound(full, X64, X64.T)
            assert torch.equal(full, full.T)  # mirrored: exactly symmetric
            up = torch.full((n, n), float("nan"), device=DEV)
            L.check(hip.psgdk_syrk(prec, int(trans), L.OUT_UPPER, n, k, 0, 1, L.ptrs([Ad]), Ad.stride(0), L.ptrs([up]),
                                   n, L.stream_of(Ad)))
            assert torch.equal(up[triu], full[triu])
            assert bool(torch.isnan(up[~triu]).all())  # the strict lower triangle is not written
    finally:
        hip.psgdk_set_option(11, 64)
    pk = K.syrk(Ad, trans, L.OUT_PACKED, bool(prec))
    check_gemm_bound(K.unpack(pk, n), X64, X64.T)
    assert torch.equal(pk, K.pack_upper(full))
    assert torch.equal(K.unpack(pk, n), full)


# --------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n,p", [(128, 64), (200, 130), (768, 768), (64, 1), (37, 300)])
@pytest.mark.parametrize("sign", [1, -1])
@pytest.mark.parametrize("prec", [0, 1])
def test_symm_reads_only_the_upper_triangle(hip, n, p, sign, prec):
    X = rnd(n, n, seed=n)
    S = (X + X.T) if sign > 0 else (X - X.T)
    B = rnd(n, p, seed=p)
    Sd = poison_lower(S).to(DEV)
    C = K.symm(Sd, B.to(DEV), sign, bool(prec))
    S64 = (bf(S) if prec else S).double()
    B64 = (bf(B) if prec else B).double()
    check_gemm_bound(C, S64, B64)
    Bt = rnd(p, n, seed=p + 1)
    Cr = K.symm_right(Bt.to(DEV), Sd, sign, bool(prec))
    check_gemm_bound(Cr, (bf(Bt) if prec else Bt).double(), S64)


@pytest.mark.parametrize("n,p", [(256, 256), (200, 77), (512, 512)])
@pytest.mark.parametrize("prec", [0, 1])
def test_trmm(hip, n, p, prec):
    """triu(Q) B through psgdk_trmm_ws (the k-contiguous kernel with the triangle's k range where the shape allows,
    psgdk_trmm otherwise: 200 x 77) and psgdk_trmm itself, Q's strict lower triangle NaN-poisoned."""
    Q = rnd(n, n, seed=3)
    B = rnd(n, p, seed=4)
    Qd, Bd = poison_lower(Q).to(DEV), B.to(DEV)
    C = K.trmm(Qd, Bd, bool(prec))
    Q64 = torch.triu((bf(Q) if prec else Q).double())
    B64 = (bf(B) if prec else B).double()
    check_gemm_bound(C, Q64, B64)
    C2 = torch.empty(n, p, device=DEV)
    L.check(hip.psgdk_trmm(prec, n, p, 0, 1, L.ptrs([Qd]), n, L.ptrs([Bd]), p, L.ptrs([C2]), p, L.stream_of(Bd)))
    check_gemm_bound(C2, Q64, B64)


@pytest.mark.parametrize("prec", [0, 1])
def test_trmm_ws_grouped_and_bf16_b(hip, prec):
    """psgdk_trmm_ws on a group of 3 problems with leading dimensions wider than the matrices, B in bf16 storage."""
    n, p, nb = 264, 136, 3
    Qs = [poison_lower(rnd(n, n + 8, seed=i)[:, :n]).contiguous() for i in range(nb)]
    Qf = [torch.cat([q, torch.zeros(n, 8)], 1).to(DEV) for q in Qs]  # ldq = n + 8
    Bs = [rnd(n, p + 8, seed=10 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]  # ldb = p + 8
    Cs = [torch.empty(n, p + 16, device=DEV) for _ in range(nb)]  # ldc = p + 16
    L.call_ws(hip.psgdk_trmm_ws, prec, n, p, 1, nb, L.ptrs(Qf), n + 8, L.ptrs(Bs), p + 8, L.ptrs(Cs), p + 16,
              ws=L.Workspace(), device=Qf[0].device, stream=L.stream_of(Qf[0]))
    for q, b, c in zip(Qs, Bs, Cs):
        Q64 = torch.triu((bf(q) if prec else q).double().nan_to_num(0.0))
        check_gemm_bound(c[:, :p], Q64, b.float().cpu()[:, :p].double())


# --------------------------------------------------------------------------------------------------------------
@pytest.mark.parametrize("n", [64, 100, 768, 1031])
@pytest.mark.parametrize("sign", [1, -1])
def test_tri_rownorm2(hip, n, sign):
    X = rnd(n, n, seed=n)
    S = (X + X.T) if sign > 0 else (X - X.T)
    rn2, amax = K.tri_rownorm2(poison_lower(S).to(DEV), sign)
    S64 = S.double()
    assert rel_err_norm(rn2, (S64 * S64).sum(1)) < 1e-6
    assert float(amax) == float(S.abs().max())


@pytest.mark.parametrize("n", [64, 200, 768])
@pytest.mark.parametrize("sign", [1, -1])
def test_tri_vmm(hip, n, sign):
    X = rnd(n, n, seed=n + 1)
    S = (X + X.T) if sign > 0 else (X - X.T)
    V = rnd(32, n, seed=9)
    W = K.tri_vmm(V.to(DEV), poison_lower(S).to(DEV), sign)
    check_gemm_bound(W, V.double(), S.double())


@pytest.mark.parametrize("n", [64, 130, 768, 1024])
@pytest.mark.parametrize("sign", [1, -1])
def test_norm_lower_bound_matches_oracle(hip, n, sign):
    from oracle.psgd_oracle import norm_lower_bound
    X = rnd(n, n // 2 + 1, seed=n + 2)
    S = X @ X.T if sign > 0 else (lambda Y: Y - Y.T)(rnd(n, n, seed=n + 3))
    V = rnd(32, n, seed=11)
    got = float(K.norm_lower_bound(poison_lower(S).to(DEV), V.to(DEV), sign))
    ref = float(norm_lower_bound(S.double(), V.double(), skew=sign < 0))
    assert got == pytest.approx(ref, rel=1e-5)
    top = float(torch.linalg.matrix_norm(S.double(), 2))
    assert got <= top * (1 + 1e-5)


_NLB_CASES = {}


def _nlb_case(n, sign):
    """SPD X X^T (rank n/2 + 1) or skew Y - Y^T, fixed per (n, sign)."""
    if (n, sign) not in _NLB_CASES:
        if sign > 0:
            X = rnd(n, n // 2 + 1, seed=n + 2)
            S = X @ X.T
        else:
            Y = rnd(n, n, seed=n + 3)
            S = Y - Y.T
        _NLB_CASES[(n, sign)] = S
    return _NLB_CASES[(n, sign)]


def nlb_full(As, Vs, sign):
    n = As[0].shape[0]
    outs = [torch.empty((), device=DEV, dtype=torch.float32) for _ in As]
    L.call_ws(L.lib().psgdk_norm_lower_bound_full, n, sign, len(As), L.ptrs(As), As[0].stride(0),
              L.dtype_code(As[0].dtype), L.ptrs(Vs), L.ptrs(outs), ws=L.Workspace(), device=As[0].device,
              stream=L.stream_of(As[0]))
    return [float(o) for o in outs]


@pytest.mark.parametrize("n,pad", [(1, 0), (37, 0), (100, 0), (100, 4), (100, 3), (130, 6), (768, 0), (768, 8),
                                   (1000, 8), (3072, 0)])
@pytest.mark.parametrize("sign", [1, -1])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("cols,target", [(-1, 1024), (1, 1024), (2, 1024), (3, 1024), (0, 1), (0, 1024),
                                         (0, 1 << 20)],
                         ids=["auto", "cols", "rows", "tri", "split1", "split1024", "splitmax"])
def test_norm_lower_bound_full_matches_oracle(hip, n, pad, sign, dtype, cols, target):
    """Full-storage bound (psgd_pro.py:19-65) of two matrices in one call, against the float64 oracle on the same
    (storage-rounded) matrices. cols = 1: the column-block V A kernel where the layout allows it (n and lda
    multiples of 16 bytes: fp32 n = 100 with a ragged last block, 768, 1000, 3072), else the split-K kernel;
    cols = 2: the same with A staged through LDS (n = 1000: ragged last k chunk and column block; fp32 n = 100:
    one partial chunk); cols = 3: the kernel that reads the upper 64-tiles only, in tournament-paired rounds (bf16,
    n a multiple of 128: 768, 3072; else as cols = 2); cols = -1: the library's choice by shape;
    cols = 0: the split-K kernel, whose workgroup target 1 gives one k slice, 2^20 the most slices, 1024 the
    default plan. pad > 0 gives lda = n + pad (pad 3: rows not 16-byte aligned, the element-load path; n = 768,
    pad 8: the upper-tile kernel on a row stride wider than n). fp32:
    rel 1e-5. bf16: the products run on bf16 V and A, rel 2e-2."""
    from oracle.psgd_oracle import norm_lower_bound
    S = _nlb_case(n, sign)
    S2 = 0.5 * S.flip(0).flip(1)  # another matrix of the same kind
    mats = [S.to(dtype), S2.to(dtype)]
    Vs = [rnd(32, n, seed=11), rnd(32, n, seed=12)]
    dev_mats = []
    for M in mats:
        buf = torch.zeros(n, n + pad, dtype=dtype)
        buf[:, :n] = M
        dev_mats.append(buf.to(DEV)[:, :n])
    lib = L.lib()
    assert lib.psgdk_set_option(2, target) == 0
    assert lib.psgdk_set_option(4, cols) == 0
    try:
        got = nlb_full(dev_mats, [v.to(DEV) for v in Vs], sign)
        again = nlb_full(dev_mats, [v.to(DEV) for v in Vs], sign)
    finally:
        lib.psgdk_set_option(2, 1024)
        lib.psgdk_set_option(4, -1)
    assert got == again  # fixed reduction orders: bitwise repeatable
    rel = 1e-5 if dtype == torch.float32 else 2e-2
    for M, V, g in zip(mats, Vs, got):
        ref = float(norm_lower_bound(M.double(), V.double(), skew=sign < 0))
        assert g == pytest.approx(ref, rel=rel, abs=1e-30)
        top = float(torch.linalg.matrix_norm(M.double(), 2))
        assert g <= top * (1 + rel)


@pytest.mark.parametrize("d,k", [(64, 16), (384, 128), (1000, 248), (3072, 768)])
@pytest.mark.parametrize("cols", [-1, 1, 2], ids=["auto", "cols", "rows"])
def test_norm_lower_bound_gram_matches_oracle(hip, d, k, cols):
    """psgdk_norm_lower_bound_gram: the SPD bound (psgd_pro.py:19-41) of P P^T from P (d x k bf16) without forming
    P P^T, for three matrices of different scales, against the float64 oracle on the same (bf16) P: rel 2e-2 (the
    products run on bf16 V and factors); at most ||P P^T||_2; bitwise repeatable. Each V A kernel of the
    rectangular products (cols as psgdk_set_option 4)."""
    from oracle.psgd_oracle import norm_lower_bound
    Ps = [((0.5 + b) * rnd(d, k, seed=d + k + b)).to(torch.bfloat16) for b in range(3)]
    Vs = [rnd(32, d, seed=7 + b) for b in range(3)]
    Pd = [P.to(DEV) for P in Ps]
    Ptd = [P.T.contiguous() for P in Pd]
    Vd = [v.to(DEV) for v in Vs]
    outs = [torch.empty((), device=DEV) for _ in Ps]

    def run():
        L.call_ws(L.lib().psgdk_norm_lower_bound_gram, d, k, len(Ps), L.ptrs(Pd), L.ptrs(Ptd), L.ptrs(Vd), L.ptrs(outs),
                  ws=L.Workspace(), device=Pd[0].device, stream=L.stream_of(Pd[0]))
        return [float(o) for o in outs]
    assert L.lib().psgdk_set_option(4, cols) == 0
    try:
        got, again = run(), run()
    finally:
        L.lib().psgdk_set_option(4, -1)
    assert got == again
    for P, V, g in zip(Ps, Vs, got):
        A = P.double() @ P.double().T
        ref = float(norm_lower_bound(A, V.double(), skew=False))
        assert g == pytest.approx(ref, rel=2e-2)
        assert g <= float(torch.linalg.matrix_norm(A, 2)) * (1 + 2e-2)


@pytest.mark.parametrize("n", [128, 256, 320, 384])
@pytest.mark.parametrize("cols", [-1, 1, 2, 3, 0], ids=["auto", "cols", "rows", "tri", "split"])
def test_norm_lower_bound_full_sixteen_matrices(hip, cols, n):
    """A full group (16 matrices, the most one call takes) of n x n bf16 SPD matrices of different scales: every
    matrix's bound against the float64 oracle (rel 2e-2), every V A kernel (n = 128, 256, 384: two, four and six
    64-tiles, the tournament-paired kernel with two matrices per XCD when forced, cols = 3, its four-round loop
    ending after two rounds for n = 128 and 384; by shape these launches take the row kernel)."""
    from oracle.psgd_oracle import norm_lower_bound
    mats, Vs = [], []
    for b in range(16):
        X = rnd(n, 40 + 8 * b, seed=100 + b)
        mats.append(((0.5 + b) * (X @ X.T)).to(torch.bfloat16))
        Vs.append(rnd(32, n, seed=200 + b))
    lib = L.lib()
    assert lib.psgdk_set_option(4, cols) == 0
    try:
        got = nlb_full([M.to(DEV) for M in mats], [v.to(DEV) for v in Vs], 1)
    finally:
        lib.psgdk_set_option(4, -1)
    for M, V, g in zip(mats, Vs, got):
        ref = float(norm_lower_bound(M.double(), V.double(), skew=False))
        assert g == pytest.approx(ref, rel=2e-2)


@pytest.mark.parametrize("sign", [1, -1])
def test_norm_lower_bound_full_routing_by_shape(hip, sign):
    """16 bf16 matrices of 2048 (32 tiles each, 512 workgroups): by shape (option 4 = -1) the launch takes the
    upper-tile kernel, so its bounds equal the forced upper-tile run (option 4 = 3) bit for bit; the row kernel
    (option 4 = 2) and both of them match the float64 oracle (rel 2e-2)."""
    from oracle.psgd_oracle import norm_lower_bound
    n, mats, Vs = 2048, [], []
    for b in range(16):
        if sign > 0:
            X = rnd(n, 24 + 4 * b, seed=300 + b)
            S = (0.5 + b) * (X @ X.T)
        else:
            Y = rnd(n, 16 + 2 * b, seed=400 + b)
            Z = rnd(n, 16 + 2 * b, seed=500 + b)
            S = (0.5 + b) * (Y @ Z.T - Z @ Y.T)
        mats.append(S.to(torch.bfloat16))
        Vs.append(rnd(32, n, seed=600 + b))
    dm, dv = [M.to(DEV) for M in mats], [v.to(DEV) for v in Vs]
    lib = L.lib()
    got = {}
    try:
        for cols in (-1, 3, 2):
            assert lib.psgdk_set_option(4, cols) == 0
            got[cols] = nlb_full(dm, dv, sign)
    finally:
        lib.psgdk_set_option(4, -1)
    assert got[-1] == got[3]
    assert got[3] != got[2]  # the two kernels sum in different orders: the equality above names the kernel taken
    for b, (M, V) in enumerate(zip(mats, Vs)):
        ref = float(norm_lower_bound(M.double(), V.double(), skew=sign < 0))
        assert got[3][b] == pytest.approx(ref, rel=2e-2)
        assert got[2][b] == pytest.approx(ref, rel=2e-2)


@pytest.mark.parametrize("d,tri", [(64, 0), (130, 0), (256, 0), (130, 1)])
@pytest.mark.parametrize("L0", [0.0, 7.5])
def test_factor_update_matches_oracle(hip, d, tri, L0):
    """psgdk_factor_update (psgd_pro.py:132-135) for two problems against the float64 formula with the oracle's
    norm bound on the same V: Q_out rel 1e-5 normwise, L rel 1e-5. term1 full, or its upper triangle (tri)."""
    from oracle.psgd_oracle import norm_lower_bound
    lr, betaL, term2 = 0.1, 0.9, 3.0
    T1s, Qs, Vs = [], [], []
    for b in range(2):
        X = rnd(d, d // 2 + 3, seed=d + b)
        T1s.append(X @ X.T)
        Qs.append(torch.eye(d) + 0.1 * rnd(d, d, seed=d + 10 + b))
        Vs.append(rnd(32, d, seed=d + 20 + b))
    T1d = [(poison_lower(t) if tri else t).to(DEV) for t in T1s]
    Qd = [q.to(DEV) for q in Qs]
    Qo = [torch.empty_like(q) for q in Qd]
    Ld = [torch.full((1,), L0, device=DEV) for _ in range(2)]
    Vd = [v.to(DEV) for v in Vs]
    L.call_ws(L.lib().psgdk_factor_update, 0, d, 2, L.ptrs(T1d), tri, L.ptrs(Qd), L.ptrs(Qo), L.ptrs(Ld),
              L.ptrs(Vd), lr, betaL, term2, ws=L.Workspace(), device=Qd[0].device, stream=L.stream_of(Qd[0]))
    for b in range(2):
        T, Q = T1s[b].double(), Qs[b].double()
        ell = float(norm_lower_bound(T, Vs[b].double(), skew=False)) + term2
        Lr = max(betaL * L0 + (1 - betaL) * ell, ell)
        ref = Q - lr / Lr * (T @ Q - term2 * Q)
        assert float(Ld[b]) == pytest.approx(Lr, rel=1e-5)
        assert rel_err_norm(Qo[b], ref) < 1e-5


@pytest.mark.parametrize("d", [64, 130, 256])
@pytest.mark.parametrize("prec", [0, 1])
def test_procrustes_matches_oracle(hip, d, prec):
    """psgdk_procrustes against the oracle's procrustes_step2 (psgd_pro.py:71-94) in float64 on the same V (for
    bf16 MFMA inputs, on the bf16-rounded Q): rel 1e-5 normwise for fp32, 5e-3 for bf16."""
    from oracle.psgd_oracle import procrustes_step2
    Qs = [torch.eye(d) + 0.05 * rnd(d, d, seed=d + b) for b in range(2)]
    Vs = [rnd(32, d, seed=d + 5 + b) for b in range(2)]
    Qd = [q.to(DEV) for q in Qs]
    Qo = [torch.empty_like(q) for q in Qd]
    Vd = [v.to(DEV) for v in Vs]  # held until the kernels have run (a freed block can become the workspace)
    L.call_ws(L.lib().psgdk_procrustes, prec, d, 2, L.ptrs(Qd), L.ptrs(Qo), L.ptrs(Vd),
              ws=L.Workspace(), device=Qd[0].device, stream=L.stream_of(Qd[0]))
    for b in range(2):
        ref = Qs[b].double().clone()
        procrustes_step2(ref, Vs[b].double())
        assert rel_err_norm(Qo[b], ref) < (1e-5 if prec == 0 else 5e-3)


@pytest.mark.parametrize("d", [64, 130, 256])
@pytest.mark.parametrize("prec", [0, 1])
def test_procrustes_r2_matches_oracle(hip, d, prec):
    """psgdk_procrustes_r2 against the oracle's procrustes_step_r2 (psgd_pro_fast.py:141-153) in float64 on the
    same V: rel 1e-5 normwise for fp32, 5e-3 for bf16 MFMA inputs; and against procrustes_step2 (the same
    rotation) at the same bars."""
    from oracle.psgd_oracle import procrustes_step2, procrustes_step_r2
    Qs = [torch.eye(d) + 0.05 * rnd(d, d, seed=d + b) for b in range(2)]
    Vs = [rnd(32, d, seed=d + 5 + b) for b in range(2)]
    Qd = [q.to(DEV) for q in Qs]
    Qo = [torch.empty_like(q) for q in Qd]
    Vd = [v.to(DEV) for v in Vs]  # held until the kernels have run (a freed block can become the workspace)
    L.call_ws(L.lib().psgdk_procrustes_r2, prec, d, 2, L.ptrs(Qd), L.ptrs(Qo), L.ptrs(Vd),
              ws=L.Workspace(), device=Qd[0].device, stream=L.stream_of(Qd[0]))
    tol = 1e-5 if prec == 0 else 5e-3
    for b in range(2):
        ref = Qs[b].double().clone()
        procrustes_step_r2(ref, Vs[b].double())
        assert rel_err_norm(Qo[b], ref) < tol
        ref2 = Qs[b].double().clone()
        procrustes_step2(ref2, Vs[b].double())
        assert rel_err_norm(Qo[b], ref2) < tol


def test_hip_ops_plugin_methods(hip):
    """The ops class methods (psgd_pro_fast.EagerOps interface) against their eager definitions."""
    ops = K.make_ops(())
    X = rnd(96, 160, seed=1).to(DEV)
    assert rel_err_norm(ops.syrk(X, True), X.double().cpu().T @ X.double().cpu()) < 1e-6
    assert rel_err_norm(ops.sym(X, False), X.double().cpu() @ X.double().cpu().T) < 1e-6
    assert rel_err_norm(ops.gram(X, 0, None), X.double().cpu() @ X.double().cpu().T) < 1e-6
    S = ops.syrk(X, False)
    Y = rnd(96, 40, seed=2).to(DEV)
    assert rel_err_norm(ops.symm(S, Y), S.double().cpu() @ Y.double().cpu()) < 1e-6
    Z = rnd(40, 96, seed=3).to(DEV)
    assert rel_err_norm(ops.symm_r(Z, S), Z.double().cpu() @ S.double().cpu()) < 1e-6
    q = rnd(96, 96, seed=4).to(DEV)
    assert rel_err_norm(ops.gram_q(q), q.double().cpu().T @ q.double().cpu()) < 1e-6
    tri = K.make_ops({"k1", "tri", "nan"})
    T = tri.sym(X, False)
    assert bool(torch.isnan(T.tril(-1)[1:, :1]).all())
    assert rel_err_norm(tri.symm(T, Y), S.double().cpu() @ Y.double().cpu()) < 1e-6
    pk = K.make_ops({"packed"})
    P = pk.sym(X, False)
    assert P.dim() == 1 and rel_err_norm(pk.symm(P, Y), S.double().cpu() @ Y.double().cpu()) < 1e-6


# -------------------------------------------------------------------------------------------------------------- bf16
@pytest.mark.parametrize("m,n,k", [(256, 256, 256), (512, 768, 320), (768, 768, 2304), (100, 70, 33), (1, 50, 77),
                                   (264, 520, 72), (3072, 768, 768), (4096, 4096, 256)])
def test_gemm_bf16_k_contiguous(hip, b16cfg, m, n, k):
    """A (m x k) B^T (B given n x k), both bf16 k-contiguous: the dedicated bf16 kernel in every tile
    configuration (interior tiles take the unchecked epilogue, ragged ones the checked one)."""
    A = rnd(m, k, seed=m).to(torch.bfloat16)
    B = rnd(n, k, seed=n + 1).to(torch.bfloat16)
    C = K.gemm(A.to(DEV), B.to(DEV), False, True, True)
    check_gemm_bound(C, A.double(), B.double().T)


@pytest.mark.parametrize("nb,m,n,k", [(1, 256, 256, 256), (1, 100, 70, 36), (1, 1, 50, 76), (1, 264, 520, 72),
                                      (1, 3072, 768, 768), (1, 1024, 1024, 3072), (12, 768, 768, 768)])
def test_gemm_f32_k_contiguous(hip, nb, m, n, k):
    """A (m x k) B^T with both fp32 operands k-contiguous (k a multiple of 4): the fp32 twin of the bf16 kernel (128
    tiles, k summed in blocks of 128). Against float64: the elementwise bound of the other GEMM tests, and a worst
    error no more than twice the general fp32 engine's on the same product (psgdk_set_option 8 = 0)."""
    As = [rnd(m, k, seed=m + i) for i in range(nb)]
    Bs = [rnd(n, k, seed=n + 7 * i + 1) for i in range(nb)]
    Ad = [a.to(DEV) for a in As]
    Bd = [b_.to(DEV) for b_ in Bs]
    Cs = [torch.empty(m, n, device=DEV) for _ in range(nb)]
    Cg = [torch.empty(m, n, device=DEV) for _ in range(nb)]

    def run(out):
        L.check(hip.psgdk_gemm(0, 0, 1, m, n, k, 1.0, 0, 0, nb, L.ptrs(Ad), k, L.ptrs(Bd), k, 0.0, L.ptrs(out), n,
                               L.stream_of(Ad[0])))
    try:
        run(Cs)
        assert hip.psgdk_set_option(8, 0) == 0
        run(Cg)
    finally:
        hip.psgdk_set_option(8, 1)
    for A, B, C, G in zip(As, Bs, Cs, Cg):
        check_gemm_bound(C, A.double(), B.double().T)
        ref = A.double() @ B.double().T
        e_kc = float((C.double().cpu() - ref).abs().max())
        e_gen = float((G.double().cpu() - ref).abs().max())
        assert e_kc <= 2.0 * e_gen + 1e-6 * float(ref.abs().max()), (e_kc, e_gen)


@pytest.mark.parametrize("order", [0, 1, 2])
@pytest.mark.parametrize("nb,m,n,k", [(12, 768, 768, 768), (12, 1024, 1024, 512), (5, 1300, 520, 264)])
def test_gemm_bf16_grouped(hip, b16cfg, order, nb, m, n, k):
    """Grouped launches under every tile order (problem-major; contiguous runs per XCD; runs with tile rows grouped
    by 4, where the last group of a problem may be shorter): each maps the grid onto every tile exactly once."""
    assert hip.psgdk_set_option(0, order) == 0
    As = [rnd(m, k, seed=i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    Bs = [rnd(n, k, seed=50 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    Cs = [torch.empty(m, n, device=DEV) for _ in range(nb)]
    L.check(hip.psgdk_gemm(1, 0, 1, m, n, k, 1.0, 1, 1, nb, L.ptrs(As), k, L.ptrs(Bs), k, 0.0, L.ptrs(Cs), n,
                           L.stream_of(As[0])))
    hip.psgdk_set_option(0, 2)
    for A, B, C in zip(As, Bs, Cs):
        check_gemm_bound(C, A.double().cpu(), B.double().cpu().T)


def test_syrk_bf16_microbench_shape(hip):
    """One bf16 SYRK at n = k = 4096 (136 triangle tiles of 256: the size rule takes the 256-tile kernel because
    K >= 4096) against float64, and bitwise equal to the 256-tile configuration forced."""
    n = 4096
    A = rnd(n, n, seed=4096).to(torch.bfloat16).to(DEV)
    C = torch.full((n, n), float("nan"), device=DEV)
    C0 = torch.full((n, n), float("nan"), device=DEV)
    st = L.stream_of(A)
    L.check(hip.psgdk_syrk(1, 0, L.OUT_UPPER, n, n, 1, 1, L.ptrs([A]), n, L.ptrs([C]), n, st))
    try:
        L.check(hip.psgdk_set_option(1, 0))
        L.check(hip.psgdk_syrk(1, 0, L.OUT_UPPER, n, n, 1, 1, L.ptrs([A]), n, L.ptrs([C0]), n, st))
    finally:
        L.check(hip.psgdk_set_option(1, -1))
    triu = torch.ones(n, n, dtype=torch.bool, device=DEV).triu()
    assert torch.equal(C[triu], C0[triu])
    Cc = C.cpu()
    triu = triu.cpu()
    assert bool(torch.isnan(Cc[~triu]).all())
    X = A.double().cpu()
    check_gemm_bound(torch.where(triu, Cc, Cc.T), X, X.T)


@pytest.mark.parametrize("kind,nb,m,n,k", [("gemm", 2, 768, 768, 2304), ("gemm", 1, 300, 520, 264),
                                            ("syrk", 3, 1000, 1000, 512), ("syrk", 1, 2304, 2304, 3072)])
def test_load_only_waves_give_the_same_sums(hip, kind, nb, m, n, k):
    """The 256-tile configuration with load-only waves and 32 x 32 x 16 MFMAs (option 1 = 3) and the 128-tile
    configuration (option 1 = 1) return bit for bit what the ping-pong configuration on 16 x 16 x 32 MFMAs (option 1 =
    0) returns, edge tiles included: every configuration sums k in the same order, so the size rule's choice (which
    looks at the whole launch) does not change a problem's result."""
    A = [rnd(m, k, seed=10 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    B = [rnd(n, k, seed=20 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    out = {c: [torch.full((m, n), float("nan"), device=DEV) for _ in range(nb)] for c in (0, 1, 3, 4)}
    st = L.stream_of(A[0])
    try:
        for c in (0, 1, 3, 4):
            L.check(hip.psgdk_set_option(1, c))
            if kind == "gemm":
                L.check(hip.psgdk_gemm(1, 0, 1, m, n, k, 1.0, 1, 1, nb, L.ptrs(A), k, L.ptrs(B), k, 0.0,
                                       L.ptrs(out[c]), n, st))
            else:
                L.check(hip.psgdk_syrk(1, 0, L.OUT_MIRROR, n, k, 1, nb, L.ptrs(A), k, L.ptrs(out[c]), n, st))
    finally:
        L.check(hip.psgdk_set_option(1, -1))
    for b in range(nb):
        assert torch.equal(out[0][b], out[3][b]), (kind, b)
        assert torch.equal(out[0][b], out[1][b]), (kind, b, "128-tile configuration")
        assert torch.equal(out[0][b], out[4][b]), (kind, b, "128-tile configuration with load-only waves")
    X = A[0].double().cpu()
    Y = X if kind == "syrk" else B[0].double().cpu()
    check_gemm_bound(out[3][0].cpu(), X, Y.T)


def test_launch_records_name_shape_and_occupancy(hip):
    """The launch profiler's records carry each launch's problem shape, its workgroup count (tiles x problems) and
    the occupancy the runtime reports for its kernel: one 256-tile workgroup per CU for configurations 0 and 3, two
    128-tile workgroups of eight waves per CU for configuration 4 (the load-only-wave loop is built for that)."""
    nb, m, n, k = 2, 520, 264, 1040
    A = [rnd(m, k, seed=30 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    B = [rnd(n, k, seed=40 + i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    C = [torch.empty(m, m, device=DEV) for _ in range(nb)]
    st = L.stream_of(A[0])
    recs = {}
    try:
        for c in (0, 1, 3, 4):
            L.check(hip.psgdk_set_option(1, c))
            L.profile_start()
            L.check(hip.psgdk_gemm(1, 0, 1, m, n, k, 1.0, 1, 1, nb, L.ptrs(A), k, L.ptrs(B), k, 0.0, L.ptrs(C), n,
                                   st))
            L.check(hip.psgdk_syrk(1, 0, L.OUT_MIRROR, m, k, 1, nb, L.ptrs(A), k, L.ptrs(C), m, st))
            recs[c] = L.profile_stop()
    finally:
        L.check(hip.psgdk_set_option(1, -1))
    for c, (g, s) in recs.items():
        t = 128 if c in (1, 4) else 256
        tm, tn = -(-m // t), -(-n // t)
        assert (g.kernel_id, g.tri, g.nb, g.m, g.n, g.k) == (5000 + 10 * c, 0, nb, m, n, k), g
        assert (s.kernel_id, s.tri, s.nb, s.m, s.n, s.k) == (5000 + 10 * c, 1, nb, m, m, k), s
        assert g.workgroups == tm * tn * nb and s.workgroups == tm * (tm + 1) // 2 * nb, (g, s)
        assert g.per_cu == s.per_cu >= 1, (g, s)
        if c in (0, 3):
            assert g.per_cu == 1, g
        if c == 4:
            assert g.per_cu == 2, g


@pytest.mark.parametrize("nb,n,k", [(1, 768, 2304), (1, 3072, 768), (16, 1024, 256), (1, 200, 72)])
def test_syrk_bf16_k_contiguous(hip, b16cfg, nb, n, k):
    As = [rnd(n, k, seed=i).to(torch.bfloat16).to(DEV) for i in range(nb)]
    Cs = [torch.full((n, n), float("nan"), device=DEV) for _ in range(nb)]
    L.check(hip.psgdk_syrk(1, 0, L.OUT_UPPER, n, k, 1, nb, L.ptrs(As), k, L.ptrs(Cs), n, L.stream_of(As[0])))
    triu = torch.ones(n, n, dtype=torch.bool).triu()
    for A, C in zip(As, Cs):
        X = A.double().cpu()
        Cc = C.cpu()
        assert bool(torch.isnan(Cc[~triu]).all())
        check_gemm_bound(torch.where(triu, Cc, Cc.T), X, X.T)


@pytest.mark.parametrize("n", [512, 1024, 2048, 4096])
@pytest.mark.parametrize("prec", [0, 1], ids=["fp32", "bf16"])
def test_microbench_cells(hip, n, prec):
    """Every cell of the SYRK / TRMM microbenchmark as `bench.py --config syrk` runs it: C = triu(A A^T) with A n x n
    (n = k) stored in the precision's dtype, one problem per call, against float64 with the strict lower triangle
    left untouched; and triu(Q) B with fp32 Q (its strict lower triangle NaN-poisoned) and B, n x n."""
    dt = torch.bfloat16 if prec else torch.float32
    A = rnd(n, n, seed=n).to(dt)
    Ad = A.to(DEV)
    C = torch.full((n, n), float("nan"), device=DEV)
    L.check(hip.psgdk_syrk(prec, 0, L.OUT_UPPER, n, n, L.dtype_code(dt), 1, L.ptrs([Ad]), n, L.ptrs([C]), n,
                           L.stream_of(Ad)))
    triu = torch.ones(n, n, dtype=torch.bool).triu()
    Cc = C.cpu()
    assert bool(torch.isnan(Cc[~triu]).all())
    X = A.double()
    check_gemm_bound(torch.where(triu, Cc, Cc.T), X, X.T)
    Q = rnd(n, n, seed=n + 1)
    B = rnd(n, n, seed=n + 2)
    Ct = K.trmm(poison_lower(Q).to(DEV), B.to(DEV), bool(prec))
    check_gemm_bound(Ct, torch.triu((bf(Q) if prec else Q).double()), (bf(B) if prec else B).double())


def test_momentum_multi_matches_per_tensor(hip):
    """psgdk_momentum_multi over tensors of different sizes and gradient dtypes in one launch equals
    psgdk_momentum on each tensor bit for bit (the same arithmetic), and m = beta m + (1 - beta) g to fp32 rounding."""
    import ctypes
    sizes = [1, 7, 512, 65 * 512, 1000, 3, 1536 * 512]
    dts = [torch.float32, torch.bfloat16, torch.float32, torch.bfloat16, torch.float32, torch.bfloat16, torch.float32]
    g = [rnd(n, seed=i).to(dt).to(DEV) for i, (n, dt) in enumerate(zip(sizes, dts))]
    m0 = [rnd(n, seed=50 + i).to(DEV) for i, n in enumerate(sizes)]
    beta = 0.75
    ma = [m.clone() for m in m0]
    numel = (ctypes.c_int64 * len(sizes))(*sizes)
    codes = (ctypes.c_int32 * len(sizes))(*[L.dtype_code(dt) for dt in dts])
    L.check(hip.psgdk_momentum_multi(len(sizes), numel, beta, codes, L.ptrs(ma), L.ptrs(g), L.stream_of(g[0])))
    mb = [m.clone() for m in m0]
    for x, gx in zip(mb, g):
        L.check(hip.psgdk_momentum(x.numel(), beta, L.dtype_code(gx.dtype), 1, L.ptrs([x]), L.ptrs([gx]),
                                   L.stream_of(g[0])))
    torch.cuda.synchronize()
    for a, b, m, gx in zip(ma, mb, m0, g):
        assert torch.equal(a, b)
        ref = beta * m.double() + (1 - beta) * gx.double()
        assert rel_err_norm(a, ref) < 1e-6
    # a gradient view off the 16-byte grid takes every tensor of the launch through the element path: same values
    gv = torch.cat([torch.zeros(1, device=DEV), g[2].float()])[1:]
    mc = [m.clone() for m in m0[:3]]
    L.check(hip.psgdk_momentum_multi(3, numel, beta, codes, L.ptrs(mc), L.ptrs([g[0], g[1], gv]), L.stream_of(g[0])))
    torch.cuda.synchronize()
    for a, b in zip(mc, mb[:3]):
        assert torch.equal(a, b)


@pytest.mark.parametrize("kind,nb,m,n,k,dt", [("syrk_upper", 1, 512, 512, 512, torch.bfloat16),
                                              ("syrk_mirror", 3, 300, 300, 1032, torch.bfloat16),
                                              ("gemm", 2, 200, 136, 2056, torch.bfloat16),
                                              ("gemm", 1, 64, 64, 8, torch.bfloat16),
                                              ("gemm", 12, 40, 72, 264, torch.bfloat16),
                                              ("syrk_upper", 1, 512, 512, 512, torch.float32),
                                              ("syrk_mirror", 2, 130, 130, 260, torch.float32),
                                              ("syrk_mirror", 9, 33, 33, 44, torch.float32),
                                              ("gemm", 4, 130, 260, 524, torch.float32)])
def test_small_kernel(hip, kind, nb, m, n, k, dt):
    """Products whose 128-tiles would leave most CUs idle take the small-problem kernel (64-tiles, k in chunks of
    512 bytes per row, option 10), or, with option 11 above their 64-tile count, the tiny-product kernel (32-tiles,
    k split over the four waves; launches of more than 8 problems split): each against float64 within the GEMM
    bound, a SYRK's lower triangle untouched in upper mode, and the pipelined kernel's result (option 10 = 0) within
    the same bound."""
    prec = 1 if dt == torch.bfloat16 else 0
    dcode = L.dtype_code(dt)
    As = [rnd(m, k, seed=5 * i + 1).to(dt).to(DEV) for i in range(nb)]
    Bs = [rnd(n, k, seed=5 * i + 2).to(dt).to(DEV) for i in range(nb)]
    st = L.stream_of(As[0])

    def run(small, tiny):
        Cs = [torch.full((m, n), float("nan"), device=DEV) for _ in range(nb)]
        assert hip.psgdk_set_option(10, small) == 0 and hip.psgdk_set_option(11, tiny) == 0
        L.profile_start()
        if kind == "gemm":
            L.check(hip.psgdk_gemm(prec, 0, 1, m, n, k, 1.0, dcode, dcode, nb, L.ptrs(As), k, L.ptrs(Bs), k, 0.0,
                                   L.ptrs(Cs), n, st))
        else:
            mode = L.OUT_UPPER if kind == "syrk_upper" else L.OUT_MIRROR
            L.check(hip.psgdk_syrk(prec, 0, mode, m, k, dcode, nb, L.ptrs(As), k, L.ptrs(Cs), m, st))
        recs = L.profile_stop()
        return Cs, recs
    try:
        small, recs_s = run(128, 0)
        tiny, recs_t = run(128, 1 << 20)
        pipe, _ = run(0, 0)
    finally:
        hip.psgdk_set_option(10, 128)
        hip.psgdk_set_option(11, 64)
    assert [r[0] for r in recs_s] == [7000 if prec else 7001], recs_s
    assert {r[0] for r in recs_t} == {7002 if prec else 7003} and len(recs_t) == 1, recs_t
    triu = torch.ones(m, n, dtype=torch.bool).triu()
    for A, B, C, T, P in zip(As, Bs, small, tiny, pipe):
        X = A.double().cpu()
        Y = X if kind != "gemm" else B.double().cpu()
        Cc, Tc, Pc = C.cpu(), T.cpu(), P.cpu()
        if kind == "syrk_upper":
            for Z in (Cc, Tc):
                assert bool(torch.isnan(Z[~triu]).all()) and not bool(torch.isnan(Z[triu]).any())
            Cc, Tc, Pc = (torch.where(triu, Z, Z.T) for Z in (Cc, Tc, Pc))
        else:
            assert not bool(torch.isnan(Cc).any()) and not bool(torch.isnan(Tc).any())
        for Z in (Cc, Tc, Pc):
            check_gemm_bound(Z, X, Y.T)


def test_mfma_rate_kernel(hip):
    """The MFMA-rate calibration kernel: every wave computes the same sums from the same lane operands (lane 0 of
    each of the 4 waves of each workgroup writes one), so the output is finite and uniform, and grows with iters."""
    outs = []
    for iters in (1, 3):
        out = torch.full((4 * 8,), float("nan"), device=DEV)
        L.check(hip.psgdk_mfma_rate(iters, 8, C_ptr(out), L.stream_of(out)))
        o = out.cpu()
        assert bool(torch.isfinite(o).all()) and bool((o == o[0]).all()), o
        outs.append(float(o[0]))
    assert abs(outs[1] - 3 * outs[0]) <= 1e-3 * abs(outs[1])
    assert hip.psgdk_mfma_rate(0, 8, C_ptr(out), L.stream_of(out)) == L.EINVAL


def test_fill_normal_matches_philox_reference(hip):
    """psgdk_fill_normal against the Python Philox4x32-10 + Box-Muller checker (itself pinned to the published
    known-answer vectors): the first 1003 fp32 normals of two (seed, stream) pairs within 2e-5 (1 + |z|) of the
    float64 values; bf16 storage equals the fp32 values rounded; another stream gives other values; one million
    normals have mean and variance within 5 standard errors of 0 and 1."""
    from philox_ref import normals
    st = L.stream_of(torch.empty(1, device=DEV))
    for seed, sid in [(0, 0), ((1 << 61) + 12345, 3)]:
        n = 1003
        out = torch.full((n + 5,), float("nan"), device=DEV)
        L.check(hip.psgdk_fill_normal(C_ptr(out), n, L.F32, seed, sid, st))
        got = out.cpu().double()
        ref = torch.tensor(normals(n, seed, sid), dtype=torch.float64)
        assert bool(torch.isnan(got[n:]).all())
        # fp32 with the hardware log2 / sqrt / sin / cos: within 2e-5 (1 + |z|) of the float64 values
        assert bool(((got[:n] - ref).abs() <= 2e-5 * (1 + ref.abs())).all()), float((got[:n] - ref).abs().max())
        o16 = torch.empty(n, device=DEV, dtype=torch.bfloat16)
        L.check(hip.psgdk_fill_normal(C_ptr(o16), n, L.BF16, seed, sid, st))
        assert torch.equal(o16.cpu(), out[:n].cpu().to(torch.bfloat16))
    a = torch.empty(1 << 20, device=DEV)
    b_ = torch.empty(1 << 20, device=DEV)
    L.check(hip.psgdk_fill_normal(C_ptr(a), a.numel(), L.F32, 7, 0, st))
    L.check(hip.psgdk_fill_normal(C_ptr(b_), b_.numel(), L.F32, 7, 1, st))
    n = a.numel()
    assert not torch.equal(a, b_)
    assert abs(float(a.double().mean())) < 5 / math.sqrt(n)
    assert abs(float(a.double().var()) - 1) < 5 * math.sqrt(2 / n)
    assert hip.psgdk_fill_normal(C_ptr(a[1:]), 8, L.F32, 7, 0, st) == L.EINVAL  # misaligned


def test_measurement_kernels(hip):
    """psgdk_read_rate reads a buffer once (stride 1) and many times (odd stride) without writing its sink;
    psgdk_clock_sample's counters advance and give an engine clock between 0.3 and 3 GHz; the two psgdk_wall_mark
    marks bracket every sample of a sampler launched between them on the same stream."""
    import ctypes as C
    buf = torch.ones(1 << 20, dtype=torch.uint8, device=DEV)
    sink = torch.zeros(64, dtype=torch.int32, device=DEV)
    st = L.stream_of(buf)
    L.check(hip.psgdk_read_rate(C_ptr(buf), 1 << 20, 64, 4, 1, C_ptr(sink), st))
    L.check(hip.psgdk_read_rate(C_ptr(buf), 1 << 20, 64, 64, 977, C_ptr(sink), st))
    samples = torch.zeros(2 * 16, dtype=torch.int64, device=DEV)
    marks = torch.zeros(2, dtype=torch.int64, device=DEV)
    L.check(hip.psgdk_wall_mark(C_ptr(marks), st))
    L.check(hip.psgdk_clock_sample(16, C_ptr(samples), st))
    L.check(hip.psgdk_wall_mark(C.c_void_p(marks.data_ptr() + 8), st))
    torch.cuda.synchronize()
    assert int(sink.abs().sum()) == 0
    s = samples.cpu().view(16, 2)
    cyc, wall = s[:, 0], s[:, 1]
    assert bool((cyc[1:] > cyc[:-1]).all()) and bool((wall[1:] > wall[:-1]).all())
    khz = C.c_int(0)
    L.check(hip.psgdk_wall_clock_rate(C.byref(khz)))
    assert khz.value > 0
    mhz = float(cyc[-1] - cyc[0]) / float(wall[-1] - wall[0]) * khz.value / 1e3
    print(f"engine clock {mhz:.0f} MHz (wall counter {khz.value} kHz)", flush=True)
    assert 300 < mhz < 3000
    m = marks.cpu()
    assert int(m[0]) <= int(wall[0]) and int(wall[-1]) <= int(m[1])


@pytest.mark.parametrize("flags", [("k1", "k2"), ("k1", "k2t", "all"), ("k2c",), ("k2b", "nan"), ("k1", "k2", "tri"),
                                   ("k1", "tri", "nan", "packed")])
def test_reference_flag_sets_compute_the_eager_methods(hip, flags):
    """Plugins built from the reference's own flag sets (kernels/ops.py:142-215) return the values of the eager
    definitions (psgd_pro_fast.py:106-126) for every method: syrk / gram_q full, sym / gram in the storage form the
    flags ask for (full, upper triangle with an optional NaN lower part, or packed), symm / symm_r from that form, the
    norm bounds equal to the full-matrix ones on the same start."""
    ops = K.make_ops(set(flags))
    X = rnd(96, 160, seed=1).to(DEV)
    X64 = X.double().cpu()
    S64 = X64 @ X64.T
    Y = rnd(96, 40, seed=2).to(DEV)
    Z = rnd(40, 96, seed=3).to(DEV)
    assert rel_err_norm(ops.syrk(X, False), S64) < 1e-6
    assert rel_err_norm(ops.gram_q(X), X64.T @ X64) < 1e-6
    S = ops.sym(X, False)
    tri, packed = "tri" in flags, "packed" in flags
    if packed:
        assert S.dim() == 1 and S.numel() == 96 * 97 // 2
        assert rel_err_norm(K.unpack(S, 96), S64) < 1e-6
    elif tri:
        assert S.shape == (96, 96) and rel_err_norm(S.triu(), S64.triu()) < 1e-6
        if "nan" in flags:
            assert bool(torch.isnan(S.tril(-1)).sum() == 96 * 95 // 2)
    else:
        assert rel_err_norm(S, S64) < 1e-6
    G = ops.gram(X, 0, None)
    assert rel_err_norm(G.triu() if tri else G, S64.triu() if tri else S64) < 1e-6
    assert rel_err_norm(ops.symm(S, Y), S64 @ Y.double().cpu()) < 1e-6
    assert rel_err_norm(ops.symm_r(Z, S), Z.double().cpu() @ S64) < 1e-6
    Sf = ops.syrk(X, False)
    V = rnd(32, 96, seed=5).to(DEV)
    ref = float(K.norm_lower_bound(Sf, V, 1))
    assert abs(float(ops.norm_lower_bound_spd(S, V)) - ref) <= 1e-5 * ref
    A = rnd(96, 96, seed=6).to(DEV)
    R = A - A.T  # skew, a non-contiguous expression as Q^T - Q is in the reference
    ref_k = float(K.norm_lower_bound(R.contiguous(), V, -1))
    assert ref_k > 0 and float(ops.norm_lower_bound_skh(R, V)) == ref_k


def test_optimizer_takes_storage_from_the_plugin(hip):
    """KronWhiten(ops=make_ops({"k1", "tri"})) keeps term1 and P as upper triangles: bitwise the same run as
    KronWhiten(tri=True), and EagerOps (the default) bitwise the same as tri=False."""
    shapes = [(96, 64), (64, 96)]
    gen = torch.Generator().manual_seed(7)
    grads = [[(0.01 * torch.randn(s, generator=gen)).to(DEV) for s in shapes] for _ in range(3)]
    out = {}
    for name, kw in (("ops_tri", dict(ops=K.make_ops({"k1", "tri"}))), ("tri", dict(tri=True)),
                     ("eager", dict(ops=K.EagerOps)), ("full", dict(tri=False))):
        W = [torch.zeros(s, device=DEV, requires_grad=True) for s in shapes]
        opt = KronWhiten(W, preconditioner_max_skew=math.inf, preconditioner_init_scale=1.0, draws="host", seed=3,
                           **kw)
        for gs in grads:
            opt.step_math(gs)
        torch.cuda.synchronize()
        out[name] = ([w.detach().clone() for w in W], [q.clone() for i in range(len(shapes)) for q in opt.factors(i)[0]])
    for a, b in (("ops_tri", "tri"), ("eager", "full")):
        for x, y in zip(out[a][0] + out[a][1], out[b][0] + out[b][1]):
            assert torch.equal(x, y), (a, b)
