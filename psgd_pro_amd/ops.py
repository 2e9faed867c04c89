"""The arithmetic plugin of the PSGD-Kron optimizer on the HIP kernels (the `ops` boundary).

Mirrors the reference's plugin interface: the `ops` class with static methods gram, gram_q, norm_lower_bound_spd,
norm_lower_bound_skh, symm, syrk, sym, symm_r and attributes qsym, flags (psgd_pro_fast.py:106-126, built by
make_ops(flags) in kernels/ops.py:142-215), and the custom ops under it (kernels/ops.py:24-116), registered here as
torch.library custom ops in the "psgdk" namespace with fake implementations. Every op runs on the HIP kernels of
libpsgdk.so; there is no CPU or eager fallback for the 2-D contractions (inputs must be CUDA tensors).

make_ops flags: the reference's set (kernels/ops.py:1-13: k1, k2, k2t, k2c, k2b, all, tri, nan, packed) and bf16;
make_ops's docstring gives what each one selects here.
"""
import torch
from torch import Tensor
from torch.library import custom_op

from . import _lib as L

_WS = {}


def _ws(t):
    """The workspace of t's device and its current stream. Calls on one stream run in order, so they share one
    buffer; calls on another stream get their own, and a buffer that grows goes back to torch's caching allocator on
    the one stream that used it."""
    key = (t.device, torch.cuda.current_stream(t.device).cuda_stream)
    w = _WS.get(key)
    if w is None:
        w = _WS[key] = L.Workspace()
    return w


def _prec(bf16):
    return L.PREC_BF16 if bf16 else L.PREC_F32


def _cuda(*ts):
    for t in ts:
        if not t.is_cuda:
            raise RuntimeError("psgd_pro_amd ops take CUDA (HIP) tensors; got a tensor on " + str(t.device))


def _as_2d(t, name):
    if t.dim() != 2:
        raise RuntimeError(f"{name}: expected a 2-D tensor, got shape {tuple(t.shape)}")
    if t.dtype not in (torch.float32, torch.bfloat16):
        raise RuntimeError(f"{name}: float32 or bfloat16 expected, got {t.dtype}")
    return t if t.stride(1) == 1 else t.contiguous()


@custom_op("psgdk::syrk", mutates_args=())
def syrk(A: Tensor, trans: bool, out_mode: int, bf16: bool) -> Tensor:
    """C = A A^T (trans False) or A^T A (trans True), only the upper-triangle tiles computed; out_mode 0 upper
    triangle (lower left uninitialised), 1 mirrored full matrix, 2 packed upper triangle (kernels/ops.py:55-109)."""
    _cuda(A)
    A = _as_2d(A, "A")
    n, k = (A.shape[1], A.shape[0]) if trans else (A.shape[0], A.shape[1])
    C = torch.empty(n * (n + 1) // 2 if out_mode == L.OUT_PACKED else (n, n), device=A.device, dtype=torch.float32)
    L.check(L.lib().psgdk_syrk(_prec(bf16), int(trans), out_mode, n, k, L.dtype_code(A.dtype), 1, L.ptrs([A]),
                               A.stride(0), L.ptrs([C]), n, L.stream_of(A)))
    return C


@syrk.register_fake
def _(A, trans, out_mode, bf16):
    n = A.shape[1] if trans else A.shape[0]
    return A.new_empty(n * (n + 1) // 2 if out_mode == L.OUT_PACKED else (n, n), dtype=torch.float32)


@custom_op("psgdk::symm", mutates_args=())
def symm(S: Tensor, B: Tensor, sign: int, bf16: bool) -> Tensor:
    """C = S B with S read from its upper triangle (sign 1 symmetric, -1 skew, 0 upper-triangular)
    (kernels/ops.py:45-52, kernels/blas.cpp:36-49)."""
    _cuda(S, B)
    S = _as_2d(S, "S").float()
    B = _as_2d(B, "B")
    n, p = S.shape[0], B.shape[1]
    C = torch.empty(n, p, device=B.device, dtype=torch.float32)
    L.check(L.lib().psgdk_symm(_prec(bf16), 0, sign, n, p, L.dtype_code(B.dtype), 1, L.ptrs([S]), S.stride(0),
                               L.ptrs([B]), B.stride(0), L.ptrs([C]), p, L.stream_of(B)))
    return C


@symm.register_fake
def _(S, B, sign, bf16):
    return B.new_empty(S.shape[0], B.shape[1], dtype=torch.float32)


@custom_op("psgdk::symm_right", mutates_args=())
def symm_right(B: Tensor, S: Tensor, sign: int, bf16: bool) -> Tensor:
    """C = B S with S read from its upper triangle (kernels/ops.py:90-97, kernels/blas.cpp:52-65)."""
    _cuda(S, B)
    S = _as_2d(S, "S").float()
    B = _as_2d(B, "B")
    n, p = S.shape[0], B.shape[0]
    C = torch.empty(p, n, device=B.device, dtype=torch.float32)
    L.check(L.lib().psgdk_symm(_prec(bf16), 1, sign, n, p, L.dtype_code(B.dtype), 1, L.ptrs([S]), S.stride(0),
                               L.ptrs([B]), B.stride(0), L.ptrs([C]), n, L.stream_of(B)))
    return C


@symm_right.register_fake
def _(B, S, sign, bf16):
    return B.new_empty(B.shape[0], S.shape[0], dtype=torch.float32)


@custom_op("psgdk::trmm", mutates_args=())
def trmm(Q: Tensor, B: Tensor, bf16: bool) -> Tensor:
    """C = triu(Q) B; Q's strict lower triangle is never read."""
    _cuda(Q, B)
    Q = _as_2d(Q, "Q").float()
    B = _as_2d(B, "B")
    n, p = Q.shape[0], B.shape[1]
    C = torch.empty(n, p, device=B.device, dtype=torch.float32)
    L.call_ws(L.lib().psgdk_trmm_ws, _prec(bf16), n, p, L.dtype_code(B.dtype), 1, L.ptrs([Q]), Q.stride(0),
              L.ptrs([B]), B.stride(0), L.ptrs([C]), p, ws=_ws(B), device=B.device, stream=L.stream_of(B))
    return C


@trmm.register_fake
def _(Q, B, bf16):
    return B.new_empty(Q.shape[0], B.shape[1], dtype=torch.float32)


@custom_op("psgdk::gemm", mutates_args=())
def gemm(A: Tensor, B: Tensor, trans_a: bool, trans_b: bool, bf16: bool) -> Tensor:
    """C = op(A) op(B) on the MFMA engine (the plain dense contractions of the hot path)."""
    _cuda(A, B)
    A = _as_2d(A, "A")
    B = _as_2d(B, "B")
    m, k = (A.shape[1], A.shape[0]) if trans_a else (A.shape[0], A.shape[1])
    n = B.shape[0] if trans_b else B.shape[1]
    C = torch.empty(m, n, device=A.device, dtype=torch.float32)
    L.check(L.lib().psgdk_gemm(_prec(bf16), int(trans_a), int(trans_b), m, n, k, 1.0, L.dtype_code(A.dtype),
                               L.dtype_code(B.dtype), 1, L.ptrs([A]), A.stride(0), L.ptrs([B]), B.stride(0), 0.0,
                               L.ptrs([C]), n, L.stream_of(A)))
    return C


@gemm.register_fake
def _(A, B, trans_a, trans_b, bf16):
    return A.new_empty(A.shape[1] if trans_a else A.shape[0], B.shape[0] if trans_b else B.shape[1],
                       dtype=torch.float32)


@custom_op("psgdk::tri_rownorm2", mutates_args=())
def tri_rownorm2(A: Tensor, sign: int) -> tuple[Tensor, Tensor]:
    """(squared row norms, max |A_ij|) of the symmetric / skew matrix in A's upper triangle
    (kernels/ops.py:34-42)."""
    _cuda(A)
    A = _as_2d(A, "A").float()
    n = A.shape[0]
    rn2 = torch.empty(n, device=A.device, dtype=torch.float32)
    amax = torch.empty((), device=A.device, dtype=torch.float32)
    L.call_ws(L.lib().psgdk_tri_rownorm2, n, sign, 1, L.ptrs([A]), A.stride(0), L.ptrs([rn2]), L.ptrs([amax]),
              ws=_ws(A), device=A.device, stream=L.stream_of(A))
    return rn2, amax


@tri_rownorm2.register_fake
def _(A, sign):
    return A.new_empty(A.shape[0], dtype=torch.float32), A.new_empty((), dtype=torch.float32)


@custom_op("psgdk::tri_vmm", mutates_args=())
def tri_vmm(V: Tensor, A: Tensor, sign: int) -> Tensor:
    """W = V A_sym, V (32, n), A_sym from A's upper triangle (kernels/ops.py:24-31)."""
    _cuda(V, A)
    A = _as_2d(A, "A").float()
    V = V.float().contiguous()
    n = A.shape[0]
    if V.shape != (L.NLB_K, n):
        raise RuntimeError(f"V: expected shape ({L.NLB_K}, {n}), got {tuple(V.shape)}")
    W = torch.empty_like(V)
    L.call_ws(L.lib().psgdk_tri_vmm, n, sign, 1, L.ptrs([V]), L.ptrs([A]), A.stride(0), L.ptrs([W]), ws=_ws(A),
              device=A.device, stream=L.stream_of(A))
    return W


@tri_vmm.register_fake
def _(V, A, sign):
    return V.new_empty(V.shape, dtype=torch.float32)


@custom_op("psgdk::norm_lower_bound", mutates_args=())
def norm_lower_bound(A: Tensor, V: Tensor, sign: int) -> Tensor:
    """Norm lower bound of the SPD (sign 1) / skew (sign -1) matrix in A's upper triangle with the random start V,
    on the device (psgd_pro.py:19-65; kernels/ops.py:124-136)."""
    _cuda(A, V)
    A = _as_2d(A, "A").float()
    V = V.float().contiguous()
    n = A.shape[0]
    if V.shape != (L.NLB_K, n):
        raise RuntimeError(f"V: expected shape ({L.NLB_K}, {n}), got {tuple(V.shape)}")
    out = torch.empty((), device=A.device, dtype=torch.float32)
    L.call_ws(L.lib().psgdk_norm_lower_bound, n, sign, 1, L.ptrs([A]), A.stride(0), L.ptrs([V]), L.ptrs([out]),
              ws=_ws(A), device=A.device, stream=L.stream_of(A))
    return out


@norm_lower_bound.register_fake
def _(A, V, sign):
    return A.new_empty((), dtype=torch.float32)


@custom_op("psgdk::unpack", mutates_args=())
def unpack(Pk: Tensor, n: int) -> Tensor:
    """Full symmetric n x n matrix from its packed upper triangle (kernels/ops.py:112-116)."""
    _cuda(Pk)
    Pk = Pk.float().contiguous()
    if Pk.numel() != n * (n + 1) // 2:
        raise RuntimeError(f"packed triangle of n = {n} needs {n * (n + 1) // 2} values, got {Pk.numel()}")
    C = torch.empty(n, n, device=Pk.device, dtype=torch.float32)
    L.check(L.lib().psgdk_unpack(n, 1, L.ptrs([Pk]), L.ptrs([C]), n, L.stream_of(Pk)))
    return C


@unpack.register_fake
def _(Pk, n):
    return Pk.new_empty(n, n, dtype=torch.float32)


def side(S):
    """Side n of a symmetric matrix held square (n x n) or as its packed upper triangle: T = n(n+1)/2 values give
    n = (sqrt(8T + 1) - 1) / 2 (kernels/ops.py:119-121)."""
    return S.shape[0] if S.dim() == 2 else int(((8 * S.shape[0] + 1) ** 0.5 - 1) / 2)


def pack_upper(A):
    """The packed storage form of square A: its upper triangle, diagonal included, read row by row (element (i, j),
    j >= i, lands at i n - i(i-1)/2 + j - i) (kernels/k1.py:40-43)."""
    iu = torch.triu_indices(A.shape[0], A.shape[0], device=A.device)
    return A[iu[0], iu[1]].contiguous()


# The reference's flag vocabulary (kernels/ops.py:1-13,139-215) and this package's own "bf16".
REFERENCE_FLAGS = frozenset({"k1", "k2", "k2t", "k2c", "k2b", "all", "tri", "nan", "packed"})
FLAGS = REFERENCE_FLAGS | {"bf16"}


def make_ops(flags=()):
    """The ops class for psgd_pro_fast-style callers (kernels/ops.py:142-215); every method runs on the HIP kernels.

    Every flag set the reference accepts is accepted, with its check that tri comes with k1 (AssertionError
    otherwise). The kernel-selection flags (k1: norm bounds, k2 / k2t / k2c / k2b: the SYRK variants, all: no
    size gates) choose among the reference's CUDA, Triton and cuBLAS kernels and the sizes from which each takes
    over from eager torch; here one HIP kernel set covers every method at every size, so they select nothing more.
    The storage flags keep their meaning: tri (term1 and P as upper triangles, read as triangles by symm / symm_r /
    the norm bounds), nan (with tri: the strict lower triangle returned as NaN), packed (term1 and P as packed upper
    triangles; takes precedence over tri for what sym returns). bf16: contractions take bfloat16 inputs (fp32
    accumulate). Flags outside this vocabulary raise ValueError."""
    flags = frozenset(flags)
    unknown = flags - FLAGS
    if unknown:
        raise ValueError(f"unknown flags {sorted(unknown)}; known: {sorted(FLAGS)}")
    assert "tri" not in flags or "k1" in flags, "tri needs k1 (term1's only other reader)"
    bf = "bf16" in flags
    tri = "tri" in flags
    packed = "packed" in flags

    def store(C):
        if "nan" in flags:
            C = C.masked_fill(torch.ones_like(C, dtype=torch.bool).tril(-1), float("nan"))
        return C

    def full(S):
        return unpack(S, side(S)) if S.dim() == 1 else S

    def syrk_full(X, trans):
        return syrk(X, trans, L.OUT_MIRROR, bf)

    def sym_store(X, trans):
        if packed:
            return syrk(X, trans, L.OUT_PACKED, bf)
        if tri:
            return store(syrk(X, trans, L.OUT_UPPER, bf))
        return syrk(X, trans, L.OUT_MIRROR, bf)

    def gram(Pg, i, expr):
        if Pg.dim() != 2:
            return expr(Pg, Pg)  # the caller's own contraction for non-matrix gradients (kernels/ops.py:201-204)
        if tri:
            return store(syrk(Pg, i == 1, L.OUT_UPPER, bf))
        return syrk_full(Pg, i == 1)

    def symm_l(S, X):
        if S.dim() == 1:
            S = full(S)
        return symm(S, X, 1, bf)

    def symm_r(X, S):
        if S.dim() == 1:
            S = full(S)
        return symm_right(X, S, 1, bf)

    def nlb_spd(A, V):
        return norm_lower_bound(full(A), V, 1)

    def nlb_skh(A, V):
        # R = Q^T - Q may arrive as a non-contiguous view; its upper triangle is read either way
        return norm_lower_bound(A.contiguous(), V, -1)

    class HipOps:
        pass

    HipOps.gram = staticmethod(gram)
    HipOps.gram_q = staticmethod(lambda q: syrk_full(q, True))
    HipOps.norm_lower_bound_spd = staticmethod(nlb_spd)
    HipOps.norm_lower_bound_skh = staticmethod(nlb_skh)
    HipOps.symm = staticmethod(symm_l)
    HipOps.symm_r = staticmethod(symm_r)
    HipOps.syrk = staticmethod(syrk_full)
    HipOps.sym = staticmethod(sym_store if (tri or packed) else syrk_full)
    HipOps.qsym = False
    HipOps.flags = flags
    HipOps._psgdk = True  # built here: KronWhiten(ops=...) accepts it
    return HipOps


# The no-flag plugin: the reference's default arithmetic class (psgd_pro_fast.py:106-126), on the HIP kernels.
HipOps = EagerOps = make_ops(())
