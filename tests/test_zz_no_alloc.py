"""psgdk_norm_lower_bound_full_noalloc (the entry point that allocates nothing: its scratch is the library's static
device array) against psgdk_norm_lower_bound_full with a caller workspace, on two calls in a row, the second with a
smaller input: the same kernels on the same inputs, so the bounds agree bit for bit."""
import ctypes as C

import pytest
import torch

from psgd_pro_amd import _lib as L

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(n, nb, dtype, sign, seed):
    g = torch.Generator().manual_seed(seed)
    A = []
    for _ in range(nb):
        X = torch.randn(n, n, generator=g)
        A.append(((X @ X.T) / n if sign > 0 else (X - X.T)).to(dtype).to(DEV))
    V = [torch.randn(32, n, generator=g).to(DEV) for _ in range(nb)]
    return A, V


@pytest.mark.parametrize("sign", [1, -1])
def test_noalloc_matches_workspace_entry_point(hip, sign):
    st = L.stream_of(torch.empty(1, device=DEV))
    for n, nb, dtype in ((1536, 3, torch.bfloat16), (640, 2, torch.float32)):
        A, V = _inputs(n, nb, dtype, sign, seed=n)
        dt = L.dtype_code(dtype)
        out_ref = [torch.full((1,), float("nan"), device=DEV) for _ in range(nb)]
        out_na = [torch.full((1,), float("nan"), device=DEV) for _ in range(nb)]
        print(f"noalloc norm bound: n {n}, nb {nb}, {dtype}, sign {sign}", flush=True)
        L.call_ws(hip.psgdk_norm_lower_bound_full, n, sign, nb, L.ptrs(A), n, dt, L.ptrs(V), L.ptrs(out_ref),
                  ws=L.Workspace(), device=A[0].device, stream=st)
        L.check(hip.psgdk_norm_lower_bound_full_noalloc(n, sign, nb, L.ptrs(A), n, dt, L.ptrs(V), L.ptrs(out_na),
                                                        st))
        torch.cuda.synchronize()
        for a, b in zip(out_ref, out_na):
            assert torch.isfinite(a).all() and float(a) > 0
            assert torch.equal(a, b), (float(a), float(b))
