"""The C-ABI library without a GPU: it loads, exports every entry point include/psgdk.h declares, answers workspace
queries, and rejects bad arguments with an error code and message before touching the device."""
import ctypes as C
import os
import re

import pytest
import torch

from psgd_pro_amd import _lib as L

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "psgdk.h")


def declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(psgdk_[a-z0-9_]+)\s*\(", src)))


def test_header_and_binding_agree():
    assert declared() == sorted(L.EXPORTED)


def test_library_exports_every_declared_symbol():
    lib = L.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert lib.psgdk_version() == L.ABI_VERSION
    assert re.search(r"#define PSGDK_VERSION (\d+)", open(HEADER).read()).group(1) == str(L.ABI_VERSION)


def test_nm_exports():
    out = os.popen(f"nm -D --defined-only {L.LIB_PATH}").read()
    syms = set(re.findall(r"\bT (psgdk_\w+)", out))
    assert set(declared()) <= syms


def _err():
    return L.lib().psgdk_last_error().decode()


def test_argument_validation():
    lib = L.lib()
    one = L.ptrs([0x1000])
    null = L.ptrs([None])
    # nb out of range
    rc = lib.psgdk_syrk(0, 0, 1, 64, 64, 0, 0, one, 64, one, 64, None)
    assert rc == L.EINVAL and "nb" in _err()
    rc = lib.psgdk_syrk(0, 0, 1, 64, 64, 0, 17, one, 64, one, 64, None)
    assert rc == L.EINVAL
    # null device pointer
    rc = lib.psgdk_syrk(0, 0, 1, 64, 64, 0, 1, null, 64, one, 64, None)
    assert rc == L.EINVAL and "A[0]" in _err()
    # bad precision / dtype / out mode / shapes
    assert lib.psgdk_syrk(7, 0, 1, 64, 64, 0, 1, one, 64, one, 64, None) == L.EINVAL
    assert lib.psgdk_syrk(0, 0, 1, 64, 64, 5, 1, one, 64, one, 64, None) == L.EINVAL
    assert lib.psgdk_syrk(0, 0, 9, 64, 64, 0, 1, one, 64, one, 64, None) == L.EINVAL
    assert lib.psgdk_syrk(0, 0, 1, 0, 64, 0, 1, one, 64, one, 64, None) == L.ESHAPE
    assert lib.psgdk_syrk(0, 0, 1, 64, 64, 0, 1, one, 32, one, 64, None) == L.ESHAPE
    assert lib.psgdk_gemm(0, 0, 0, 8, 8, 8, 1.0, 0, 0, 1, one, 4, one, 8, 0.0, one, 8, None) == L.ESHAPE
    assert lib.psgdk_symm(0, 2, 1, 8, 8, 0, 1, one, 8, one, 8, one, 8, None) == L.EINVAL
    assert lib.psgdk_symm(0, 1, 0, 8, 8, 0, 1, one, 8, one, 8, one, 8, None) == L.EINVAL
    assert lib.psgdk_symm(0, 0, 3, 8, 8, 0, 1, one, 8, one, 8, one, 8, None) == L.EINVAL


DEFAULTS = {0: 2, 1: -1, 2: 1024, 3: 4, 4: -1, 5: 1, 6: 3, 7: 1, 8: 1, 9: 64, 10: 128, 11: 64, 12: 1}


def _get(opt):
    v = C.c_int(-99)
    assert L.lib().psgdk_get_option(opt, C.byref(v)) == 0
    return v.value


def test_option_ranges():
    """psgdk_set_option accepts each option's documented values and refuses the rest (host state only)."""
    lib = L.lib()
    try:
        for opt, good, bad in [(0, [0, 1, 2], [3, -1]), (1, [-1, 0, 1, 2, 3, 4], [5, -2]), (2, [1, 4096], [0, -5]),
                               (3, [2, 4, 8], [1, 16]), (4, [-1, 0, 1, 2, 3], [4, -2]), (5, [0, 1], [2]),
                               (6, [0, 3, 8], [9, -1]), (7, [0, 1], [2]), (8, [0, 1], [2]), (9, [1, 12, 64], [0, 65]),
                               (10, [0, 64, 1000], [-1]), (11, [0, 16, 1000], [-1]), (12, [0, 1], [2, -1])]:
            for v in bad:
                assert lib.psgdk_set_option(opt, v) == L.EINVAL, (opt, v)
            for v in good:
                assert lib.psgdk_set_option(opt, v) == 0, (opt, v)
                assert _get(opt) == v
    finally:
        for opt, v in DEFAULTS.items():
            assert lib.psgdk_set_option(opt, v) == 0
    assert lib.psgdk_set_option(99, 0) == L.EINVAL
    v = C.c_int(0)
    assert lib.psgdk_get_option(99, C.byref(v)) == L.EINVAL and lib.psgdk_get_option(0, None) == L.EINVAL


def test_options_and_errors_are_per_thread():
    """Two host threads set different options, query workspace sizes (which depend on option 2) and trigger argument
    errors at the same time: each sees its own options, sizes and error messages; a new thread starts from the
    defaults; the main thread's options are untouched."""
    import threading
    lib = L.lib()
    barrier = threading.Barrier(2)
    out = {}

    def worker(tag, target, nb):
        barrier.wait()
        assert lib.psgdk_set_option(2, target) == 0
        assert lib.psgdk_set_option(1, 1 if tag == "a" else 0) == 0
        sizes, errs = [], []
        for _ in range(200):
            sz = C.c_size_t(0)
            assert lib.psgdk_norm_lower_bound_full(3072, 1, nb, None, 3072, 1, None, None, None, C.byref(sz),
                                                   None) == 0
            sizes.append(sz.value)
            assert lib.psgdk_syrk(0, 0, 1, 64, 64, 0, 17 + nb, L.ptrs([0x1000]), 64, L.ptrs([0x1000]), 64,
                                  None) == L.EINVAL
            errs.append(lib.psgdk_last_error().decode())
            barrier.wait()
        out[tag] = (set(sizes), set(errs), _get(2), _get(1))

    ta = threading.Thread(target=worker, args=("a", 64, 2))
    tb = threading.Thread(target=worker, args=("b", 4096, 3))
    ta.start(); tb.start(); ta.join(); tb.join()
    (sa, ea, oa2, oa1), (sb, eb, ob2, ob1) = out["a"], out["b"]
    assert len(sa) == 1 and len(sb) == 1 and sa != sb
    assert ea == {"nb = 19: must be in 1..16"} and eb == {"nb = 20: must be in 1..16"}
    assert (oa2, oa1, ob2, ob1) == (64, 1, 4096, 0)
    assert all(_get(o) == v for o, v in DEFAULTS.items())
    fresh = {}
    t = threading.Thread(target=lambda: fresh.update({o: _get(o) for o in DEFAULTS}))
    t.start(); t.join()
    assert fresh == DEFAULTS


def test_noalloc_norm_bound_refuses_oversized_problems_without_device_work():
    """psgdk_norm_lower_bound_full_noalloc computes the workspace it needs before touching the device and refuses a
    problem whose workspace exceeds its static scratch (PSGDK_NOALLOC_SCRATCH_MIB MiB), with a message."""
    lib = L.lib()
    limit = 32 << 20
    sz = C.c_size_t(0)
    assert lib.psgdk_norm_lower_bound_full(3072, 1, 16, None, 3072, 1, None, None, None, C.byref(sz), None) == 0
    assert sz.value > limit
    fake = L.ptrs([0x1000] * 16)
    rc = lib.psgdk_norm_lower_bound_full_noalloc(3072, 1, 16, fake, 3072, 1, fake, fake, None)
    assert rc == L.ESHAPE and "static scratch" in _err()
    assert lib.psgdk_norm_lower_bound_full_noalloc(3072, 1, 0, fake, 3072, 1, fake, fake, None) == L.EINVAL


def test_factor_step_entry_points_reject_aliasing_without_device_work():
    """psgdk_factor_update / psgdk_procrustes write Q_out from Q in one pass, so Q_out may not alias Q: refused
    after the size query and before any launch (fake device addresses are never touched)."""
    lib = L.lib()
    sz = C.c_size_t(0)
    assert lib.psgdk_procrustes(0, 256, 2, None, None, None, None, C.byref(sz), None) == L.OK and sz.value > 0
    ws = C.c_void_p(0x100000)
    q, other = L.ptrs([0x2000, 0x3000]), L.ptrs([0x4000, 0x5000])
    big = C.c_size_t(sz.value)
    assert lib.psgdk_procrustes(0, 256, 2, q, q, other, ws, C.byref(big), None) == L.EINVAL
    assert "alias" in _err()
    assert lib.psgdk_factor_update(0, 256, 2, None, 0, None, None, None, None, 0.1, 0.9, 1.0, None, C.byref(sz),
                                   None) == L.OK
    big = C.c_size_t(sz.value)
    assert lib.psgdk_factor_update(0, 256, 2, other, 0, q, q, other, other, 0.1, 0.9, 1.0, ws, C.byref(big),
                                   None) == L.EINVAL
    assert "alias" in _err()
    assert lib.psgdk_procrustes(3, 256, 2, q, other, other, ws, C.byref(big), None) == L.EINVAL


def test_workspace_queries_need_no_device():
    lib = L.lib()
    sz = C.c_size_t(0)
    assert lib.psgdk_norm_lower_bound(768, 1, 12, None, 768, None, None, None, C.byref(sz), None) == L.OK
    n, nb = 768, 12
    T = (n + 63) // 64
    assert sz.value >= nb * (2 * 32 * n + T * T * 64) * 4
    small = sz.value
    assert lib.psgdk_norm_lower_bound(3072, 1, 12, None, 3072, None, None, None, C.byref(sz), None) == L.OK
    assert sz.value > small
    # too small a workspace is an error, not an overrun
    g = L.Kron2d()
    g.nb, g.prec, g.m, g.n = 1, 0, 64, 32
    g.kind[0], g.kind[1] = L.FACTOR_DENSE, L.FACTOR_DIAG
    for f in range(2):
        g.Q[f][0] = g.P[f][0] = g.L[f][0] = 0x1000
    g.G[0] = 0x1000
    o = L.UpdateOpts(0.1, 0.9, 1e-9, 1.19e-7, 0, 0)
    assert lib.psgdk_kron2d_update(g, o, L.ptrs([0x1000]), L.ptrs([0x1000]), None, C.byref(sz), None) == L.OK
    need = sz.value
    assert need > 3 * 64 * 32 * 4
    tiny = C.c_size_t(16)
    assert lib.psgdk_kron2d_update(g, o, L.ptrs([0x1000]), L.ptrs([0x1000]), C.c_void_p(0x1000), C.byref(tiny),
                                   None) == L.EWORKSPACE


def test_group_validation():
    lib = L.lib()
    sz = C.c_size_t(0)
    g = L.Kron2d()
    g.nb, g.prec, g.m, g.n = 1, 0, 4, 8
    g.kind[0], g.kind[1] = L.FACTOR_NONE, L.FACTOR_DENSE  # NONE needs size 1
    g.G[0] = 0x1000
    for f in range(2):
        g.Q[f][0] = g.P[f][0] = g.L[f][0] = 0x1000
    o = L.UpdateOpts(0.1, 0.9, 1e-9, 1.19e-7, 0, 0)
    assert lib.psgdk_kron2d_update(g, o, None, None, None, C.byref(sz), None) == L.ESHAPE
    g.kind[0] = 7
    assert lib.psgdk_kron2d_update(g, o, None, None, None, C.byref(sz), None) == L.EINVAL
    g.kind[0] = L.FACTOR_DENSE
    g.Q[0][0] = None
    assert lib.psgdk_kron2d_update(g, o, None, None, None, C.byref(sz), None) == L.EINVAL
    assert "Q" in _err()
    g.Q[0][0] = 0x1000
    o.r2 = 1  # procrustes_step_r2: a valid choice (workspace query)
    assert lib.psgdk_kron2d_update(g, o, None, None, None, C.byref(sz), None) == L.OK
    o.r2 = 2
    assert lib.psgdk_kron2d_update(g, o, None, None, None, C.byref(sz), None) == L.EINVAL
    assert "r2" in _err()


def test_update_groups_validation():
    """psgdk_kron2d_update_groups refuses a bad group count, options that differ in a shared field, and a group that
    is not on the bf16 path, with a message, before touching the device."""
    lib = L.lib()
    sz = C.c_size_t(0)

    def group(prec=L.PREC_BF16, shadows=True):
        g = L.Kron2d()
        g.nb, g.prec, g.m, g.n = 1, prec, 64, 128
        g.kind[0], g.kind[1] = L.FACTOR_DENSE, L.FACTOR_DENSE
        g.G[0] = 0x1000
        for f in range(2):
            g.Q[f][0] = g.P[f][0] = g.L[f][0] = 0x1000
            if shadows:
                g.Qt16[f][0] = g.P16[f][0] = 0x1000
        return g

    def call(gs, os):
        ga = (C.POINTER(L.Kron2d) * len(gs))(*[C.pointer(g) for g in gs])
        oa = (C.POINTER(L.UpdateOpts) * len(os))(*[C.pointer(o) for o in os])
        return lib.psgdk_kron2d_update_groups(len(gs), ga, oa, None, None, None, C.byref(sz), None)

    o = L.UpdateOpts(0.1, 0.9, 1e-9, 7.8e-3, 0, 0)
    assert call([group(), group()], [o, o]) == L.OK and sz.value > 0
    assert lib.psgdk_kron2d_update_groups(0, None, None, None, None, None, C.byref(sz), None) == L.EINVAL
    o2 = L.UpdateOpts(0.2, 0.9, 1e-9, 7.8e-3, 0, 0)
    assert call([group(), group()], [o, o2]) == L.EINVAL and "same" in _err()
    assert call([group(), group(shadows=False)], [o, o]) == L.EINVAL and "bf16" in _err()
    assert call([group(prec=L.PREC_F32)], [o]) == L.EINVAL

    # the drawn-noise form: the same size query without noise; with a workspace, a group needs noise pointers or
    # draws, and draw offsets must be multiples of 4 (refused before any device work)
    ga = (C.POINTER(L.Kron2d) * 2)(*[C.pointer(group()), C.pointer(group())])
    oa = (C.POINTER(L.UpdateOpts) * 2)(C.pointer(o), C.pointer(o))
    sz2 = C.c_size_t(0)
    assert lib.psgdk_kron2d_update_groups_drawn(2, ga, oa, None, None, None, None, C.byref(sz2), None, None) == L.OK
    assert sz2.value == sz.value
    V = (C.POINTER(C.c_void_p) * 2)(L.ptrs([0x1000]), L.ptrs([0x1000]))
    ws = C.c_void_p(0x100000)

    def drawn(offsets):
        ds = []
        for off in offsets:
            if off is None:
                ds.append(None)
                continue
            d = L.Draws(7, 1)
            d.offset[0] = off
            ds.append(C.pointer(d))
        da = (C.POINTER(L.Draws) * 2)(*ds)
        n = (C.POINTER(C.c_void_p) * 2)(None, None)
        return lib.psgdk_kron2d_update_groups_drawn(2, ga, oa, n, da, V, ws, C.byref(sz2), None, None)

    assert drawn([0, None]) == L.EINVAL and "neither" in _err()
    assert drawn([0, 6]) == L.EINVAL and "multiple of 4" in _err()
    assert drawn([-4, 8]) == L.EINVAL
    assert lib.psgdk_kron2d_update_groups_drawn(2, ga, oa, None, None, V, ws, C.byref(sz2), None, None) == L.EINVAL


def test_python_surface_on_cpu():
    """The optimizer and the ops refuse CPU tensors with a clear error (no silent CPU path)."""
    from psgd_pro_amd import KronWhiten, make_ops
    W = torch.zeros(8, 8, requires_grad=True)
    with pytest.raises(RuntimeError, match="GPU"):
        KronWhiten([W], preconditioner_init_scale=1.0)
    ops = make_ops(())
    with pytest.raises(RuntimeError, match="CUDA"):
        ops.syrk(torch.zeros(4, 4), False)
    with pytest.raises(ValueError):
        make_ops({"k3"})
    with pytest.raises(ValueError):
        KronWhiten([W], compile="default")


def test_measurement_entry_points_validate_without_device_work():
    """psgdk_read_rate / psgdk_clock_sample / psgdk_wall_mark refuse bad arguments before any launch."""
    lib = L.lib()
    sink = C.c_void_p(0x1000)
    assert lib.psgdk_read_rate(None, 4096, 1, 1, 1, sink, None) == L.EINVAL
    assert lib.psgdk_read_rate(C.c_void_p(0x1000), 4096, 1, 1, 1, None, None) == L.EINVAL
    for nbytes in (0, 2048, 4097, 3 << 20):
        assert lib.psgdk_read_rate(C.c_void_p(0x1000), nbytes, 1, 1, 1, sink, None) == L.EINVAL, nbytes
        assert "power of two" in _err()
    for wgs, iters, stride in ((0, 1, 1), (1, 0, 1), (1, 1, 0)):
        assert lib.psgdk_read_rate(C.c_void_p(0x1000), 4096, wgs, iters, stride, sink, None) == L.EINVAL
    assert lib.psgdk_clock_sample(0, C.c_void_p(0x1000), None) == L.EINVAL
    assert lib.psgdk_clock_sample((1 << 24) + 1, C.c_void_p(0x1000), None) == L.EINVAL
    assert lib.psgdk_clock_sample(4, None, None) == L.EINVAL
    assert lib.psgdk_wall_mark(None, None) == L.EINVAL
    assert lib.psgdk_wall_clock_rate(None) == L.EINVAL
