"""ctypes binding of libpsgdk.so (include/psgdk.h).

The library is loaded after torch, so that it binds to the HIP runtime torch already loaded (same soname) and works
on torch's streams and allocations. There is no fallback: when the library is missing, `lib()` raises.
"""
import collections
import ctypes as C
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("PSGDK_LIB", os.path.join(_HERE, "libpsgdk.so"))

MAXB = 16
MAX_GROUPS = 64
MAX_TENSORS = 64  # tensors per psgdk_momentum_multi call
NLB_K = 32
OK, EINVAL, ESHAPE, EHIP, EWORKSPACE = 0, 1, 2, 3, 4
F32, BF16 = 0, 1
PREC_F32, PREC_BF16 = 0, 1
OUT_UPPER, OUT_MIRROR, OUT_PACKED = 0, 1, 2
FACTOR_NONE, FACTOR_DIAG, FACTOR_DENSE = 0, 1, 2

_vp = C.c_void_p
_vpa = C.POINTER(C.c_void_p)  # host array of device pointers
_i64 = C.c_int64
_i32 = C.c_int
_f = C.c_float
_szp = C.POINTER(C.c_size_t)


class Kron2d(C.Structure):
    _fields_ = [("nb", C.c_int32), ("prec", C.c_int32), ("m", C.c_int64), ("n", C.c_int64),
                ("kind", C.c_int32 * 2), ("g_dtype", C.c_int32), ("p_dtype", C.c_int32),
                ("G", C.c_void_p * MAXB), ("Q", (C.c_void_p * MAXB) * 2), ("P", (C.c_void_p * MAXB) * 2),
                ("L", (C.c_void_p * MAXB) * 2), ("Qt16", (C.c_void_p * MAXB) * 2), ("P16", (C.c_void_p * MAXB) * 2)]


class UpdateOpts(C.Structure):
    _fields_ = [("lr", C.c_float), ("betaL", C.c_float), ("damping", C.c_float), ("grad_eps", C.c_float),
                ("tri", C.c_int32), ("r2", C.c_int32)]


class ApplyOpts(C.Structure):
    _fields_ = [("lr_params", C.c_float), ("max_avg_amp", C.c_float), ("max_element_amp", C.c_float),
                ("tri", C.c_int32)]


class Draws(C.Structure):
    """psgdk_draws_t: a group's noise generated inside the update (normals offset[b] .. of the
    psgdk_fill_normal(seed, stream_id) sequence)."""
    _fields_ = [("seed", C.c_uint64), ("stream_id", C.c_uint64), ("offset", C.c_int64 * MAXB)]


class ProfRecord(C.Structure):
    _fields_ = [("kernel_id", C.c_int32), ("tri", C.c_int32), ("nb", C.c_int32), ("ms", C.c_float),
                ("flops", C.c_double), ("bytes", C.c_double), ("m", C.c_int64), ("n", C.c_int64), ("k", C.c_int64),
                ("workgroups", C.c_int32), ("per_cu", C.c_int32)]


Launch = collections.namedtuple("Launch", [f for f, _ in ProfRecord._fields_])


_SIGS = {
    "psgdk_last_error": (C.c_char_p, []),
    "psgdk_version": (_i32, []),
    "psgdk_syrk": (_i32, [_i32, _i32, _i32, _i64, _i64, _i32, _i32, _vpa, _i64, _vpa, _i64, _vp]),
    "psgdk_symm": (_i32, [_i32, _i32, _i32, _i64, _i64, _i32, _i32, _vpa, _i64, _vpa, _i64, _vpa, _i64, _vp]),
    "psgdk_trmm": (_i32, [_i32, _i64, _i64, _i32, _i32, _vpa, _i64, _vpa, _i64, _vpa, _i64, _vp]),
    "psgdk_trmm_ws": (_i32, [_i32, _i64, _i64, _i32, _i32, _vpa, _i64, _vpa, _i64, _vpa, _i64, _vp, _szp, _vp]),
    "psgdk_gemm": (_i32, [_i32, _i32, _i32, _i64, _i64, _i64, _f, _i32, _i32, _i32, _vpa, _i64, _vpa, _i64, _f,
                          _vpa, _i64, _vp]),
    "psgdk_tri_rownorm2": (_i32, [_i64, _i32, _i32, _vpa, _i64, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_tri_vmm": (_i32, [_i64, _i32, _i32, _vpa, _vpa, _i64, _vpa, _vp, _szp, _vp]),
    "psgdk_norm_lower_bound": (_i32, [_i64, _i32, _i32, _vpa, _i64, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_mfma_rate": (_i32, [_i32, _i32, _vp, _vp]),
    "psgdk_read_rate": (_i32, [_vp, _i64, _i32, _i32, _i64, _vp, _vp]),
    "psgdk_clock_sample": (_i32, [_i32, _vp, _vp]),
    "psgdk_wall_mark": (_i32, [_vp, _vp]),
    "psgdk_wall_clock_rate": (_i32, [C.POINTER(C.c_int)]),
    "psgdk_fill_normal": (_i32, [_vp, _i64, _i32, C.c_uint64, C.c_uint64, _vp]),
    "psgdk_norm_lower_bound_full": (_i32, [_i64, _i32, _i32, _vpa, _i64, _i32, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_norm_lower_bound_full_noalloc": (_i32, [_i64, _i32, _i32, _vpa, _i64, _i32, _vpa, _vpa, _vp]),
    "psgdk_norm_lower_bound_gram": (_i32, [_i64, _i64, _i32, _vpa, _vpa, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_unpack": (_i32, [_i64, _i32, _vpa, _vpa, _i64, _vp]),
    "psgdk_kron2d_update": (_i32, [C.POINTER(Kron2d), C.POINTER(UpdateOpts), _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_kron2d_update_groups": (_i32, [_i32, C.POINTER(C.POINTER(Kron2d)), C.POINTER(C.POINTER(UpdateOpts)),
                                          C.POINTER(_vpa), C.POINTER(_vpa), _vp, _szp, _vp]),
    "psgdk_kron2d_update_groups_ev": (_i32, [_i32, C.POINTER(C.POINTER(Kron2d)), C.POINTER(C.POINTER(UpdateOpts)),
                                             C.POINTER(_vpa), C.POINTER(_vpa), _vp, _szp, _vp, _vpa]),
    "psgdk_kron2d_update_groups_drawn": (_i32, [_i32, C.POINTER(C.POINTER(Kron2d)),
                                                C.POINTER(C.POINTER(UpdateOpts)), C.POINTER(_vpa),
                                                C.POINTER(C.POINTER(Draws)), C.POINTER(_vpa), _vp, _szp, _vp, _vpa]),
    "psgdk_kron2d_apply": (_i32, [C.POINTER(Kron2d), C.POINTER(ApplyOpts), _vpa, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_apply2d": (_i32, [C.POINTER(Kron2d), C.POINTER(ApplyOpts), _vpa, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_factor_update": (_i32, [_i32, _i64, _i32, _vpa, _i32, _vpa, _vpa, _vpa, _vpa, C.c_float, C.c_float,
                                   C.c_float, _vp, _szp, _vp]),
    "psgdk_procrustes": (_i32, [_i32, _i64, _i32, _vpa, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_procrustes_r2": (_i32, [_i32, _i64, _i32, _vpa, _vpa, _vpa, _vp, _szp, _vp]),
    "psgdk_kron2d_refresh_p": (_i32, [C.POINTER(Kron2d), _i32, _i32, _vp]),
    "psgdk_kron2d_balance": (_i32, [C.POINTER(Kron2d), C.POINTER(C.c_int32), _i32, _vp, _szp, _vp]),
    "psgdk_momentum": (_i32, [_i64, _f, _i32, _i32, _vpa, _vpa, _vp]),
    "psgdk_momentum_multi": (_i32, [_i32, C.POINTER(C.c_int64), _f, C.POINTER(C.c_int32), _vpa, _vpa, _vp]),
    "psgdk_set_option": (_i32, [_i32, _i32]),
    "psgdk_get_option": (_i32, [_i32, C.POINTER(C.c_int)]),
    "psgdk_profile_start": (_i32, []),
    "psgdk_profile_stop": (_i32, [C.POINTER(ProfRecord), _i32, C.POINTER(C.c_int)]),
    "psgdk_debug_mfma": (_i32, [_i32, _vp, _vp, _vp, _vp]),
}

EXPORTED = tuple(_SIGS)
ABI_VERSION = 4  # PSGDK_VERSION of include/psgdk.h that these signatures and structures follow

_lib = None


def lib():
    """The loaded library with typed entry points; raises when it is missing (build it with
    `python -m psgd_pro_amd.build`)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"psgd_pro_amd: {LIB_PATH} not found; build it with `python -m psgd_pro_amd.build`")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in _SIGS.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        if L.psgdk_version() != ABI_VERSION:  # a stale build: its structures may not match these bindings
            raise RuntimeError(f"psgd_pro_amd: {LIB_PATH} has ABI version {L.psgdk_version()}, the bindings expect "
                               f"{ABI_VERSION}; rebuild it with `python -m psgd_pro_amd.build`")
        _lib = L
    return _lib


def check(rc):
    if rc != OK:
        msg = lib().psgdk_last_error().decode()
        raise RuntimeError(f"psgdk error {rc}: {msg}")


def ptrs(seq):
    """Host array of device addresses for a list of tensors (or ints / None)."""
    arr = (C.c_void_p * max(1, len(seq)))()
    for i, t in enumerate(seq):
        arr[i] = None if t is None else (t if isinstance(t, int) else t.data_ptr())
    return arr


def stream_of(t=None):
    """The raw handle of torch's current stream on t's device."""
    dev = t.device if t is not None else None
    return C.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def dtype_code(dt):
    if dt == torch.float32:
        return F32
    if dt == torch.bfloat16:
        return BF16
    raise TypeError(f"unsupported dtype {dt}: float32 or bfloat16")


class Workspace:
    """A device byte buffer reused across calls, grown on demand (torch's caching allocator owns it)."""

    def __init__(self):
        self.buf = None

    def get(self, nbytes, device):
        nbytes = max(int(nbytes), 256)
        if self.buf is None or self.buf.numel() < nbytes or self.buf.device != device:
            self.buf = torch.empty(nbytes, dtype=torch.uint8, device=device)
        return self.buf


def kernel_name(kernel_id):
    """Kernel template name of a profiling kernel id."""
    if kernel_id >= 7000:  # the small-problem kernels: 7000 / 7001 64-tiles, 7002 / 7003 tiny (bf16 / fp32)
        kind = "tiny" if kernel_id % 10 >= 2 else "small"
        return f"gemm_{kind}_kernel<{'float' if kernel_id % 2 else 'unsigned short'}>"
    if kernel_id >= 5000:  # 5000 (bf16) or 6000 (fp32 k-contiguous) + 10 cfg + epilogue
        base = 6000 if kernel_id >= 6000 else 5000
        cfg, epi = divmod(kernel_id - base, 10)
        tile = {0: "256, 256, 2, 4", 1: "128, 128, 2, 2", 2: "256, 256, 2, 2", 3: "256, 256, 2, 4",
                4: "128, 128, 2, 2"}[cfg]
        ws = ", 4" if cfg in (3, 4) else ""  # the warp-specialized kernels' 4 producer waves
        return f"gemm_{'f32kc' if base == 6000 else 'bf16'}_kernel<{tile}, {epi}{ws}>"
    cfg, rest = divmod(kernel_id, 1000)
    prec, rest = divmod(rest, 100)
    adt, bdt = divmod(rest, 10)
    t = {0: "float", 1: "unsigned short"}
    tile = "32, 128, 1, 4" if cfg else "128, 128, 2, 2"
    return f"gemm_kernel<{prec}, {t[adt]}, {t[bdt]}, {tile}>"


def profile_start():
    check(lib().psgdk_profile_start())


def profile_stop():
    """A Launch (kernel_id, tri, nb, ms, flops, bytes, m, n, k, workgroups, per_cu) per launch since
    profile_start()."""
    n = C.c_int(0)
    check(lib().psgdk_profile_stop(None, 0, C.byref(n)))
    arr = (ProfRecord * max(1, n.value))()
    check(lib().psgdk_profile_stop(arr, n.value, C.byref(n)))
    return [Launch(*(getattr(r, f) for f in Launch._fields)) for r in arr[:n.value]]


def call_ws(fn, *args, ws, device, stream):
    """Calls an entry point that takes (..., ws, ws_bytes, stream): queries the size, then runs."""
    sz = C.c_size_t(0)
    check(fn(*args, None, C.byref(sz), stream))
    buf = ws.get(sz.value, device)
    sz2 = C.c_size_t(buf.numel())
    check(fn(*args, C.c_void_p(buf.data_ptr()), C.byref(sz2), stream))
