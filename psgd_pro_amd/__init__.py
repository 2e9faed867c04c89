"""psgd_pro_amd: the PSGD-Kron preconditioner update + gradient apply on MI355X (gfx950) HIP kernels.

    from psgd_pro_amd import KronWhiten, make_ops

KronWhiten is a drop-in for the reference optimizer (psgd_pro.KronWhiten / psgd_pro_fast.KronWhiten); make_ops /
HipOps is the drop-in for its arithmetic plugin (kernels/ops.py make_ops). Both run on libpsgdk.so, built with
`python -m psgd_pro_amd.build`.
"""
from .kron import KronWhiten
from .ops import EagerOps, HipOps, make_ops

__all__ = ["KronWhiten", "EagerOps", "HipOps", "make_ops"]
