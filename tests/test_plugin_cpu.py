"""The plugin boundary on the CPU: make_ops over the reference's whole flag vocabulary (kernels/ops.py:139-215), the
method set of the reference's EagerOps (psgd_pro_fast.py:106-126), and what KronWhiten(ops=...) takes from a plugin.
No device work: construction only."""
import itertools

import pytest
import torch

from psgd_pro_amd import EagerOps, KronWhiten, make_ops
from psgd_pro_amd import ops as hip_ops

# psgd_pro_fast.py:106-126: the reference's EagerOps attributes (gram / gram_q may be None there)
EAGER_METHODS = ("gram", "gram_q", "norm_lower_bound_spd", "norm_lower_bound_skh", "symm", "syrk", "sym", "symm_r")
REF_FLAGS = ("k1", "k2", "k2t", "k2c", "k2b", "all", "tri", "nan", "packed")


def test_reference_flag_vocabulary():
    assert hip_ops.REFERENCE_FLAGS == frozenset(REF_FLAGS)


@pytest.mark.parametrize("bf16", [False, True])
def test_every_reference_flag_set_builds(bf16):
    """All 512 subsets of the reference's flags: the reference's one check (tri needs k1, AssertionError) and
    otherwise a class with EagerOps's method set, every method callable, qsym False and flags as given."""
    n_ok = 0
    for r in range(len(REF_FLAGS) + 1):
        for combo in itertools.combinations(REF_FLAGS, r):
            flags = set(combo) | ({"bf16"} if bf16 else set())
            if "tri" in flags and "k1" not in flags:
                with pytest.raises(AssertionError, match="tri needs k1"):
                    make_ops(flags)
                continue
            ops = make_ops(flags)
            n_ok += 1
            for name in EAGER_METHODS:
                assert callable(getattr(ops, name)), (combo, name)
            assert ops.qsym is False and ops.flags == frozenset(flags)
            assert ops._psgdk
    assert n_ok == 512 - 128  # tri without k1: 2^7 subsets


def test_reference_call_forms():
    """The reference's own call forms: make_ops({"k1", "k2", "tri"}) and the default EagerOps."""
    ops = make_ops({"k1", "k2", "tri"})
    assert ops.flags == {"k1", "k2", "tri"}
    assert set(EAGER_METHODS) <= set(dir(EagerOps)) and EagerOps.flags == frozenset()


def test_storage_flags_reach_the_optimizer():
    """KronWhiten(ops=...) takes the storage form (tri / packed: upper triangles) and bf16 from the plugin; the
    kernel-selection flags change nothing; an explicit tri= or precision= wins."""
    W = torch.zeros(8, 8, requires_grad=True)
    assert KronWhiten([W])._tri == 0 and KronWhiten([W]).ops is EagerOps
    assert KronWhiten([W], ops=None).ops is EagerOps
    for flags, tri in (((), 0), (("k1",), 0), (("k2", "k2t", "all"), 0), (("k1", "tri"), 3), (("packed",), 3),
                       (("k1", "k2", "tri", "nan"), 3), (("k1", "tri", "packed"), 3)):
        opt = KronWhiten([W], ops=make_ops(flags))
        assert opt._tri == tri, flags
        assert opt._prec == 0
    assert KronWhiten([W], ops=make_ops({"bf16"}))._prec == 1
    assert KronWhiten([W], ops=make_ops({"bf16"}), precision="fp32")._prec == 0
    assert KronWhiten([W], ops=make_ops({"k1", "tri"}), tri=False)._tri == 0


def test_plugins_the_engine_cannot_use_raise():
    """A class make_ops did not build (the engine cannot call a foreign plugin's methods) raises TypeError; a plugin
    asking for the Q-symmetrization (psgd_pro_fast.py:231-233) raises NotImplementedError."""
    W = torch.zeros(8, 8, requires_grad=True)

    class Foreign:
        flags = frozenset()
        qsym = False

    with pytest.raises(TypeError, match="make_ops"):
        KronWhiten([W], ops=Foreign)
    qs = make_ops({"k1"})
    qs.qsym = True
    with pytest.raises(NotImplementedError, match="qsym"):
        KronWhiten([W], ops=qs)


def test_reference_execution_switches():
    """batch / cache_p / graph_rng / p2d are accepted, with the reference's own checks (psgd_pro_fast.py:286,290);
    graphs=True and compile raise."""
    W = torch.zeros(8, 8, requires_grad=True)
    for kw in (dict(batch=True), dict(cache_p=True), dict(graph_rng=True), dict(p2d=True), dict(r2=True)):
        KronWhiten([W], **kw)
    with pytest.raises(AssertionError, match="p2d"):
        KronWhiten([W], p2d=True, batch=True)
    with pytest.raises(AssertionError, match="cache_p"):
        KronWhiten([W], cache_p=True, compile="default")
    with pytest.raises(NotImplementedError, match="graphs=True"):
        KronWhiten([W], graphs=True)
